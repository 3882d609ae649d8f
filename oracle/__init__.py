"""CPU oracle for the attention hot path -- TEST INFRASTRUCTURE ONLY.

This package is a float64 (optionally float32) numpy restatement of the
reference algorithm (aabhimittal/TPU-Native-Pallas-FlashAttention,
``src/pallas_flash``). It is the checker the parity tests compare the HIP
kernels against, and the timed CPU baseline in ``bench.py``. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it; the shipped package (``tpu-native-pallas-flashattention_amd/pallas_flash``)
never does, and has no CPU fallback.

Every function cites the reference file:line it follows. How each one is
pinned (closed forms, known-answer tests, finite differences, brute force) is
listed per function in ``attention.py``'s header; tests live in
``tests/test_oracle.py``.
"""

from .attention import (  # noqa: F401
    NEG_INF,
    attention_ref,
    attention_bwd_ref,
    precompute_rope_ref,
    apply_rope_ref,
    apply_rope_vjp_ref,
    rope_attention_ref,
    rope_attention_bwd_ref,
    decode_ref,
    paged_ref,
    gather_pages_ref,
    cache_write_ref,
    paged_write_ref,
    decode_step_ref,
    brute_force_attention,
)

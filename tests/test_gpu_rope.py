"""GPU tier: fused-RoPE forward kernel vs the oracle and vs the unfused path.

Re-expresses the reference's test_fused_rope.py (fused == unfused for
MHA/GQA/MQA x causal :26-39, ragged :42-50, decode with separate tables at
pos 37 :53-70, bf16 :73-82).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import check_fwd, dev, host, max_abs, note
from oracle import precompute_rope_ref, rope_attention_ref
from pallas_flash import apply_rope, flash_attention, flash_attention_rope, precompute_rope

pytestmark = pytest.mark.gpu
THETA = 10000.0


def _inputs(n_heads, n_kv_heads, seq, dim=128, seed=0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((1, n_heads, seq, dim)), rng.standard_normal((1, n_kv_heads, seq, dim)),
            rng.standard_normal((1, n_kv_heads, seq, dim)))


@pytest.mark.parametrize("n_heads,n_kv_heads", [(2, 2), (4, 2), (4, 1)])
@pytest.mark.parametrize("causal", [False, True])
def test_fused_matches_oracle_and_unfused(n_heads, n_kv_heads, causal):
    seq = 256
    note(f"rope Hq={n_heads} Hkv={n_kv_heads} causal={causal}")
    q, k, v = _inputs(n_heads, n_kv_heads, seq)
    cos, sin = precompute_rope(seq, 128, THETA, device="cuda")
    tq, tk, tv = dev(q, "f32"), dev(k, "f32"), dev(v, "f32")
    fused = flash_attention_rope(tq, tk, tv, cos, sin, causal=causal, interpret=True)
    assert fused.shape == tq.shape
    ref = rope_attention_ref(q, k, v, host(cos), host(sin), causal=causal)
    check_fwd(host(fused), ref, "f32")
    unfused = flash_attention(apply_rope(tq, cos, sin), apply_rope(tk, cos, sin), tv, causal=causal)
    assert max_abs(host(fused), host(unfused)) < 2e-3


@pytest.mark.parametrize("seq", [130, 200])
def test_fused_ragged_lengths(seq):
    q, k, v = _inputs(2, 2, seq, seed=1)
    cos, sin = precompute_rope(seq, 128, THETA, device="cuda")
    note(f"rope ragged {seq}")
    fused = flash_attention_rope(dev(q, "f32"), dev(k, "f32"), dev(v, "f32"), cos, sin, causal=True)
    ref = rope_attention_ref(q, k, v, host(cos), host(sin), causal=True)
    check_fwd(host(fused), ref, "f32")


def test_fused_decode_shape_separate_tables():
    pos, cache_size = 37, 256
    rng = np.random.default_rng(2)
    q = rng.standard_normal((1, 2, 1, 128))
    k = rng.standard_normal((1, 2, cache_size, 128))
    v = rng.standard_normal((1, 2, cache_size, 128))
    cos, sin = precompute_rope(cache_size, 128, THETA, device="cuda")
    note("rope decode tables")
    fused = flash_attention_rope(dev(q, "f32"), dev(k, "f32"), dev(v, "f32"), cos[pos:pos + 1],
                                 sin[pos:pos + 1], cos, sin, causal=False, block_q=1, kv_len=pos + 1)
    ref = rope_attention_ref(q, k, v, host(cos[pos:pos + 1]), host(sin[pos:pos + 1]), host(cos),
                             host(sin), kv_len=pos + 1)
    check_fwd(host(fused), ref, "f32")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("causal", [False, True])
def test_fused_half(dt, causal):
    q, k, v = _inputs(4, 2, 192, seed=3)
    cos, sin = precompute_rope(192, 128, THETA, device="cuda")
    tq, tk, tv = dev(q, dt), dev(k, dt), dev(v, dt)
    note(f"rope {dt} causal={causal}")
    out = flash_attention_rope(tq, tk, tv, cos, sin, causal=causal)
    assert out.dtype == tq.dtype
    ref = rope_attention_ref(host(tq), host(tk), host(tv), host(cos), host(sin), causal=causal)
    check_fwd(host(out), ref, dt)


def test_bf16_tables_and_head_dim_64():
    q, k, v = _inputs(4, 2, 96, dim=64, seed=4)
    cos, sin = precompute_rope(96, 64, THETA, device="cuda")
    note("rope bf16 tables d64")
    out = flash_attention_rope(dev(q, "f32"), dev(k, "f32"), dev(v, "f32"), cos.bfloat16(),
                               sin.bfloat16(), causal=True)
    ref = rope_attention_ref(q, k, v, host(cos.bfloat16()), host(sin.bfloat16()), causal=True)
    check_fwd(host(out), ref, "f32")


def test_precompute_rope_matches_closed_form():
    cos, sin = precompute_rope(4096, 128, THETA, device="cuda")
    rc, rs = precompute_rope_ref(4096, 128, THETA)
    # float32 argument rounding grows with position (|pos * inv_freq| <= 4095)
    assert max_abs(host(cos), rc) < 5e-4 and max_abs(host(sin), rs) < 5e-4
    assert max_abs(host(cos[:64]), rc[:64]) < 1e-5


def test_rope_is_forward_only():
    q, k, v = _inputs(2, 2, 64, seed=5)
    cos, sin = precompute_rope(64, 128, THETA, device="cuda")
    tq = dev(q, "f32").requires_grad_(True)
    out = flash_attention_rope(tq, dev(k, "f32"), dev(v, "f32"), cos, sin)
    with pytest.raises(NotImplementedError):
        out.sum().backward()

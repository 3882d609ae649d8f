"""MI355X-native attention hot path with the reference ``pallas_flash`` API.

Drop-in for the attention functions of aabhimittal/TPU-Native-Pallas-
FlashAttention (src/pallas_flash/__init__.py:7-11, 33-60): the same names,
signatures and argument validation, operating on torch tensors that live on a
ROCm device. The arithmetic is hand-written HIP for gfx950 in
``libpallas_flash_amd.so`` (C ABI: include/pallas_flash_amd.h). The decode
loop's cache writes, ring-buffer slots and single-row RoPE are device
primitives here too (``write_kv_cache``, ``flash_attention_decode_step``,
``write_to_paged_cache``); the tiny-LLaMA model and its generation loops are
not part of this package -- they are consumers of these functions.
"""

from .flash_attention import flash_attention, flash_attention_decode, flash_attention_with_lse
from .fused_rope import flash_attention_rope
from .paged import paged_flash_attention, init_paged_cache, write_to_paged_cache
from .cache import flash_attention_decode_step, write_kv_cache, ring_kv_len
from .reference import reference_attention
from .rope import precompute_rope, apply_rope

__all__ = [
    "flash_attention",
    "flash_attention_decode",
    "flash_attention_with_lse",
    "flash_attention_rope",
    "paged_flash_attention",
    "init_paged_cache",
    "write_to_paged_cache",
    "flash_attention_decode_step",
    "write_kv_cache",
    "ring_kv_len",
    "reference_attention",
    "precompute_rope",
    "apply_rope",
]

__version__ = "0.1.0"

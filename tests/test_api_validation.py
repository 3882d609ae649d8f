"""CPU tier: the Python API raises the reference's ``ValueError``s before any
device work, and refuses to run anywhere but a ROCm device (no CPU fallback).

Mirrors the reference's rejection tests: test_flash_attention.py:57-61,
test_decode.py:52-56, test_fused_rope.py:85-99, test_paged.py:118-125, plus
the remaining conditions of flash_attention.py:527-545, fused_rope.py:154-181
and paged.py:129-149.
"""

from __future__ import annotations

import pytest
import torch

from pallas_flash import (
    flash_attention,
    flash_attention_decode,
    flash_attention_rope,
    paged_flash_attention,
)


def z(*shape, dtype=torch.float32):
    return torch.zeros(shape, dtype=dtype)


def test_gqa_requires_divisible_heads():
    with pytest.raises(ValueError):
        flash_attention(z(1, 6, 128, 128), z(1, 4, 128, 128), z(1, 4, 128, 128), interpret=True)


@pytest.mark.parametrize("q,k,v", [
    (z(6, 128, 128), z(1, 6, 128, 128), z(1, 6, 128, 128)),     # rank
    (z(1, 2, 8, 128), z(1, 2, 8, 128), z(1, 2, 9, 128)),         # k.shape != v.shape
    (z(2, 2, 8, 128), z(1, 2, 8, 128), z(1, 2, 8, 128)),         # batch mismatch
    (z(1, 2, 8, 128), z(1, 2, 8, 64), z(1, 2, 8, 64)),           # head_dim mismatch
    (z(1, 2, 8, 128), z(1, 0, 8, 128), z(1, 0, 8, 128)),         # zero kv heads
])
def test_flash_attention_shape_errors(q, k, v):
    with pytest.raises(ValueError):
        flash_attention(q, k, v)


@pytest.mark.parametrize("kv_len", [0, -1, 9])
def test_kv_len_range(kv_len):
    with pytest.raises(ValueError):
        flash_attention(z(1, 2, 8, 128), z(1, 2, 8, 128), z(1, 2, 8, 128), kv_len=kv_len)


def test_mixed_dtypes_reach_the_device_check():
    # Accepted (computed in float32 on the device, as the reference computes);
    # on CPU tensors the call stops at the no-fallback check.
    with pytest.raises(RuntimeError, match="ROCm device"):
        flash_attention(z(1, 2, 8, 128), z(1, 2, 8, 128, dtype=torch.bfloat16), z(1, 2, 8, 128))


def test_cpu_tensors_refused_no_fallback():
    with pytest.raises(RuntimeError, match="ROCm device"):
        flash_attention(z(1, 2, 8, 128), z(1, 2, 8, 128), z(1, 2, 8, 128))


def test_decode_rejects_multi_row_query():
    with pytest.raises(ValueError):
        flash_attention_decode(z(1, 2, 4, 128), z(1, 2, 128, 128), z(1, 2, 128, 128), 128,
                               interpret=True)


def test_decode_cache_len_range():
    with pytest.raises(ValueError):
        flash_attention_decode(z(1, 2, 1, 128), z(1, 2, 16, 128), z(1, 2, 16, 128), 17)


def test_rope_rejects_bad_table_shape():
    q = z(1, 2, 128, 128)
    cos = z(64, 128)
    with pytest.raises(ValueError):
        flash_attention_rope(q, q, q, cos, cos, interpret=True)


def test_rope_requires_k_tables_when_lengths_differ():
    q, k = z(1, 2, 1, 128), z(1, 2, 128, 128)
    cos = z(1, 128)
    with pytest.raises(ValueError):
        flash_attention_rope(q, k, k, cos, cos, block_q=1, interpret=True)


def test_rope_rejects_odd_head_dim_and_bad_heads():
    q = z(1, 2, 8, 7)
    with pytest.raises(ValueError):
        flash_attention_rope(q, q, q, z(8, 7), z(8, 7))
    q, k = z(1, 6, 8, 128), z(1, 4, 8, 128)
    with pytest.raises(ValueError):
        flash_attention_rope(q, k, k, z(8, 128), z(8, 128))


def test_paged_rejects_multi_row_query():
    kp = z(4, 2, 32, 128)
    with pytest.raises(ValueError):
        paged_flash_attention(z(1, 2, 4, 128), kp, kp, torch.zeros((1, 2), dtype=torch.int32),
                              torch.tensor([32], dtype=torch.int32), interpret=True)


@pytest.mark.parametrize("case", ["pages_shape", "head_dim", "heads", "table", "lens"])
def test_paged_validation(case):
    q, kp = z(2, 4, 1, 128), z(8, 2, 16, 128)
    vp = kp
    table = torch.zeros((2, 3), dtype=torch.int32)
    lens = torch.tensor([5, 6], dtype=torch.int32)
    if case == "pages_shape":
        vp = z(8, 2, 8, 128)
    elif case == "head_dim":
        q = z(2, 4, 1, 64)
    elif case == "heads":
        q = z(2, 3, 1, 128)
    elif case == "table":
        table = torch.zeros((3, 3), dtype=torch.int32)
    else:
        lens = torch.tensor([5], dtype=torch.int32)
    with pytest.raises(ValueError):
        paged_flash_attention(q, kp, vp, table, lens)


# ------------------------------------------------ decode-loop primitives --
from pallas_flash import flash_attention_decode_step, ring_kv_len, write_kv_cache  # noqa: E402


def test_ring_kv_len_matches_reference():
    # test_streaming.py:28-32
    assert ring_kv_len(3, 8) == 3
    assert ring_kv_len(8, 8) == 8
    assert ring_kv_len(50, 8) == 8
    assert ring_kv_len(1, 8) == 1


def test_decode_step_validation_before_device():
    z = lambda *s: torch.zeros(s)
    q, kn, vn, kc, vc = z(2, 8, 1, 128), z(2, 2, 1, 128), z(2, 2, 1, 128), z(2, 2, 64, 128), z(2, 2, 64, 128)
    with pytest.raises(ValueError):
        flash_attention_decode_step(z(2, 8, 2, 128), kn, vn, kc, vc, 0)        # two query rows
    with pytest.raises(ValueError):
        flash_attention_decode_step(q, z(2, 2, 2, 128), vn, kc, vc, 0)          # k_new rows
    with pytest.raises(ValueError):
        flash_attention_decode_step(z(2, 6, 1, 128), kn, vn, z(2, 4, 64, 128), z(2, 4, 64, 128), 0)
    with pytest.raises(ValueError):
        flash_attention_decode_step(q, kn, vn, kc, vc, 0, cos=z(64, 128))       # sin missing
    with pytest.raises(ValueError):
        flash_attention_decode_step(q, kn, vn, kc, vc, [0, 1, 2])               # 3 positions for batch 2
    with pytest.raises(ValueError):
        flash_attention_decode_step(q, kn, vn, kc, vc, torch.tensor([0.5, 1.0]))
    with pytest.raises(ValueError):                                             # model.py:329-331
        flash_attention_decode_step(q, kn, vn, kc, vc, 64)
    with pytest.raises(RuntimeError):                                           # valid, but no device path
        flash_attention_decode_step(q, kn, vn, kc, vc, 0)


def test_write_kv_cache_validation_before_device():
    z = lambda *s: torch.zeros(s)
    with pytest.raises(ValueError):
        write_kv_cache(z(2, 2, 8, 64), z(2, 2, 8, 64), z(2, 3, 1, 64), z(2, 3, 1, 64), 0)
    with pytest.raises(ValueError):
        write_kv_cache(z(2, 2, 8, 64), z(2, 2, 9, 64), z(2, 2, 1, 64), z(2, 2, 1, 64), 0)
    with pytest.raises(RuntimeError):
        write_kv_cache(z(2, 2, 8, 64), z(2, 2, 8, 64), z(2, 2, 1, 64), z(2, 2, 1, 64), 0)


def test_write_to_paged_cache_validation_before_device():
    from pallas_flash import write_to_paged_cache
    z = lambda *s: torch.zeros(s)
    with pytest.raises(ValueError):   # table rows != batch
        write_to_paged_cache(z(4, 2, 16, 64), z(4, 2, 16, 64), z(2, 2, 1, 64), z(2, 2, 1, 64),
                             torch.zeros(3, 4, dtype=torch.int32), 0)
    with pytest.raises(RuntimeError):
        write_to_paged_cache(z(4, 2, 16, 64), z(4, 2, 16, 64), z(1, 2, 1, 64), z(1, 2, 1, 64),
                             torch.zeros(4, dtype=torch.int32), 0)

"""GPU tier: split-KV decode kernel vs the oracle on the cache prefix.

Re-expresses the reference's test_decode.py kernel half (:26-56): n_kv_heads
x cache_len grid, the NaN-tail known-answer test, plus multi-chunk splits,
bf16, head_dim 64 and the exact tail-invariance property.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import check_fwd, dev, host, max_abs, note
from oracle import decode_ref
from pallas_flash import flash_attention, flash_attention_decode

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_kv_heads", [4, 2, 1])
@pytest.mark.parametrize("cache_len", [1, 5, 130, 256])
def test_decode_matches_reference(n_kv_heads, cache_len):
    note(f"decode n_kv={n_kv_heads} cache_len={cache_len}")
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 4, 1, 128))
    k = rng.standard_normal((1, n_kv_heads, 256, 128))
    v = rng.standard_normal((1, n_kv_heads, 256, 128))
    out = host(flash_attention_decode(dev(q, "f32"), dev(k, "f32"), dev(v, "f32"), cache_len,
                                      interpret=True))
    ref = decode_ref(q, k, v, cache_len)
    assert out.shape == (1, 4, 1, 128)
    check_fwd(out, ref, "f32")
    assert max_abs(out, ref) < 2e-3


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_decode_ignores_unwritten_slots(dt):
    """test_decode.py:38-49: ones + NaN tail -> exactly 1."""
    filled = 8
    k = np.concatenate([np.ones((1, 2, filled, 128)), np.full((1, 2, 120, 128), np.nan)], axis=2)
    q = np.ones((1, 2, 1, 128))
    note(f"decode nan KAT {dt}")
    out = host(flash_attention_decode(dev(q, dt), dev(k, dt), dev(k, dt), filled))
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out, 1.0, atol=1e-5)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("B,Hq,Hkv,cap,L,D", [
    (2, 8, 2, 4096, 3001, 128),     # several split-KV chunks + partial last block
    (3, 4, 4, 1000, 999, 128),      # MHA
    (2, 64, 1, 700, 613, 128),      # MQA, 64 heads -> two 32-head slices
    (2, 8, 2, 600, 577, 64),        # head_dim 64
])
def test_decode_splits(dt, B, Hq, Hkv, cap, L, D):
    note(f"decode split dt={dt} B={B} Hq={Hq} Hkv={Hkv} cap={cap} L={L} D={D}")
    rng = np.random.default_rng(2)
    q = rng.standard_normal((B, Hq, 1, D))
    k = rng.standard_normal((B, Hkv, cap, D))
    v = rng.standard_normal((B, Hkv, cap, D))
    k[:, :, L:] = np.nan
    v[:, :, L:] = np.nan
    tq, tk, tv = dev(q, dt), dev(k, dt), dev(v, dt)
    out = host(flash_attention_decode(tq, tk, tv, L))
    ref = decode_ref(host(tq), host(tk), host(tv), L)
    check_fwd(out, ref, dt)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, L:] = 1.0
    v2[:, :, L:] = 2.0
    out2 = host(flash_attention_decode(tq, dev(k2, dt), dev(v2, dt), L))
    np.testing.assert_array_equal(out, out2)


def test_decode_with_grad_routes_through_flash_attention():
    rng = np.random.default_rng(3)
    q = dev(rng.standard_normal((1, 4, 1, 128)), "f32").requires_grad_(True)
    k = dev(rng.standard_normal((1, 2, 64, 128)), "f32").requires_grad_(True)
    v = dev(rng.standard_normal((1, 2, 64, 128)), "f32").requires_grad_(True)
    note("decode grad path")
    out = flash_attention_decode(q, k, v, 40)
    out.sum().backward()
    ref = flash_attention(q.detach(), k.detach(), v.detach(), kv_len=40)
    assert torch.allclose(out, ref, atol=1e-6)
    assert (k.grad[:, :, 40:] == 0).all()


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_ring_layout_is_permutation_invariant(dt):
    """test_streaming.py:82-103: decode over a ring rotated by `shift` slots
    equals decode over the same keys in order, and both match the oracle."""
    note(f"decode ring permutation dt={dt}")
    rng = np.random.default_rng(9)
    capacity, dim = 8, 128
    q = rng.standard_normal((1, 2, 1, dim))
    k = rng.standard_normal((1, 2, capacity, dim))
    v = rng.standard_normal((1, 2, capacity, dim))
    in_order = host(flash_attention_decode(dev(q, dt), dev(k, dt), dev(v, dt), capacity, block_k=capacity))
    for shift in (1, 3, 7):
        rolled = host(flash_attention_decode(dev(q, dt), dev(np.roll(k, shift, axis=2), dt),
                                             dev(np.roll(v, shift, axis=2), dt), capacity))
        assert max_abs(in_order, rolled) < (2e-3 if dt == "f32" else 2e-2)
    check_fwd(in_order, decode_ref(host(dev(q, dt)), host(dev(k, dt)), host(dev(v, dt)), capacity), dt)

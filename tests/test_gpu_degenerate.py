"""GPU tier: degenerate shapes through the reference API -- an empty batch,
zero query rows, a single key, a single query row -- for the forward (and
its LSE), the backward, decode, paged decode, fused RoPE, the cache writes and
the decode step. Empty work returns correctly shaped outputs (zero gradients
for keys no query attends) without a launch; one-element cases are checked
against the oracle at the dtype's bar.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import DEV, check_fwd, check_grad, dev, host, note
from oracle import attention_bwd_ref, attention_ref, decode_ref, paged_ref, precompute_rope_ref, rope_attention_ref
from pallas_flash import (flash_attention, flash_attention_decode, flash_attention_decode_step,
                          flash_attention_rope, flash_attention_with_lse, paged_flash_attention,
                          write_kv_cache, write_to_paged_cache)

pytestmark = pytest.mark.gpu


def _z(*shape, dtype=torch.bfloat16):
    return torch.zeros(shape, dtype=dtype, device=DEV)


@pytest.mark.parametrize("shape", [(0, 4, 2, 16, 16), (2, 4, 2, 0, 16)])
def test_empty_forward_backward(shape):
    B, Hq, Hkv, Sq, Sk = shape
    note(f"degenerate: forward/backward B={B} Sq={Sq}")
    q = torch.randn((B, Hq, Sq, 128), device=DEV).to(torch.bfloat16).requires_grad_(True)
    k = torch.randn((B, Hkv, Sk, 128), device=DEV).to(torch.bfloat16).requires_grad_(True)
    v = torch.randn((B, Hkv, Sk, 128), device=DEV).to(torch.bfloat16).requires_grad_(True)
    out = flash_attention(q, k, v, causal=True)
    assert out.shape == q.shape and out.dtype == q.dtype
    out.backward(torch.ones_like(out))
    torch.cuda.synchronize()
    for t in (q, k, v):
        assert t.grad.shape == t.shape
        assert not t.grad.float().abs().any()  # nothing attends anything
    o2, lse = flash_attention_with_lse(q.detach(), k.detach(), v.detach())
    assert o2.shape == q.shape and lse.shape == (B, Hq, Sq) and lse.dtype == torch.float32


def test_single_key_and_single_query():
    note("degenerate: Sk=1 non-causal, Sq=1 causal")
    rng = np.random.default_rng(11)
    q, k, v, do = (rng.standard_normal(s) for s in ((2, 4, 5, 128), (2, 2, 1, 128), (2, 2, 1, 128), (2, 4, 5, 128)))
    tq, tk, tv = (dev(x, "f32").requires_grad_(True) for x in (q, k, v))
    out = flash_attention(tq, tk, tv)
    out.backward(dev(do, "f32"))
    torch.cuda.synchronize()
    ref, _ = attention_ref(q, k, v)
    check_fwd(host(out), ref, "f32")  # every row is v's one row
    # With one key P = 1 whatever the scores: dq = dk = 0 exactly (dS = dP -
    # delta cancels; only float32 rounding of the two terms is left), and dv
    # is the sum of the group's do rows.
    _, _, dv_want = attention_bwd_ref(q, k, v, do)
    check_grad(host(tv.grad), dv_want, "f32", "dv")
    for name, t in (("dq", tq), ("dk", tk)):
        assert np.abs(host(t.grad)).max() < 1e-3, name
    # one causal query row at position 0 sees key 0 only
    q1 = rng.standard_normal((1, 8, 1, 128))
    k1, v1 = rng.standard_normal((1, 2, 300, 128)), rng.standard_normal((1, 2, 300, 128))
    out1 = flash_attention(dev(q1, "bf16"), dev(k1, "bf16"), dev(v1, "bf16"), causal=True)
    torch.cuda.synchronize()
    ref1, _ = attention_ref(host(dev(q1, "bf16")), host(dev(k1, "bf16")), host(dev(v1, "bf16")), causal=True)
    check_fwd(host(out1), ref1, "bf16")


def test_empty_decode_and_paged():
    note("degenerate: decode / paged with batch 0")
    out = flash_attention_decode(_z(0, 8, 1, 128), _z(0, 2, 64, 128), _z(0, 2, 64, 128), 10)
    assert out.shape == (0, 8, 1, 128)
    pool = _z(4, 2, 16, 128)
    out = paged_flash_attention(_z(0, 8, 1, 128), pool, pool, torch.zeros((0, 3), dtype=torch.int32),
                                torch.zeros((0,), dtype=torch.int32))
    assert out.shape == (0, 8, 1, 128)
    torch.cuda.synchronize()


def test_single_slot_decode_and_single_page():
    note("degenerate: decode cache_len=1, paged one token")
    rng = np.random.default_rng(12)
    q, kc, vc = (rng.standard_normal(s) for s in ((3, 8, 1, 128), (3, 2, 32, 128), (3, 2, 32, 128)))
    tq, tk, tv = dev(q, "bf16"), dev(kc, "bf16"), dev(vc, "bf16")
    out = flash_attention_decode(tq, tk, tv, 1)
    torch.cuda.synchronize()
    check_fwd(host(out), decode_ref(host(tq), host(tk)[:, :, :1], host(tv)[:, :, :1], 1), "bf16")
    kp, vp = rng.standard_normal((5, 2, 16, 128)), rng.standard_normal((5, 2, 16, 128))
    table = np.array([[3, -1], [1, -1], [4, 0]], np.int32)
    lens = np.array([1, 0, 17], np.int32)
    tkp, tvp = dev(kp, "bf16"), dev(vp, "bf16")
    outp = paged_flash_attention(tq, tkp, tvp, torch.as_tensor(table), torch.as_tensor(lens))
    torch.cuda.synchronize()
    want = paged_ref(host(tq), host(tkp), host(tvp), table, lens)
    check_fwd(host(outp), want, "bf16")
    assert not host(outp)[1].any()  # the empty sequence gives zeros


def test_empty_rope_and_cache_writes():
    note("degenerate: rope Sq=0, cache writes of zero rows, decode step batch 0")
    cos, sin = (torch.as_tensor(x, dtype=torch.float32, device=DEV) for x in precompute_rope_ref(16, 128))
    q, k = _z(1, 4, 0, 128), _z(1, 2, 4, 128)
    out = flash_attention_rope(q, k, k, cos[:0], sin[:0], k_cos=cos[:4], k_sin=sin[:4])
    assert out.shape == q.shape
    kc, vc = _z(2, 2, 8, 128), _z(2, 2, 8, 128)
    write_kv_cache(kc, vc, _z(2, 2, 0, 128), _z(2, 2, 0, 128), 3)
    pool = _z(4, 2, 16, 128)
    write_to_paged_cache(pool, pool, _z(2, 2, 0, 128), _z(2, 2, 0, 128), torch.zeros((2, 2), dtype=torch.int32),
                         torch.zeros((2,), dtype=torch.int32))
    o = flash_attention_decode_step(_z(0, 8, 1, 128), _z(0, 2, 1, 128), _z(0, 2, 1, 128), _z(0, 2, 8, 128),
                                    _z(0, 2, 8, 128), torch.zeros((0,), dtype=torch.int32))
    assert o.shape == (0, 8, 1, 128)
    torch.cuda.synchronize()
    assert not kc.float().abs().any() and not pool.float().abs().any()


def test_rope_single_row():
    note("degenerate: fused rope Sq=Sk=1")
    rng = np.random.default_rng(13)
    q, k, v = (rng.standard_normal((1, 4, 1, 128)) for _ in range(3))
    cos, sin = precompute_rope_ref(1, 128)
    tq, tk, tv = dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16")
    out = flash_attention_rope(tq, tk, tv, torch.as_tensor(cos, dtype=torch.float32, device=DEV),
                               torch.as_tensor(sin, dtype=torch.float32, device=DEV), causal=True)
    torch.cuda.synchronize()
    check_fwd(host(out), rope_attention_ref(host(tq), host(tk), host(tv), cos, sin, causal=True), "bf16")

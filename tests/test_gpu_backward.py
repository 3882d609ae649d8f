"""GPU tier: backward kernels (delta, dQ, dK/dV with GQA group sum) vs the
float64 analytic oracle.

Re-expresses the reference's test_backward.py (CASES :45-52 x causal, block
sizes :68-76, bf16 dtype/finite :79-91, value-and-grad :94-105) with the
north-star tolerances (1e-5 relative for fp32, 5e-2 relative for bf16).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import check_grad, dev, host, note, rel_err
from oracle import attention_bwd_ref, attention_ref
from pallas_flash import flash_attention

pytestmark = pytest.mark.gpu

CASES = [
    (1, 2, 2, 128),
    (1, 2, 2, 256),
    (2, 4, 4, 256),
    (1, 4, 2, 256),   # GQA
    (1, 4, 1, 256),   # MQA
    (1, 2, 2, 200),   # ragged
]


def _grads(dt, B, Hq, Hkv, Sq, Sk, causal, seed=0, kv_len=None, D=128, sm_scale=None,
           nan_tail=False, **kw):
    note(f"bwd dt={dt} B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Sk={Sk} D={D} causal={causal} kv_len={kv_len}")
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Hq, Sq, D))
    k = rng.standard_normal((B, Hkv, Sk, D))
    v = rng.standard_normal((B, Hkv, Sk, D))
    do = rng.standard_normal((B, Hq, Sq, D))
    if nan_tail:
        k[:, :, kv_len:] = np.nan
        v[:, :, kv_len:] = np.nan
    tq, tk, tv = (dev(x, dt).requires_grad_(True) for x in (q, k, v))
    tdo = dev(do, dt)
    out = flash_attention(tq, tk, tv, causal=causal, kv_len=kv_len, sm_scale=sm_scale, **kw)
    out.backward(tdo)
    torch.cuda.synchronize()
    for t in (tq, tk, tv):
        assert t.grad.dtype == t.dtype and t.grad.shape == t.shape
    qh, kh, vh, doh = host(tq), host(tk), host(tv), host(tdo)
    if nan_tail:
        kh[:, :, kv_len:] = 0.0
        vh[:, :, kv_len:] = 0.0
    want = attention_bwd_ref(qh, kh, vh, doh, causal=causal, kv_len=kv_len, sm_scale=sm_scale)
    got = tuple(host(t.grad) for t in (tq, tk, tv))
    return got, want, host(out)


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("causal", [False, True])
def test_grads_match_reference_f32(case, causal):
    B, Hq, Hkv, S = case
    got, want, _ = _grads("f32", B, Hq, Hkv, S, S, causal)
    for name, g, w in zip("qkv", got, want):
        check_grad(g, w, "f32", "d" + name)
        assert rel_err(g, w) < 1e-4  # the reference's own bound


@pytest.mark.parametrize("block", [(64, 64), (128, 256), (256, 128)])
def test_grads_block_size_hints(block):
    got, want, _ = _grads("f32", 1, 2, 2, 256, 256, True, seed=3, block_q=block[0], block_k=block[1])
    for name, g, w in zip("qkv", got, want):
        check_grad(g, w, "f32", "d" + name)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("case", [(1, 2, 2, 128), (1, 4, 2, 256), (2, 4, 1, 200)])
@pytest.mark.parametrize("causal", [False, True])
def test_grads_half(dt, case, causal):
    B, Hq, Hkv, S = case
    got, want, _ = _grads(dt, B, Hq, Hkv, S, S, causal, seed=4)
    for name, g, w in zip("qkv", got, want):
        check_grad(g, w, dt, "d" + name)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
def test_grads_kv_len_nan_tail_and_unequal_lengths(dt, causal):
    got, want, _ = _grads(dt, 2, 4, 2, 150, 260, causal, seed=5, kv_len=190, nan_tail=True)
    for name, g, w in zip("qkv", got, want):
        check_grad(g, w, dt, "d" + name)
    # keys at or past kv_len get exactly zero gradient
    assert (got[1][:, :, 190:] == 0).all() and (got[2][:, :, 190:] == 0).all()


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_grads_head_dim_64_and_scale(dt):
    got, want, _ = _grads(dt, 1, 4, 2, 180, 180, True, seed=6, D=64, sm_scale=0.3)
    for name, g, w in zip("qkv", got, want):
        check_grad(g, w, dt, "d" + name)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("Sq,Sk", [(64, 300), (300, 64), (192, 192), (40, 200)])
def test_grads_sq_ne_sk_causal(dt, Sq, Sk):
    # top-left causal with Sq != Sk; 16-bit dK/dV steps cover 128 query rows
    # as two 64-row passes: Sq = 192 (a last step with one valid pass) and
    # Sq < 64 exercise the partially and fully invalid passes
    got, want, _ = _grads(dt, 1, 2, 1, Sq, Sk, True, seed=7)
    for name, g, w in zip("qkv", got, want):
        check_grad(g, w, dt, "d" + name)


def test_value_and_grad_loss():
    """test_backward.py:94-105: the loss value and its gradients."""
    rng = np.random.default_rng(5)
    q, k, v, cot = (rng.standard_normal((1, 2, 128, 128)) for _ in range(4))
    tq, tk, tv = (dev(x, "f32").requires_grad_(True) for x in (q, k, v))
    note("bwd value_and_grad")
    loss = (flash_attention(tq, tk, tv, causal=True) * dev(cot, "f32")).sum()
    loss.backward()
    ref, _ = attention_ref(q, k, v, causal=True)
    assert float(loss) == pytest.approx(float((ref * cot).sum()), rel=1e-4, abs=1e-4)
    assert all(torch.isfinite(t.grad).all() for t in (tq, tk, tv))


def test_bf16_grads_keep_dtype_and_finite():
    rng = np.random.default_rng(4)
    q, k, v = (rng.standard_normal((1, 2, 128, 128)) for _ in range(3))
    cot = dev(rng.standard_normal((1, 2, 128, 128)), "f32")
    tq, tk, tv = (dev(x, "bf16").requires_grad_(True) for x in (q, k, v))
    note("bwd bf16 dtype")
    (flash_attention(tq, tk, tv, causal=True).float() * cot).sum().backward()
    for t in (tq, tk, tv):
        assert t.grad.dtype == torch.bfloat16
        assert torch.isfinite(t.grad.float()).all()


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_delta_entry_point_and_dq_agree(dt):
    """delta = rowsum(o * do) (flash_attention.py:363-365) from the stored
    output: pf_attn_bwd_delta and the value pf_attn_bwd_dq writes (it computes
    delta for its own rows) both match the float64 rowsum; the three C-ABI
    launches delta -> dq -> dkv and the combined pf_attn_bwd (dq -> dkv) give
    the same gradients."""
    from pallas_flash import _lib, flash_attention_with_lse
    note(f"bwd delta entry points {dt}")
    rng = np.random.default_rng(31)
    B, Hq, Hkv, S, D = 2, 4, 2, 192, 128
    q, k, v, do = (dev(rng.standard_normal(s), dt) for s in
                   ((B, Hq, S, D), (B, Hkv, S, D), (B, Hkv, S, D), (B, Hq, S, D)))
    o, lse = flash_attention_with_lse(q, k, v, causal=True)
    want = (host(o) * host(do)).sum(-1)
    L = _lib.lib()
    st = torch.cuda.current_stream().cuda_stream

    def run(order):
        # NaN-filled: a launch that leaves a value unwritten shows as NaN, and
        # nothing here reads uninitialised memory (the delta-only run writes
        # no gradient, so only its delta is compared)
        delta = torch.full((B, Hq, S), float("nan"), dtype=torch.float32, device="cuda")
        dq, dk, dv = (torch.full_like(t, float("nan")) for t in (q, k, v))
        a = _lib.BwdArgs(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(), lse.data_ptr(),
                         delta.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, Hq, Hkv, S, S, D, S, 1,
                         D ** -0.5, _lib.dtype_tag(q))
        for name in order:
            assert getattr(L, name)(a, st) == _lib.PF_OK, name
        torch.cuda.synchronize()
        return host(delta), host(dq), host(dk), host(dv)

    d_only = run(["pf_attn_bwd_delta"])[0]
    d_dq = run(["pf_attn_bwd_dq"])[0]
    tol = 1e-5 * np.abs(want).max()
    assert np.abs(d_only - want).max() <= tol and np.abs(d_dq - want).max() <= tol
    split = run(["pf_attn_bwd_delta", "pf_attn_bwd_dq", "pf_attn_bwd_dkv"])
    fused = run(["pf_attn_bwd"])
    for name, x, y in zip(("dq", "dk", "dv"), split[1:], fused[1:]):
        assert np.isfinite(x).all() and np.isfinite(y).all(), name
        assert rel_err(x, y) <= (1e-5 if dt == "f32" else 2e-2), name

"""GPU tier: forward prefill kernel vs the float64 oracle.

Re-expresses the reference's test_flash_attention.py (shapes :24-30, GQA
:44-54, block sizes :64-70, custom scale :73-78) and test_bfloat16.py
(:18-47) against this build's oracle, with the north-star tolerances, plus
cases the reference leaves implicit (kv_len with a NaN tail, Sq != Sk, LSE,
head_dim 64, float16).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import DEV, check_fwd, dev, host, max_abs, note, qkv, rel_err
from oracle import attention_ref
from pallas_flash import flash_attention, flash_attention_with_lse

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1, 128), (1, 2, 256), (2, 3, 384), (1, 2, 200), (1, 2, 130)]


def _run(dt, B, Hq, Hkv, Sq, Sk, causal, seed=0, D=128, kv_len=None, sm_scale=None, **kw):
    note(f"fwd dt={dt} B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Sk={Sk} D={D} causal={causal} kv_len={kv_len}")
    rng = np.random.default_rng(seed)
    q, k, v = qkv(rng, B, Hq, Hkv, Sq, Sk, D)
    tq, tk, tv = dev(q, dt), dev(k, dt), dev(v, dt)
    out = flash_attention(tq, tk, tv, causal=causal, kv_len=kv_len, sm_scale=sm_scale, **kw)
    torch.cuda.synchronize()
    assert out.shape == tq.shape and out.dtype == tq.dtype
    ref, _ = attention_ref(host(tq), host(tk), host(tv), causal=causal, kv_len=kv_len,
                           sm_scale=sm_scale)
    return host(out), ref, (q, k, v)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_matches_reference_f32(shape, causal):
    B, H, S = shape
    out, ref, _ = _run("f32", B, H, H, S, S, causal)
    check_fwd(out, ref, "f32")
    assert max_abs(out, ref) < 2e-3  # the reference's own bound


def test_baseline_config1_fp32_mha():
    """BASELINE config 1, the reference's own fp32 parity case
    (tests/test_flash_attention.py:33-41): fp32, non-causal, MHA B=1 H=8
    S=512 D=128, q, k, v ~ N(0, 1) from np.random.default_rng(0) (in that
    order). o and LSE within 1e-5 relative of the float64 oracle, and o within
    the reference's own 2e-3 absolute bound."""
    B, H, S, D = 1, 8, 512, 128
    note("config 1: f32 MHA B=1 H=8 S=512 D=128 non-causal")
    rng = np.random.default_rng(0)
    q = rng.standard_normal((B, H, S, D))
    k = rng.standard_normal((B, H, S, D))
    v = rng.standard_normal((B, H, S, D))
    tq, tk, tv = dev(q, "f32"), dev(k, "f32"), dev(v, "f32")
    out = flash_attention(tq, tk, tv, causal=False)
    o2, lse = flash_attention_with_lse(tq, tk, tv, causal=False)
    torch.cuda.synchronize()
    ref, ref_lse = attention_ref(host(tq), host(tk), host(tv), causal=False)
    o_rel, lse_rel = rel_err(host(out), ref), rel_err(host(lse), ref_lse)
    note(f"config 1: o rel {o_rel:.3e} (abs {max_abs(host(out), ref):.3e}), lse rel {lse_rel:.3e}")
    assert o_rel <= 1e-5
    assert lse_rel <= 1e-5
    assert max_abs(host(out), ref) < 2e-3
    assert torch.equal(out, o2)


@pytest.mark.parametrize("n_heads,n_kv_heads", [(8, 2), (8, 1), (4, 4)])
@pytest.mark.parametrize("causal", [False, True])
def test_grouped_query_attention(n_heads, n_kv_heads, causal):
    out, ref, _ = _run("f32", 1, n_heads, n_kv_heads, 256, 256, causal, seed=7)
    check_fwd(out, ref, "f32")


@pytest.mark.parametrize("block", [(64, 64), (128, 256), (256, 128)])
def test_block_size_hints_accepted(block):
    out, ref, _ = _run("f32", 1, 2, 2, 512, 512, True, seed=1, block_q=block[0], block_k=block[1])
    check_fwd(out, ref, "f32")


def test_custom_scale():
    out, ref, _ = _run("f32", 1, 2, 2, 256, 256, False, seed=2, sm_scale=0.05)
    check_fwd(out, ref, "f32")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("n_heads,n_kv_heads", [(2, 2), (4, 2)])
@pytest.mark.parametrize("causal", [False, True])
def test_half_forward(dt, n_heads, n_kv_heads, causal):
    out, ref, (q, k, v) = _run(dt, 1, n_heads, n_kv_heads, 256, 256, causal)
    check_fwd(out, ref, dt)
    # test_bfloat16.py:29-38: against the f32 oracle on the *unrounded* inputs
    ref_unrounded, _ = attention_ref(q, k, v, causal=causal)
    assert max_abs(out, ref_unrounded) < 3e-2


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Sq,Sk", [(100, 300), (300, 100), (1, 200), (129, 129)])
def test_ragged_and_unequal_lengths(dt, causal, Sq, Sk):
    out, ref, _ = _run(dt, 2, 4, 2, Sq, Sk, causal, seed=3)
    check_fwd(out, ref, dt)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
def test_kv_len_with_nan_tail(dt, causal):
    rng = np.random.default_rng(4)
    q, k, v = qkv(rng, 1, 4, 2, 200, 320)
    kv_len = 157
    k[:, :, kv_len:] = np.nan
    v[:, :, kv_len:] = np.nan
    note(f"fwd nan-tail dt={dt} causal={causal}")
    tq, tk, tv = dev(q, dt), dev(k, dt), dev(v, dt)
    out = host(flash_attention(tq, tk, tv, causal=causal, kv_len=kv_len))
    ref, _ = attention_ref(host(tq), host(tk), host(tv), causal=causal, kv_len=kv_len)
    check_fwd(out, ref, dt)
    # bitwise: the tail's content cannot matter
    k2, v2 = k.copy(), v.copy()
    k2[:, :, kv_len:] = 7.0
    v2[:, :, kv_len:] = -3.0
    out2 = host(flash_attention(tq, dev(k2, dt), dev(v2, dt), causal=causal, kv_len=kv_len))
    np.testing.assert_array_equal(out, out2)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
def test_lse(dt, causal):
    rng = np.random.default_rng(5)
    q, k, v = qkv(rng, 2, 4, 1, 190, 190)
    tq, tk, tv = dev(q, dt), dev(k, dt), dev(v, dt)
    note(f"fwd lse dt={dt} causal={causal}")
    out, lse = flash_attention_with_lse(tq, tk, tv, causal=causal, kv_len=170)
    ro, rl = attention_ref(host(tq), host(tk), host(tv), causal=causal, kv_len=170)
    check_fwd(host(out), ro, dt)
    assert lse.dtype == torch.float32 and lse.shape == (2, 4, 190)
    assert max_abs(host(lse), rl) < (1e-5 if dt == "f32" else 1e-3)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
def test_head_dim_64(dt, causal):
    out, ref, _ = _run(dt, 1, 4, 2, 200, 200, causal, D=64, seed=6)
    check_fwd(out, ref, dt)


def test_closed_forms_on_device():
    # one valid key -> v0 exactly (up to rounding of 1.0 * v0)
    rng = np.random.default_rng(8)
    q, k, v = qkv(rng, 1, 2, 1, 64, 64)
    note("fwd closed forms")
    out = host(flash_attention(dev(q, "f32"), dev(k, "f32"), dev(v, "f32"), kv_len=1))
    np.testing.assert_allclose(out, np.broadcast_to(v[0, 0, 0], out.shape), rtol=1e-6)
    # causal row 0 -> v[0]
    out = host(flash_attention(dev(q, "f32"), dev(k, "f32"), dev(v, "f32"), causal=True))
    np.testing.assert_allclose(out[0, :, 0], np.broadcast_to(v[0, 0, 0], (2, 128)), rtol=1e-6)


def test_nondefault_stream_and_device_guard():
    rng = np.random.default_rng(9)
    q, k, v = qkv(rng, 1, 2, 2, 64, 64)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        tq, tk, tv = dev(q, "f32"), dev(k, "f32"), dev(v, "f32")
        out = flash_attention(tq, tk, tv, causal=True)
    s.synchronize()
    ref, _ = attention_ref(host(tq), host(tk), host(tv), causal=True)
    assert rel_err(host(out), ref) < 1e-5


@pytest.mark.parametrize("B,Hq,Hkv,S", [(2, 16, 8, 300), (4, 64, 8, 160), (1, 16, 16, 200), (3, 24, 8, 96)])
@pytest.mark.parametrize("causal", [False, True])
def test_pair_grouped_work_order(B, Hq, Hkv, S, causal):
    """(batch, kv head) pairs a multiple of 8 and more than 8: each XCD runs
    its pairs in L2-sized groups (fwd_work_item). Every row of o and LSE must
    still be produced exactly once and match the oracle (GQA group sizes 2,
    8, 1 and 3; ragged query blocks)."""
    note(f"pair-grouped order B={B} Hq={Hq} Hkv={Hkv} S={S} causal={causal}")
    rng = np.random.default_rng(B * 100 + Hq)
    q, k, v = qkv(rng, B, Hq, Hkv, S, S)
    tq, tk, tv = dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16")
    out, lse = flash_attention_with_lse(tq, tk, tv, causal=causal)
    torch.cuda.synchronize()
    ref, ref_lse = attention_ref(host(tq), host(tk), host(tv), causal=causal)
    check_fwd(host(out), ref, "bf16")
    assert max_abs(host(lse), ref_lse) <= 1e-3


@pytest.mark.parametrize("B,Hq,Hkv,S", [(4, 16, 8, 4096), (2, 16, 8, 8192)])
@pytest.mark.parametrize("pct", [0, 30])
def test_pair_grouped_multi_group_order(B, Hq, Hkv, S, pct):
    """Pairs whose K/V do not all fit an XCD's L2 at once: B=4 Hkv=8 S=4096
    (2 MiB per pair, two of an XCD's four pairs at a time) and B=2 Hkv=8
    S=8192 (4 MiB, one of two at a time), so fwd_work_item's later pair
    groups run; with the static order (tail_dynamic_pct 0) and with the
    default dynamic tail. Causal bf16; o and LSE of 96 sampled rows per head
    against the oracle, and no row left unwritten (outputs NaN-filled)."""
    from pallas_flash import _lib
    note(f"pair groups > 0: B={B} Hq={Hq} Hkv={Hkv} S={S} tail {pct}%")
    g = torch.Generator(device=DEV).manual_seed(S + B)
    tq, tk, tv = (torch.randn(s, generator=g, device=DEV).to(torch.bfloat16)
                  for s in ((B, Hq, S, 128), (B, Hkv, S, 128), (B, Hkv, S, 128)))
    o = torch.full_like(tq, float("nan"))
    lse = torch.full((B, Hq, S), float("nan"), device=DEV)
    a = _lib.FwdArgs(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), o.data_ptr(), lse.data_ptr(),
                     B, Hq, Hkv, S, S, 128, S, 1, 128 ** -0.5, _lib.dtype_tag(tq))
    with _lib.tuning(tail_dynamic_pct=pct):
        assert _lib.lib().pf_attn_fwd(a, torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(lse).all()
    rows = np.unique(np.concatenate([np.arange(0, S, S // 64), [1, 31, 32, 63, S - 33, S - 1],
                                     np.random.default_rng(S).integers(0, S, 26)]))
    ref, ref_lse = attention_ref(host(tq), host(tk), host(tv), causal=True, q_rows=rows)
    check_fwd(host(o)[:, :, rows], ref, "bf16")
    assert max_abs(host(lse)[:, :, rows], ref_lse) <= 1e-3

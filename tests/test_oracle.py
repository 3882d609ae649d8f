"""CPU tier: pin the float64 oracle (oracle/attention.py) without retyping it.

Each check is chosen so that a plausible mistake in the restatement (dropped
scale, wrong GQA head map, causal direction or alignment, transposed operand,
missing kv_len mask, wrong LSE base, wrong gradient term or group sum) fails
at least one of them: brute force with independent loops, closed forms,
library routines (scipy), finite differences and invariants.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
from scipy.special import logsumexp, softmax

from oracle import (
    apply_rope_ref,
    attention_bwd_ref,
    attention_ref,
    brute_force_attention,
    decode_ref,
    gather_pages_ref,
    paged_ref,
    precompute_rope_ref,
    rope_attention_ref,
)


def _qkv(rng, B, Hq, Hkv, Sq, Sk, D):
    q = rng.standard_normal((B, Hq, Sq, D))
    k = rng.standard_normal((B, Hkv, Sk, D))
    v = rng.standard_normal((B, Hkv, Sk, D))
    return q, k, v


# ----------------------------------------------------------------- forward --
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Sq,Sk,kv_len", [(5, 5, None), (3, 7, None), (6, 4, None), (5, 9, 6)])
def test_forward_matches_brute_force(rng, causal, Sq, Sk, kv_len):
    q, k, v = _qkv(rng, 2, 4, 2, Sq, Sk, 8)
    o, lse = attention_ref(q, k, v, causal=causal, kv_len=kv_len, sm_scale=0.37)
    ob, lb = brute_force_attention(q.tolist(), k.tolist(), v.tolist(), causal=causal,
                                   kv_len=kv_len, sm_scale=0.37)
    np.testing.assert_allclose(o, ob, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse, lb, rtol=1e-12, atol=1e-12)


def test_lse_is_scipy_logsumexp(rng):
    q, k, v = _qkv(rng, 1, 2, 2, 6, 9, 16)
    scale = 0.21
    _, lse = attention_ref(q, k, v, causal=True, sm_scale=scale, kv_len=7)
    for h in range(2):
        s = q[0, h] @ k[0, h].T * scale
        for i in range(6):
            valid = [j for j in range(7) if j <= i]
            assert lse[0, h, i] == pytest.approx(logsumexp(s[i, valid]), rel=1e-13)


def test_softmax_weights_are_scipy_softmax(rng):
    q, k, v = _qkv(rng, 1, 1, 1, 4, 6, 8)
    scale = 0.5
    o, _ = attention_ref(q, k, v, sm_scale=scale)
    w = softmax(q[0, 0] @ k[0, 0].T * scale, axis=-1)
    np.testing.assert_allclose(o[0, 0], w @ v[0, 0], rtol=1e-13)


def test_default_scale_is_inverse_sqrt_d(rng):
    q, k, v = _qkv(rng, 1, 1, 1, 3, 5, 16)
    o1, _ = attention_ref(q, k, v)
    o2, _ = attention_ref(q, k, v, sm_scale=1 / math.sqrt(16))
    np.testing.assert_array_equal(o1, o2)
    o3, _ = attention_ref(q, k, v, sm_scale=1.0)
    assert np.abs(o1 - o3).max() > 1e-3


def test_single_valid_key_returns_v0(rng):
    q, k, v = _qkv(rng, 1, 2, 1, 3, 10, 8)
    o, lse = attention_ref(q, k, v, kv_len=1)
    for h in range(2):
        np.testing.assert_allclose(o[0, h], np.broadcast_to(v[0, 0, 0], (3, 8)), rtol=1e-14)
        np.testing.assert_allclose(lse[0, h], q[0, h] @ k[0, 0, 0] / math.sqrt(8), rtol=1e-13)


def test_causal_row0_is_v0_and_last_row_sees_all(rng):
    q, k, v = _qkv(rng, 1, 1, 1, 6, 6, 8)
    o, _ = attention_ref(q, k, v, causal=True)
    onc, _ = attention_ref(q, k, v, causal=False)
    np.testing.assert_allclose(o[0, 0, 0], v[0, 0, 0], rtol=1e-14)
    np.testing.assert_allclose(o[0, 0, -1], onc[0, 0, -1], rtol=1e-13)


def test_causal_is_top_left_aligned_when_sq_ne_sk(rng):
    # Sq < Sk: row i sees keys 0..i only (not the bottom-right convention).
    q, k, v = _qkv(rng, 1, 1, 1, 2, 5, 8)
    o, _ = attention_ref(q, k, v, causal=True)
    np.testing.assert_allclose(o[0, 0, 0], v[0, 0, 0], rtol=1e-14)
    o2, _ = attention_ref(q[:, :, 1:2], k[:, :, :2], v[:, :, :2])
    np.testing.assert_allclose(o[0, 0, 1], o2[0, 0, 0], rtol=1e-13)


@pytest.mark.parametrize("which", ["q", "scale"])
def test_zero_scores_give_mean_of_valid_values(rng, which):
    q, k, v = _qkv(rng, 1, 1, 1, 4, 9, 8)
    if which == "q":
        q[:] = 0
        o, _ = attention_ref(q, k, v, kv_len=6)
    else:
        o, _ = attention_ref(q, k, v, kv_len=6, sm_scale=0.0)
    np.testing.assert_allclose(o[0, 0], np.broadcast_to(v[0, 0, :6].mean(0), (4, 8)), rtol=1e-13)


def test_all_ones_gives_one_and_nan_tail_is_ignored():
    # tests/test_decode.py:38-49 known-answer test
    k = np.concatenate([np.ones((1, 2, 8, 16)), np.full((1, 2, 24, 16), np.nan)], axis=2)
    q = np.ones((1, 2, 1, 16))
    o = decode_ref(q, k, k, 8)
    assert np.isfinite(o).all()
    np.testing.assert_allclose(o, 1.0, rtol=0, atol=1e-14)


def test_key_permutation_invariance(rng):
    q, k, v = _qkv(rng, 1, 2, 2, 5, 11, 8)
    perm = rng.permutation(11)
    o1, l1 = attention_ref(q, k, v)
    o2, l2 = attention_ref(q, k[:, :, perm], v[:, :, perm])
    np.testing.assert_allclose(o1, o2, rtol=1e-12)
    np.testing.assert_allclose(l1, l2, rtol=1e-12)


def test_gqa_equals_explicit_repeat(rng):
    q, k, v = _qkv(rng, 2, 6, 2, 5, 7, 8)
    o1, l1 = attention_ref(q, k, v, causal=True)
    kr, vr = np.repeat(k, 3, axis=1), np.repeat(v, 3, axis=1)  # h -> h // 3
    o2, l2 = attention_ref(q, kr, vr, causal=True)
    np.testing.assert_allclose(o1, o2, rtol=1e-14)
    np.testing.assert_allclose(l1, l2, rtol=1e-14)
    # a wrong (interleaved, h % Hkv) map would differ:
    kt, vt = np.tile(k, (1, 3, 1, 1)), np.tile(v, (1, 3, 1, 1))
    o3, _ = attention_ref(q, kt, vt, causal=True)
    assert np.abs(o1 - o3).max() > 1e-3


def test_q_rows_subset_matches_full(rng):
    q, k, v = _qkv(rng, 1, 2, 1, 9, 9, 8)
    o, l = attention_ref(q, k, v, causal=True)
    rows = [0, 4, 8]
    os_, ls = attention_ref(q, k, v, causal=True, q_rows=rows)
    np.testing.assert_array_equal(os_, o[:, :, rows])
    np.testing.assert_array_equal(ls, l[:, :, rows])


def test_float32_mode_close_to_float64(rng):
    q, k, v = _qkv(rng, 1, 2, 2, 16, 16, 32)
    o64, _ = attention_ref(q, k, v, causal=True)
    o32, _ = attention_ref(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32),
                           causal=True, dtype=np.float32)
    assert o32.dtype == np.float32
    np.testing.assert_allclose(o32, o64, atol=1e-5)


# ---------------------------------------------------------------- backward --
def _loss(q, k, v, do, **kw):
    o, _ = attention_ref(q, k, v, **kw)
    return float((o * do).sum())


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Hq,Hkv,Sq,Sk,kv_len", [(2, 2, 4, 4, None), (4, 2, 3, 5, 4), (3, 1, 5, 3, None)])
def test_backward_matches_finite_differences(rng, causal, Hq, Hkv, Sq, Sk, kv_len):
    q, k, v = _qkv(rng, 1, Hq, Hkv, Sq, Sk, 4)
    do = rng.standard_normal(q.shape)
    kw = dict(causal=causal, kv_len=kv_len, sm_scale=0.7)
    dq, dk, dv = attention_bwd_ref(q, k, v, do, **kw)
    eps = 1e-6
    for x, g in ((q, dq), (k, dk), (v, dv)):
        num = np.zeros_like(x)
        it = np.nditer(x, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            old = x[idx]
            x[idx] = old + eps
            fp = _loss(q, k, v, do, **kw)
            x[idx] = old - eps
            fm = _loss(q, k, v, do, **kw)
            x[idx] = old
            num[idx] = (fp - fm) / (2 * eps)
        np.testing.assert_allclose(g, num, rtol=1e-6, atol=1e-7)


def test_backward_identities(rng):
    q, k, v = _qkv(rng, 1, 2, 2, 6, 6, 8)
    do = rng.standard_normal(q.shape)
    scale = 1 / math.sqrt(8)
    dq, dk, dv = attention_bwd_ref(q, k, v, do, causal=True, kv_len=5)
    # keys >= kv_len: exactly zero gradient
    assert (dk[:, :, 5:] == 0).all() and (dv[:, :, 5:] == 0).all()
    # dV = P^T dO and sum_j dS_ij = 0 (softmax Jacobian annihilates constants)
    for h in range(2):
        s = q[0, h] @ k[0, h, :5].T * scale
        mask = np.tril(np.ones((6, 5), bool))
        s = np.where(mask, s, -np.inf)
        p = softmax(s, axis=-1)
        np.testing.assert_allclose(dv[0, h, :5], p.T @ do[0, h], rtol=1e-12)
        o = p @ v[0, h, :5]
        ds = p * (do[0, h] @ v[0, h, :5].T - (o * do[0, h]).sum(1, keepdims=True))
        np.testing.assert_allclose(ds.sum(1), 0, atol=1e-12)
        np.testing.assert_allclose(dq[0, h], ds @ k[0, h, :5] * scale, rtol=1e-10)


def test_backward_gqa_group_sum(rng):
    q, k, v = _qkv(rng, 1, 4, 2, 5, 5, 8)
    do = rng.standard_normal(q.shape)
    dq, dk, dv = attention_bwd_ref(q, k, v, do, causal=True)
    kr, vr = np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1)
    dq2, dk2, dv2 = attention_bwd_ref(q, kr, vr, do, causal=True)
    np.testing.assert_allclose(dq, dq2, rtol=1e-13)
    np.testing.assert_allclose(dk, dk2.reshape(1, 2, 2, 5, 8).sum(2), rtol=1e-12)
    np.testing.assert_allclose(dv, dv2.reshape(1, 2, 2, 5, 8).sum(2), rtol=1e-12)


def test_backward_delta_uses_given_output(rng):
    q, k, v = _qkv(rng, 1, 1, 1, 4, 4, 8)
    do = rng.standard_normal(q.shape)
    o, _ = attention_ref(q, k, v)
    a = attention_bwd_ref(q, k, v, do)
    b = attention_bwd_ref(q, k, v, do, o=o)
    for x, y in zip(a, b):
        np.testing.assert_allclose(x, y, rtol=1e-12)
    c = attention_bwd_ref(q, k, v, do, o=o + 0.1)
    assert np.abs(c[0] - a[0]).max() > 1e-4


# -------------------------------------------------------------------- RoPE --
def test_precompute_rope_closed_form():
    cos, sin = precompute_rope_ref(33, 16, 10000.0)
    for p in (0, 1, 17, 32):
        for i in range(8):
            ang = p * 10000.0 ** (-i / 8)
            assert cos[p, i] == pytest.approx(math.cos(ang), abs=1e-14)
            assert cos[p, i + 8] == pytest.approx(math.cos(ang), abs=1e-14)
            assert sin[p, i] == pytest.approx(math.sin(ang), abs=1e-14)
    np.testing.assert_array_equal(cos[0], 1.0)
    np.testing.assert_array_equal(sin[0], 0.0)


def test_apply_rope_identity_norm_and_relative_position(rng):
    cos, sin = precompute_rope_ref(64, 16, 10000.0)
    x = rng.standard_normal((1, 1, 64, 16))
    r = apply_rope_ref(x, cos, sin)
    np.testing.assert_allclose(r[0, 0, 0], x[0, 0, 0], rtol=1e-15)
    # each (i, i + D/2) pair is rotated: its norm is preserved
    n0 = x[..., :8] ** 2 + x[..., 8:] ** 2
    n1 = r[..., :8] ** 2 + r[..., 8:] ** 2
    np.testing.assert_allclose(n0, n1, rtol=1e-12)
    # <R_m q, R_n k> depends only on m - n
    qv, kv = rng.standard_normal(16), rng.standard_normal(16)
    xs = np.zeros((1, 1, 64, 16))
    def rot(vec, pos):
        xs[0, 0, pos] = vec
        return apply_rope_ref(xs, cos, sin)[0, 0, pos]
    a = rot(qv, 10) @ rot(kv, 3)
    b = rot(qv, 40) @ rot(kv, 33)
    assert a == pytest.approx(b, rel=1e-12)
    # rotate-half sign convention: position p, pair i rotates by +angle
    e = np.zeros(16); e[0] = 1.0
    y = rot(e, 5)
    assert y[0] == pytest.approx(math.cos(5.0), abs=1e-14)
    assert y[8] == pytest.approx(math.sin(5.0), abs=1e-14)


def test_rope_attention_is_attention_of_rotated(rng):
    q, k, v = _qkv(rng, 1, 2, 1, 6, 6, 8)
    cos, sin = precompute_rope_ref(6, 8)
    o = rope_attention_ref(q, k, v, cos, sin, causal=True)
    o2, _ = attention_ref(apply_rope_ref(q, cos, sin), apply_rope_ref(k, cos, sin), v, causal=True)
    np.testing.assert_array_equal(o, o2)
    # unrotated attention differs (the rotation is not a no-op)
    o3, _ = attention_ref(q, k, v, causal=True)
    assert np.abs(o - o3).max() > 1e-3


# ------------------------------------------------------------------- paged --
def _paged_inputs(rng, B, Hq, Hkv, page, pps, num_pages, D=8):
    q = rng.standard_normal((B, Hq, 1, D))
    kp = rng.standard_normal((num_pages, Hkv, page, D))
    vp = rng.standard_normal((num_pages, Hkv, page, D))
    table = np.stack([rng.choice(num_pages, size=pps, replace=False) for _ in range(B)]).astype(np.int32)
    return q, kp, vp, table


def test_paged_equals_contiguous_gather(rng):
    q, kp, vp, table = _paged_inputs(rng, 3, 4, 2, 4, 5, 16)
    lens = np.array([1, 7, 20], np.int32)
    o = paged_ref(q, kp, vp, table, lens)
    for b in range(3):
        kc = np.concatenate([kp[table[b, p]] for p in range(5)], axis=1)[:, :lens[b]]
        vc = np.concatenate([vp[table[b, p]] for p in range(5)], axis=1)[:, :lens[b]]
        ob, _ = attention_ref(q[b:b + 1], kc[None], vc[None])
        np.testing.assert_allclose(o[b], ob[0], rtol=1e-13)


def test_paged_padding_nan_and_zero_len(rng):
    q, kp, vp, table = _paged_inputs(rng, 2, 2, 2, 4, 4, 8)
    lens = np.array([6, 0], np.int32)
    o1 = paged_ref(q, kp, vp, table, lens)
    table2 = table.copy()
    table2[0, 2:] = -1                       # pages past ceil(6/4) = 2 are padding
    kp2, vp2 = kp.copy(), vp.copy()
    kp2[table[0, 1], :, 2:] = np.nan         # beyond-len tail of the last live page
    vp2[table[0, 1], :, 2:] = np.nan
    unused = sorted(set(range(8)) - set(table[0, :2].tolist()))
    kp2[unused] = np.nan
    vp2[unused] = np.nan
    o2 = paged_ref(q, kp2, vp2, table2, lens)
    np.testing.assert_array_equal(o1, o2)
    np.testing.assert_array_equal(o2[1], 0.0)


def test_paged_shared_pages_and_permutation(rng):
    q, kp, vp, table = _paged_inputs(rng, 1, 2, 2, 4, 3, 6)
    q2 = np.concatenate([q, q])
    t2 = np.concatenate([table, table])
    o = paged_ref(q2, kp, vp, t2, np.array([10, 10]))
    np.testing.assert_array_equal(o[0], o[1])
    # identity table over a re-laid-out pool gives the same result
    kid = kp[table[0]]
    vid = vp[table[0]]
    o3 = paged_ref(q, kid, vid, np.arange(3, dtype=np.int32)[None], np.array([10]))
    np.testing.assert_allclose(o3[0], o[0], rtol=1e-13)


def test_gather_never_reads_past_live_pages():
    pages = np.arange(4 * 1 * 2 * 1, dtype=float).reshape(4, 1, 2, 1)
    g = gather_pages_ref(pages, np.array([2, -1, -1]), 2)
    np.testing.assert_array_equal(g[0, :, 0], [4.0, 5.0])


# ------------------------------------------- decode-loop cache primitives --
from oracle import cache_write_ref, decode_step_ref, paged_write_ref  # noqa: E402


def test_cache_write_linear_is_slice_assignment(rng):
    cache = rng.standard_normal((2, 3, 10, 4))
    rows = rng.standard_normal((2, 3, 4, 4))
    got = cache_write_ref(cache, rows, [2, 8])
    want = cache.copy()
    want[0, :, 2:6] = rows[0]          # fits
    want[1, :, 8:10] = rows[1, :, :2]  # rows past the capacity are dropped
    assert np.array_equal(got, want)


def test_cache_write_ring_batch_equals_one_at_a_time(rng):
    C, S = 6, 15
    cache = rng.standard_normal((1, 2, C, 3))
    rows = rng.standard_normal((1, 2, S, 3))
    at_once = cache_write_ref(cache, rows, 0, ring=True)
    seq = cache.copy()
    for i in range(S):
        seq = cache_write_ref(seq, rows[:, :, i:i + 1], i, ring=True)
    assert np.array_equal(at_once, seq)
    # the ring holds the last C tokens, token p at slot p % C (np.roll of the window)
    window = rows[0, :, S - C:]
    assert np.array_equal(at_once[0], np.roll(window, (S - C) % C, axis=1))


def test_paged_write_then_gather_round_trip(rng):
    num_pages, page = 9, 4
    pool = np.full((num_pages, 2, page, 3), np.nan)
    table = np.array([[5, 1, 7, -1], [2, 0, -1, -1]])
    lens = [11, 6]
    rows = rng.standard_normal((2, 2, 11, 3))
    out = pool
    for b in range(2):
        out = paged_write_ref(out, rows[b:b + 1, :, :lens[b]], table[b:b + 1], 0)
    for b in range(2):
        assert np.array_equal(gather_pages_ref(out, table[b], lens[b]), rows[b, :, :lens[b]])
    # pages no live token maps to stay untouched (NaN); -1 entries are never written
    untouched = [p for p in range(num_pages) if p not in (5, 1, 7, 2, 0)]
    assert np.isnan(out[untouched]).all()
    # a write past the table or through -1 padding is dropped
    again = paged_write_ref(out, rows[1:2, :, :1], table[1:2], 9)  # logical page 2 -> -1
    assert np.array_equal(np.nan_to_num(again, nan=7.0), np.nan_to_num(out, nan=7.0))


def _decode_problem(rng, B, Hq, Hkv, C, D):
    q = rng.standard_normal((B, Hq, 1, D))
    kn = rng.standard_normal((B, Hkv, 1, D))
    vn = rng.standard_normal((B, Hkv, 1, D))
    kc = rng.standard_normal((B, Hkv, C, D))
    vc = rng.standard_normal((B, Hkv, C, D))
    return q, kn, vn, kc, vc


def test_decode_step_equals_decode_on_built_cache(rng):
    B, Hq, Hkv, C, D = 2, 4, 2, 12, 8
    q, kn, vn, kc, vc = _decode_problem(rng, B, Hq, Hkv, C, D)
    pos = [5, 11]
    o, kc2, vc2 = decode_step_ref(q, kn, vn, kc, vc, pos)
    for b in range(B):
        kb, vb = kc.copy(), vc.copy()
        kb[b, :, pos[b]] = kn[b, :, 0]
        vb[b, :, pos[b]] = vn[b, :, 0]
        assert np.array_equal(kc2[b], kb[b]) and np.array_equal(vc2[b], vb[b])
        ref = decode_ref(q[b:b + 1], kb[b:b + 1], vb[b:b + 1], pos[b] + 1)
        np.testing.assert_allclose(o[b], ref[0], rtol=0, atol=1e-12)
    # invalid positions: nothing written, o = 0
    o_bad, kc3, _ = decode_step_ref(q, kn, vn, kc, vc, [-1, C])
    assert not o_bad.any() and np.array_equal(kc3, kc)


def test_decode_step_ring_equals_window_in_order(rng):
    """test_streaming.py:82-103: a wrapped ring gives attention over the window."""
    B, Hq, Hkv, C, D, T = 1, 2, 2, 8, 8, 21
    toks_k = rng.standard_normal((B, Hkv, T, D))
    toks_v = rng.standard_normal((B, Hkv, T, D))
    q = rng.standard_normal((B, Hq, 1, D))
    kc = np.zeros((B, Hkv, C, D))
    vc = np.zeros((B, Hkv, C, D))
    for p in range(T - 1):
        kc = cache_write_ref(kc, toks_k[:, :, p:p + 1], p, ring=True)
        vc = cache_write_ref(vc, toks_v[:, :, p:p + 1], p, ring=True)
    o, _, _ = decode_step_ref(q, toks_k[:, :, T - 1:], toks_v[:, :, T - 1:], kc, vc, T - 1, ring=True)
    window_o, _ = attention_ref(q, toks_k[:, :, T - C:], toks_v[:, :, T - C:])
    np.testing.assert_allclose(o, window_o, rtol=0, atol=1e-12)


def test_decode_step_rope_relative_position_invariance(rng):
    """Shifting every position by a constant leaves o unchanged once the ring
    has wrapped (every slot live; scores <R_m q, R_n k> depend on m - n and
    attention ignores slot order); position 0 is the unrotated problem."""
    B, Hq, Hkv, C, D, T = 1, 2, 1, 16, 8, 20
    cos, sin = precompute_rope_ref(64, D)
    ks = rng.standard_normal((B, Hkv, T, D))
    vs = rng.standard_normal((B, Hkv, T, D))
    q = rng.standard_normal((B, Hq, 1, D))

    def run(shift):
        kc = np.zeros((B, Hkv, C, D))
        vc = np.zeros((B, Hkv, C, D))
        o = None
        for t in range(T):
            o, kc, vc = decode_step_ref(q, ks[:, :, t:t + 1], vs[:, :, t:t + 1], kc, vc, t + shift,
                                        cos, sin, ring=True)
        return o

    np.testing.assert_allclose(run(0), run(7), rtol=0, atol=1e-10)
    # position 0, single token: rotation is the identity (cos = 1, sin = 0)
    q0, kn, vn, kc, vc = _decode_problem(rng, 1, 2, 1, 4, D)
    o_rot, kc_rot, _ = decode_step_ref(q0, kn, vn, kc, vc, 0, cos, sin)
    o_plain, kc_plain, _ = decode_step_ref(q0, kn, vn, kc, vc, 0)
    np.testing.assert_allclose(o_rot, o_plain, rtol=0, atol=1e-12)
    np.testing.assert_allclose(kc_rot, kc_plain, rtol=0, atol=1e-12)


# ----------------------------------------------------- RoPE-aware backward --
from oracle import rope_attention_bwd_ref  # noqa: E402


def _random_tables(rng, S, D):
    """cos/sin tables of any values, the two halves of every row different
    (flash_attention_rope accepts any [S, D] table, fused_rope.py:170-173)."""
    c, s = rng.standard_normal((S, D)), rng.standard_normal((S, D))
    assert np.abs(s[:, :D // 2] - s[:, D // 2:]).min() > 0
    return c, s


def test_rope_vjp_is_the_transpose_of_the_rotation(rng):
    """apply_rope_vjp_ref == J^T g, with J built column by column from unit
    vectors through apply_rope_ref, and the adjoint (dot-product) identity,
    for random tables whose halves differ."""
    from oracle import apply_rope_vjp_ref
    S, D = 5, 8
    cos, sin = _random_tables(rng, S, D)
    for p in range(S):
        J = np.stack([apply_rope_ref(np.eye(D)[j][None, None, None], cos[p:p + 1], sin[p:p + 1])[0, 0, 0]
                      for j in range(D)], axis=1)  # J[:, j] = rotation of e_j
        g = rng.standard_normal(D)
        got = apply_rope_vjp_ref(g[None, None, None], cos[p:p + 1], sin[p:p + 1])[0, 0, 0]
        np.testing.assert_allclose(got, J.T @ g, rtol=1e-13, atol=1e-13)
    x, g = rng.standard_normal((2, 3, S, D)), rng.standard_normal((2, 3, S, D))
    lhs = float((apply_rope_ref(x, cos, sin) * g).sum())
    rhs = float((x * apply_rope_vjp_ref(g, cos, sin)).sum())
    assert lhs == pytest.approx(rhs, rel=1e-12)
    # with these tables the transpose is NOT the rotation with -sin (which is
    # only right when sin[:, :D/2] == sin[:, D/2:], as in precompute_rope's)
    wrong = apply_rope_ref(g, cos, -sin)
    assert np.abs(wrong - apply_rope_vjp_ref(g, cos, sin)).max() > 1e-2
    # precompute_rope tables: the two agree
    pc, ps = precompute_rope_ref(S, D, 100.0)
    np.testing.assert_allclose(apply_rope_ref(g, pc, -ps), apply_rope_vjp_ref(g, pc, ps), rtol=1e-13,
                               atol=1e-13)


@pytest.mark.parametrize("causal,Hq,Hkv,Sq,Sk,kv_len,tables", [
    (True, 2, 1, 5, 5, None, "precompute"), (False, 4, 2, 3, 6, 5, "precompute"),
    (True, 2, 1, 5, 5, None, "random"), (False, 4, 2, 3, 6, 5, "random")])
def test_rope_backward_matches_finite_differences(rng, causal, Hq, Hkv, Sq, Sk, kv_len, tables):
    D = 6
    q, k, v = _qkv(rng, 1, Hq, Hkv, Sq, Sk, D)
    do = rng.standard_normal(q.shape)
    if tables == "precompute":
        qc, qs = precompute_rope_ref(Sq + 3, D, 50.0)
        kc, ks = precompute_rope_ref(Sk + 3, D, 50.0)
        qc, qs = qc[3:], qs[3:]          # query positions 3.. (decode-like offset)
        kc, ks = kc[:Sk], ks[:Sk]
    else:
        qc, qs = _random_tables(rng, Sq, D)
        kc, ks = _random_tables(rng, Sk, D)
        qc, qs, kc, ks = 0.5 * qc, 0.5 * qs, 0.5 * kc, 0.5 * ks
    kw = dict(causal=causal, kv_len=kv_len, sm_scale=0.6)
    dq, dk, dv = rope_attention_bwd_ref(q, k, v, do, qc, qs, kc, ks, **kw)

    def loss():
        return float((rope_attention_ref(q, k, v, qc, qs, kc, ks, **kw) * do).sum())

    eps = 1e-6
    for x, g in ((q, dq), (k, dk), (v, dv)):
        num = np.zeros_like(x)
        it = np.nditer(x, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            old = x[idx]
            x[idx] = old + eps
            fp = loss()
            x[idx] = old - eps
            fm = loss()
            x[idx] = old
            num[idx] = (fp - fm) / (2 * eps)
        np.testing.assert_allclose(g, num, rtol=1e-6, atol=1e-7)

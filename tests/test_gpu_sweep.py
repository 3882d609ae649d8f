"""GPU tier: a seeded random sweep of prefill shapes through the forward (with
LSE) and the backward, against the float64 oracle at the north-star bars.

The fixed-shape tests re-express the reference's own cases; this sweep adds
the combinations they leave out: every dtype with both head dims, GQA ratios
1 to 8, Sq and Sk from below one tile to a few tiles (independently, so
Sq != Sk with top-left causal masking), kv_len < Sk and a non-default scale.
A second, smaller set per test draws the same way at head_dim 256
(bfloat16/float16, the dtypes that have it).
"""

from __future__ import annotations

import numpy as np
import pytest

from gpu_util import check_fwd, check_grad, dev, host, note
from oracle import attention_bwd_ref, attention_ref
from pallas_flash import flash_attention, flash_attention_with_lse

pytestmark = pytest.mark.gpu

N_CASES = 24


def _cases(seed: int):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(N_CASES):
        dt = ("f32", "bf16", "f16")[i % 3]
        D = (64, 128)[(i // 3) % 2]
        Hkv = int(rng.integers(1, 3))
        g = int(rng.choice([1, 2, 4, 8]))
        B = int(rng.integers(1, 3))
        Sq = int(rng.integers(1, 300))
        Sk = int(rng.integers(1, 300))
        causal = bool(rng.integers(0, 2))
        kv_len = int(rng.integers(1, Sk + 1)) if rng.integers(0, 2) else None
        scale = float(rng.uniform(0.05, 0.3)) if i % 5 == 4 else None
        cases.append(pytest.param(dt, D, B, Hkv * g, Hkv, Sq, Sk, causal, kv_len, scale, id=f"c{i}-{dt}-D{D}"))
    return cases


def _wide(cases, seed: int, n: int, tag: str):
    """n cases drawn like `cases`' generator but at head_dim 256, 16-bit dtypes:
    the parameters of n of them with D and dt replaced."""
    rng = np.random.default_rng(seed)
    out = []
    for i, c in enumerate(rng.choice(len(cases), size=n, replace=False)):
        v = list(cases[c].values)
        v[0], v[1] = ("bf16", "f16")[i % 2], 256
        out.append(pytest.param(*v, id=f"{tag}{i}-{v[0]}-D256"))
    return out


def _inputs(seed, dt, B, Hq, Hkv, Sq, Sk, D):
    rng = np.random.default_rng(seed)
    q = dev(rng.standard_normal((B, Hq, Sq, D)), dt)
    k = dev(rng.standard_normal((B, Hkv, Sk, D)), dt)
    v = dev(rng.standard_normal((B, Hkv, Sk, D)), dt)
    do = dev(rng.standard_normal((B, Hq, Sq, D)), dt)
    return q, k, v, do


@pytest.mark.parametrize("dt,D,B,Hq,Hkv,Sq,Sk,causal,kv_len,scale", _cases(101) + _wide(_cases(101), 505, 6, "w"))
def test_sweep_forward_and_lse(dt, D, B, Hq, Hkv, Sq, Sk, causal, kv_len, scale):
    note(f"sweep fwd dt={dt} D={D} B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Sk={Sk} causal={causal} "
         f"kv_len={kv_len} scale={scale}")
    q, k, v, _ = _inputs(11, dt, B, Hq, Hkv, Sq, Sk, D)
    o, lse = flash_attention_with_lse(q, k, v, causal=causal, kv_len=kv_len, sm_scale=scale)
    want_o, want_lse = attention_ref(host(q), host(k), host(v), causal=causal, kv_len=kv_len, sm_scale=scale)
    check_fwd(host(o), want_o, dt)
    # LSE is float32 for every input dtype; the bar is relative to its scale
    lse_err = np.abs(host(lse) - want_lse).max() / (np.abs(want_lse).max() + 1.0)
    assert lse_err <= (1e-5 if dt == "f32" else 1e-3), f"lse error {lse_err:.3e}"


@pytest.mark.parametrize("dt,D,B,Hq,Hkv,Sq,Sk,causal,kv_len,scale", _cases(202) + _wide(_cases(202), 606, 6, "w"))
def test_sweep_backward(dt, D, B, Hq, Hkv, Sq, Sk, causal, kv_len, scale):
    note(f"sweep bwd dt={dt} D={D} B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Sk={Sk} causal={causal} "
         f"kv_len={kv_len} scale={scale}")
    q, k, v, do = _inputs(12, dt, B, Hq, Hkv, Sq, Sk, D)
    for t in (q, k, v):
        t.requires_grad_(True)
    flash_attention(q, k, v, causal=causal, kv_len=kv_len, sm_scale=scale).backward(do)
    want = attention_bwd_ref(host(q), host(k), host(v), host(do), causal=causal, kv_len=kv_len, sm_scale=scale)
    for name, t, w in zip("qkv", (q, k, v), want):
        check_grad(host(t.grad), w, dt, "d" + name)
    if kv_len is not None:
        # keys at or past kv_len get exactly zero gradient
        assert (host(k.grad)[:, :, kv_len:] == 0).all() and (host(v.grad)[:, :, kv_len:] == 0).all()


def _rope_cases(seed: int, n: int):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        dt = ("bf16", "f16", "f32")[i % 3]
        D = (128, 64)[(i // 3) % 2]
        Hkv = int(rng.integers(1, 3))
        g = int(rng.choice([1, 2, 4]))
        Sq = int(rng.integers(1, 260))
        Sk = Sq if i % 2 == 0 else int(rng.integers(1, 260))
        causal = bool(rng.integers(0, 2))
        kv_len = int(rng.integers(1, Sk + 1)) if rng.integers(0, 2) else None
        cases.append(pytest.param(dt, D, Hkv * g, Hkv, Sq, Sk, causal, kv_len, id=f"r{i}-{dt}-D{D}"))
    return cases


@pytest.mark.parametrize("dt,D,Hq,Hkv,Sq,Sk,causal,kv_len",
                         _rope_cases(303, 12) + _wide(_rope_cases(303, 12), 707, 4, "rw"))
def test_sweep_rope_forward_backward(dt, D, Hq, Hkv, Sq, Sk, causal, kv_len):
    """Fused RoPE (separate K tables when Sq != Sk, fused_rope.py:154-160)
    forward and its RoPE-aware backward vs the oracle."""
    from oracle import rope_attention_bwd_ref, rope_attention_ref
    from pallas_flash import flash_attention_rope, precompute_rope
    note(f"sweep rope dt={dt} D={D} Hq={Hq} Hkv={Hkv} Sq={Sq} Sk={Sk} causal={causal} kv_len={kv_len}")
    q, k, v, do = _inputs(13, dt, 1, Hq, Hkv, Sq, Sk, D)
    cos, sin = precompute_rope(max(Sq, Sk), D, 10000.0, device="cuda")
    qc, qs, kc, ks = cos[:Sq], sin[:Sq], cos[:Sk], sin[:Sk]
    for t in (q, k, v):
        t.requires_grad_(True)
    out = flash_attention_rope(q, k, v, qc, qs, kc, ks, causal=causal, kv_len=kv_len)
    out.backward(do)
    args = (host(q), host(k), host(v))
    tabs = (host(qc), host(qs), host(kc), host(ks))
    check_fwd(host(out), rope_attention_ref(*args, *tabs, causal=causal, kv_len=kv_len), dt)
    want = rope_attention_bwd_ref(*args, host(do), *tabs, causal=causal, kv_len=kv_len)
    for name, t, w in zip("qkv", (q, k, v), want):
        check_grad(host(t.grad), w, dt, "d" + name)


def _decode_cases(seed: int, n: int):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        dt = ("bf16", "f16", "f32")[i % 3]
        D = (128, 64)[(i // 3) % 2]
        Hkv = int(rng.integers(1, 4))
        g = int(rng.choice([1, 2, 4, 8]))
        B = int(rng.integers(1, 5))
        cap = int(rng.integers(1, 700))
        L = int(rng.integers(1, cap + 1))
        cases.append(pytest.param(dt, D, B, Hkv * g, Hkv, cap, L, id=f"d{i}-{dt}-D{D}"))
    return cases


@pytest.mark.parametrize("dt,D,B,Hq,Hkv,cap,L", _decode_cases(404, 12) + _wide(_decode_cases(404, 12), 808, 4, "dw"))
def test_sweep_decode(dt, D, B, Hq, Hkv, cap, L):
    """Decode over the [0, L) prefix of a cache of `cap` slots whose tail is
    NaN (test_decode.py:33, :38-49)."""
    from oracle import decode_ref
    from pallas_flash import flash_attention_decode
    note(f"sweep decode dt={dt} D={D} B={B} Hq={Hq} Hkv={Hkv} cap={cap} L={L}")
    rng = np.random.default_rng(14)
    q = rng.standard_normal((B, Hq, 1, D))
    k = rng.standard_normal((B, Hkv, cap, D))
    v = rng.standard_normal((B, Hkv, cap, D))
    k[:, :, L:] = np.nan
    v[:, :, L:] = np.nan
    tq, tk, tv = dev(q, dt), dev(k, dt), dev(v, dt)
    out = host(flash_attention_decode(tq, tk, tv, L))
    check_fwd(out, decode_ref(host(tq), host(tk), host(tv), L), dt)


@pytest.mark.parametrize("seed", range(12))
def test_sweep_paged(seed):
    """Paged decode over scrambled, partly shared pages with -1 padding past
    each sequence's last page and NaN everywhere no valid row lives
    (paged.py:119-121; test_paged.py:25-28, :61-91). Seeds 8-11: head_dim 256."""
    from oracle import paged_ref
    from pallas_flash import paged_flash_attention
    import torch
    rng = np.random.default_rng(500 + seed)
    if seed < 8:
        dt = ("bf16", "f16", "f32")[seed % 3]
        D = (128, 64)[(seed // 3) % 2]
    else:
        dt, D = ("bf16", "f16")[seed % 2], 256
    Hkv = int(rng.integers(1, 4))
    Hq = Hkv * int(rng.choice([1, 2, 4, 8]))
    page = int(rng.choice([16, 32, 64, 128]))
    B = int(rng.integers(1, 6))
    lens = rng.integers(0, 5 * page + 1, B).astype(np.int32)
    P = int(max(1, -(-int(lens.max()) // page)))
    num_pages = B * P + 3
    note(f"sweep paged dt={dt} D={D} B={B} Hq={Hq} Hkv={Hkv} page={page} lens={lens.tolist()}")
    table = np.full((B, P), -1, np.int32)
    perm = rng.permutation(num_pages)
    used = 0
    for b in range(B):
        n = -(-int(lens[b]) // page)
        table[b, :n] = perm[used:used + n]
        used += n
    if B > 1 and lens[0] > 0 and lens[1] > 0:
        table[1, 0] = table[0, 0]  # a page shared by the first two sequences
    # Rows no sequence reads stay NaN; a shared page gets the valid rows of
    # both sequences (the later fill overwrites the earlier one's rows).
    kp = np.full((num_pages, Hkv, page, D), np.nan)
    vp = np.full((num_pages, Hkv, page, D), np.nan)
    for b in range(B):
        for j in range(-(-int(lens[b]) // page)):
            rows = min(page, int(lens[b]) - j * page)
            kp[table[b, j], :, :rows] = rng.standard_normal((Hkv, rows, D))
            vp[table[b, j], :, :rows] = rng.standard_normal((Hkv, rows, D))
    q = rng.standard_normal((B, Hq, 1, D))
    tq, tk, tv = dev(q, dt), dev(kp, dt), dev(vp, dt)
    out = host(paged_flash_attention(tq, tk, tv, torch.as_tensor(table), torch.as_tensor(lens)))
    check_fwd(out, paged_ref(host(tq), host(tk), host(tv), table, lens), dt)

"""GPU tier: head_dim 256 (bfloat16/float16) on every path, and head dims in
(128, 256) padded or read in place, vs the float64 oracle.

The reference bounds no head_dim (flash_attention.py:527-545; fused_rope.py:
168-169 asks only for an even one; paged.py:135-139 only that q and the pages
agree). Here the 16-bit kernels take head_dim 256 -- the forward, dQ and
decode kernels at one workgroup per CU, dK/dV as two workgroups per key block,
one per 128-column half of dK/dV (both recompute S and dP over all 256
columns) -- and float32 compute stops at 128 (NotImplementedError above).
Head dims between 128 and 256 are zero-padded for prefill and read in place
by decode, paged decode and the cache writes when their rows are whole
16-byte chunks (a multiple of 8 elements).

Bars as everywhere: outputs 2e-2 max-abs (16-bit), gradients 5e-2 relative.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from gpu_util import DEV, check_fwd, check_grad, dev, host, note
from oracle import (attention_bwd_ref, attention_ref, decode_ref, paged_ref, precompute_rope_ref,
                    rope_attention_bwd_ref, rope_attention_ref)
from pallas_flash import (_lib, flash_attention, flash_attention_decode, flash_attention_rope,
                          paged_flash_attention)

pytestmark = pytest.mark.gpu


def _fwd_bwd(dt, B, Hq, Hkv, Sq, Sk, d, causal, kv_len, seed):
    rng = np.random.default_rng(seed)
    q, do = rng.standard_normal((B, Hq, Sq, d)), rng.standard_normal((B, Hq, Sq, d))
    k, v = rng.standard_normal((B, Hkv, Sk, d)), rng.standard_normal((B, Hkv, Sk, d))
    tq, tk, tv = (dev(x, dt).requires_grad_(True) for x in (q, k, v))
    tdo = dev(do, dt)
    out = flash_attention(tq, tk, tv, causal=causal, kv_len=kv_len)
    assert out.shape == (B, Hq, Sq, d) and out.dtype == tq.dtype
    out.backward(tdo)
    torch.cuda.synchronize()
    qh, kh, vh, doh = host(tq), host(tk), host(tv), host(tdo)
    ref, _ = attention_ref(qh, kh, vh, causal=causal, kv_len=kv_len)
    check_fwd(host(out), ref, dt)
    want = attention_bwd_ref(qh, kh, vh, doh, causal=causal, kv_len=kv_len)
    for name, t, w in zip("qkv", (tq, tk, tv), want):
        assert t.grad.shape == t.shape and t.grad.dtype == t.dtype
        check_grad(host(t.grad), w, dt, f"d{name}")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,causal,kv_len", [
    (1, 4, 2, 200, 200, True, None),      # GQA 2, ragged blocks, causal
    (2, 2, 2, 129, 300, False, 257),      # MHA, Sq != Sk, kv_len tail
    (1, 8, 1, 256, 256, True, 190),       # MQA, causal with a kv_len cut
])
def test_head_dim_256_forward_backward(dt, B, Hq, Hkv, Sq, Sk, causal, kv_len):
    note(f"d256: fwd+bwd dt={dt} B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Sk={Sk} causal={causal} kv_len={kv_len}")
    _fwd_bwd(dt, B, Hq, Hkv, Sq, Sk, 256, causal, kv_len, seed=Sq + Sk)


@pytest.mark.parametrize("d", [136, 192, 200])
def test_head_dims_above_128_padded_to_256(d):
    note(f"d256: padded head_dim={d} bf16 fwd+bwd")
    _fwd_bwd("bf16", 1, 4, 2, 160, 160, d, True, 150, seed=d)


def test_head_dim_256_float32_is_not_implemented():
    """Float32 compute (float32 or mixed inputs) stops at head_dim 128."""
    x = torch.zeros((1, 2, 8, 256), device=DEV)
    with pytest.raises(NotImplementedError):
        flash_attention(x, x, x)
    with pytest.raises(NotImplementedError):
        flash_attention(x.bfloat16(), x, x)   # mixed: computed in float32


@pytest.mark.parametrize("d", [256, 192])
def test_rope_head_dim_above_128(d):
    note(f"d256: rope head_dim={d} bf16 fwd+bwd")
    rng = np.random.default_rng(d + 3)
    B, Hq, Hkv, S = 1, 4, 2, 150
    q, k, v, do = (rng.standard_normal(s) for s in ((B, Hq, S, d), (B, Hkv, S, d), (B, Hkv, S, d),
                                                   (B, Hq, S, d)))
    cos, sin = precompute_rope_ref(S, d)
    tq, tk, tv = (dev(x, "bf16").requires_grad_(True) for x in (q, k, v))
    tcos, tsin = (torch.as_tensor(x, dtype=torch.float32, device=DEV) for x in (cos, sin))
    out = flash_attention_rope(tq, tk, tv, tcos, tsin, causal=True)
    out.backward(dev(do, "bf16"))
    torch.cuda.synchronize()
    qh, kh, vh = host(tq), host(tk), host(tv)
    # the kernel rounds the rotated q and k to bfloat16 before the products:
    # the bar is the bf16 one on the output, relative 5e-2 on the gradients
    check_fwd(host(out), rope_attention_ref(qh, kh, vh, cos, sin, causal=True), "bf16")
    want = rope_attention_bwd_ref(qh, kh, vh, host(dev(do, "bf16")), cos, sin, causal=True)
    for name, t, w in zip("qkv", (tq, tk, tv), want):
        check_grad(host(t.grad), w, "bf16", f"d{name}")


def _peak_extra(fn):
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    out = fn()
    torch.cuda.synchronize()
    return out, torch.cuda.max_memory_allocated() - before


@pytest.mark.parametrize("d,dt", [(256, "bf16"), (256, "f16"), (200, "bf16"), (136, "f16")])
def test_decode_head_dim_above_128_in_place(d, dt):
    note(f"d256: decode in place head_dim={d} dt={dt}")
    rng = np.random.default_rng(d + 5)
    B, Hq, Hkv, cap, L = 3, 16, 4, 1024, 700
    q = rng.standard_normal((B, Hq, 1, d))
    kc, vc = rng.standard_normal((B, Hkv, cap, d)), rng.standard_normal((B, Hkv, cap, d))
    kc[:, :, L:] = np.nan
    vc[:, :, L:] = np.nan
    tq, tk, tv = dev(q, dt), dev(kc, dt), dev(vc, dt)
    out, extra = _peak_extra(lambda: flash_attention_decode(tq, tk, tv, L))
    cache_bytes = tk.numel() * tk.element_size()
    assert extra < cache_bytes // 4, f"call allocated {extra} bytes beside a {cache_bytes}-byte cache"
    assert out.shape == (B, Hq, 1, d)
    check_fwd(host(out), decode_ref(host(tq), host(tk)[:, :, :L], host(tv)[:, :, :L], L), dt)


@pytest.mark.parametrize("d,page", [(256, 16), (256, 5), (200, 32)])
def test_paged_head_dim_above_128_in_place(d, page):
    """Scrambled, -1-padded table; NaN in every unreferenced page and past
    each sequence's length; no pool-sized allocation."""
    note(f"d256: paged in place head_dim={d} page={page}")
    rng = np.random.default_rng(d + page)
    num_pages, pps, B, Hq, Hkv = 160, 24, 4, 8, 2
    kp = rng.standard_normal((num_pages, Hkv, page, d))
    vp = rng.standard_normal((num_pages, Hkv, page, d))
    lens = np.array([pps * page, 1, 37, pps * page // 2 + 3], np.int32)
    table = np.full((B, pps), -1, np.int32)
    perm = rng.permutation(num_pages)
    used = 0
    for b in range(B):
        n = -(-int(lens[b]) // page)
        table[b, :n] = perm[used:used + n]
        used += n
    kp[perm[used:]] = np.nan
    vp[perm[used:]] = np.nan
    for b in range(B):
        n, r = -(-int(lens[b]) // page), int(lens[b]) % page
        if r:
            kp[table[b, n - 1], :, r:] = np.nan
            vp[table[b, n - 1], :, r:] = np.nan
    q = rng.standard_normal((B, Hq, 1, d))
    tq, tk, tv = dev(q, "bf16"), dev(kp, "bf16"), dev(vp, "bf16")
    tt, tl = torch.as_tensor(table).to(DEV), torch.as_tensor(lens).to(DEV)
    out, extra = _peak_extra(lambda: paged_flash_attention(tq, tk, tv, tt, tl))
    pool_bytes = tk.numel() * tk.element_size()
    assert extra < pool_bytes // 4, f"call allocated {extra} bytes beside a {pool_bytes}-byte pool"
    check_fwd(host(out), paged_ref(host(tq), np.nan_to_num(host(tk)), np.nan_to_num(host(tv)), table, lens),
              "bf16")


def test_head_dim_256_dynamic_tail_bit_identical():
    """At a size with enough work items for the forward and dQ dynamic tail
    (B=2, Hq=32, Hkv=8, S=2048: 1024 items each), the three prefill launches
    give the same bits with every item placed statically and with 30% and
    100% of the items drawn at run time; outputs are NaN-filled before each
    call, so an item no workgroup took would show."""
    note("d256: dynamic tail bit-identity")
    B, Hq, Hkv, S, D = 2, 32, 8, 2048, 256
    g = torch.Generator(device=DEV).manual_seed(9)
    mk = lambda *s: torch.randn(s, generator=g, device=DEV).to(torch.bfloat16)
    q, k, v, do = mk(B, Hq, S, D), mk(B, Hkv, S, D), mk(B, Hkv, S, D), mk(B, Hq, S, D)
    o = torch.empty_like(q)
    lse, delta = torch.empty((B, Hq, S), device=DEV), torch.empty((B, Hq, S), device=DEV)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    sc = D ** -0.5
    fa = _lib.FwdArgs(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                      B, Hq, Hkv, S, S, D, S, 1, sc, _lib.dtype_tag(q))
    ba = _lib.BwdArgs(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(), lse.data_ptr(),
                      delta.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                      B, Hq, Hkv, S, S, D, S, 1, sc, _lib.dtype_tag(q))
    outs = (o, lse, delta, dq, dk, dv)
    L = _lib.lib()
    st = torch.cuda.current_stream().cuda_stream

    def run():
        for t in outs:
            t.fill_(float("nan"))
        assert L.pf_attn_fwd(ctypes.byref(fa), st) == 0
        assert L.pf_attn_bwd_dq(ctypes.byref(ba), st) == 0
        assert L.pf_attn_bwd_dkv(ctypes.byref(ba), st) == 0
        torch.cuda.synchronize()

    with _lib.tuning(tail_dynamic_pct=0):
        run()
        ref = [t.clone() for t in outs]
    assert all(torch.isfinite(t).all() for t in ref)
    for pct in (30, 100):
        with _lib.tuning(tail_dynamic_pct=pct):
            for rep in range(2):
                run()
                assert all(torch.equal(x, y) for x, y in zip(outs, ref)), f"share {pct}%, call {rep}"

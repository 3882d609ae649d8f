"""GPU tier: head dims other than 64/128 and mixed input dtypes through the
reference's API (zero-padding to the kernels' head_dim, float32 compute for
mixed dtypes; pallas_flash._shape) vs the float64 oracle on the caller's
unpadded inputs.

The reference takes any head_dim and casts every operand to float32 in its
kernels (flash_attention.py:91-93, fused_rope.py:70-72, paged.py:68-70),
returning q's dtype (flash_attention.py:212) and each input's dtype for the
gradients (flash_attention.py:438-442). Bars: an output or gradient stored in
bf16/f16 is held to that dtype's bar, one stored in float32/float64 (float32
compute) to the float32 bar.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import DEV, check_fwd, check_grad, dev, host, note
from oracle import (attention_bwd_ref, attention_ref, decode_ref, paged_ref, precompute_rope_ref,
                    rope_attention_bwd_ref, rope_attention_ref)
from pallas_flash import (flash_attention, flash_attention_decode, flash_attention_rope,
                          paged_flash_attention)

pytestmark = pytest.mark.gpu

BAR = {torch.float32: "f32", torch.float64: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


def _t(x, dtype):
    return torch.as_tensor(np.ascontiguousarray(x)).to(DEV).to(dtype).contiguous()


@pytest.mark.parametrize("d", [32, 80, 96])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_head_dim_padding_forward_backward(d, dt):
    note(f"shapes: head_dim={d} dt={dt}")
    rng = np.random.default_rng(d)
    B, Hq, Hkv, S, kv_len = 1, 4, 2, 160, 150
    q, k, v, do = (rng.standard_normal(s) for s in ((B, Hq, S, d), (B, Hkv, S, d), (B, Hkv, S, d),
                                                   (B, Hq, S, d)))
    tq, tk, tv = (dev(x, dt).requires_grad_(True) for x in (q, k, v))
    tdo = dev(do, dt)
    out = flash_attention(tq, tk, tv, causal=True, kv_len=kv_len)
    assert out.shape == (B, Hq, S, d) and out.dtype == tq.dtype
    out.backward(tdo)
    torch.cuda.synchronize()
    qh, kh, vh, doh = host(tq), host(tk), host(tv), host(tdo)
    ref, _ = attention_ref(qh, kh, vh, causal=True, kv_len=kv_len)   # default scale 1/sqrt(d)
    check_fwd(host(out), ref, dt)
    want = attention_bwd_ref(qh, kh, vh, doh, causal=True, kv_len=kv_len)
    for name, t, w in zip("qkv", (tq, tk, tv), want):
        assert t.grad.shape == t.shape and t.grad.dtype == t.dtype
        check_grad(host(t.grad), w, dt, f"d{name}")


def test_mixed_dtypes_compute_in_float32():
    note("shapes: mixed dtypes q bf16, k f32, v f16")
    rng = np.random.default_rng(7)
    q, k, v, do = (rng.standard_normal(s) for s in ((1, 4, 96, 128), (1, 2, 96, 128), (1, 2, 96, 128),
                                                   (1, 4, 96, 128)))
    tq = _t(q, torch.bfloat16).requires_grad_(True)
    tk = _t(k, torch.float32).requires_grad_(True)
    tv = _t(v, torch.float16).requires_grad_(True)
    out = flash_attention(tq, tk, tv, causal=True)
    assert out.dtype == torch.bfloat16
    out.backward(_t(do, torch.bfloat16))
    torch.cuda.synchronize()
    qh, kh, vh = host(tq), host(tk), host(tv)
    ref, _ = attention_ref(qh, kh, vh, causal=True)
    check_fwd(host(out), ref, "bf16")
    want = attention_bwd_ref(qh, kh, vh, host(_t(do, torch.bfloat16)), causal=True)
    for name, t, w in zip("qkv", (tq, tk, tv), want):
        assert t.grad.dtype == t.dtype
        check_grad(host(t.grad), w, BAR[t.dtype], f"d{name}")


def test_float64_inputs_compute_in_float32():
    note("shapes: float64 inputs")
    rng = np.random.default_rng(8)
    q, k, v = (rng.standard_normal((1, 2, 64, 64)) for _ in range(3))
    out = flash_attention(*(_t(x, torch.float64) for x in (q, k, v)))
    assert out.dtype == torch.float64
    ref, _ = attention_ref(*(x.astype(np.float32).astype(np.float64) for x in (q, k, v)))
    check_fwd(host(out), ref, "f32")


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_decode_head_dim_80(dt):
    note(f"shapes: decode head_dim=80 dt={dt}")
    rng = np.random.default_rng(80)
    cap, L = 300, 257
    q = rng.standard_normal((3, 8, 1, 80))
    kc = rng.standard_normal((3, 2, cap, 80))
    vc = rng.standard_normal((3, 2, cap, 80))
    kc[:, :, L:] = np.nan
    vc[:, :, L:] = np.nan
    tq, tk, tv = dev(q, dt), dev(kc, dt), dev(vc, dt)
    out = flash_attention_decode(tq, tk, tv, L)
    torch.cuda.synchronize()
    assert out.shape == (3, 8, 1, 80)
    check_fwd(host(out), decode_ref(host(tq), host(tk)[:, :, :L], host(tv)[:, :, :L], L), dt)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_paged_head_dim_32(dt):
    note(f"shapes: paged head_dim=32 dt={dt}")
    rng = np.random.default_rng(32)
    num_pages, page, pps, B = 24, 16, 5, 3
    kp = rng.standard_normal((num_pages, 2, page, 32))
    vp = rng.standard_normal((num_pages, 2, page, 32))
    table = rng.permutation(num_pages)[:B * pps].reshape(B, pps).astype(np.int32)
    lens = np.array([70, 16, 5], np.int32)
    q = rng.standard_normal((B, 4, 1, 32))
    tq, tk, tv = dev(q, dt), dev(kp, dt), dev(vp, dt)
    out = paged_flash_attention(tq, tk, tv, torch.as_tensor(table), torch.as_tensor(lens))
    torch.cuda.synchronize()
    check_fwd(host(out), paged_ref(host(tq), host(tk), host(tv), table, lens), dt)


def _peak_extra(fn):
    """Run fn; return (its result, device bytes allocated at the peak beyond
    what was allocated before the call)."""
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    out = fn()
    torch.cuda.synchronize()
    return out, torch.cuda.max_memory_allocated() - before


@pytest.mark.parametrize("d,dt", [(96, "bf16"), (80, "bf16"), (80, "f16"), (96, "f32"), (36, "f32")])
def test_decode_head_dim_read_in_place(d, dt):
    """Decode at a head_dim the kernels read in place: checked against the
    oracle, NaN past cache_len, and no cache-sized allocation in the call."""
    note(f"shapes: decode in place head_dim={d} dt={dt}")
    rng = np.random.default_rng(d)
    B, Hq, Hkv, cap, L = 4, 16, 4, 2048, 1500
    q = rng.standard_normal((B, Hq, 1, d))
    kc = rng.standard_normal((B, Hkv, cap, d))
    vc = rng.standard_normal((B, Hkv, cap, d))
    kc[:, :, L:] = np.nan
    vc[:, :, L:] = np.nan
    tq, tk, tv = dev(q, dt), dev(kc, dt), dev(vc, dt)
    out, extra = _peak_extra(lambda: flash_attention_decode(tq, tk, tv, L))
    cache_bytes = tk.numel() * tk.element_size()
    assert extra < cache_bytes // 4, f"call allocated {extra} bytes beside a {cache_bytes}-byte cache"
    assert out.shape == (B, Hq, 1, d)
    check_fwd(host(out), decode_ref(host(tq), host(tk)[:, :, :L], host(tv)[:, :, :L], L), dt)


@pytest.mark.parametrize("d,dt", [(96, "bf16"), (80, "bf16"), (80, "f32")])
def test_paged_head_dim_read_in_place(d, dt):
    """Paged decode at a head_dim the kernels read in place over a scrambled,
    -1-padded table with NaN in unreferenced pages: checked against the oracle
    and no pool-sized allocation in the call."""
    note(f"shapes: paged in place head_dim={d} dt={dt}")
    rng = np.random.default_rng(d + 1)
    num_pages, page, pps, B, Hq, Hkv = 512, 16, 40, 8, 16, 4
    kp = rng.standard_normal((num_pages, Hkv, page, d))
    vp = rng.standard_normal((num_pages, Hkv, page, d))
    lens = rng.integers(1, pps * page + 1, size=B).astype(np.int32)
    table = np.full((B, pps), -1, np.int32)
    perm = rng.permutation(num_pages)
    used = 0
    for b in range(B):
        n = -(-int(lens[b]) // page)
        table[b, :n] = perm[used:used + n]
        used += n
    unused = perm[used:]
    kp[unused] = np.nan
    vp[unused] = np.nan
    for b in range(B):  # rows past each sequence's length in its last page
        n, r = -(-int(lens[b]) // page), int(lens[b]) % page
        if r:
            kp[table[b, n - 1], :, r:] = np.nan
            vp[table[b, n - 1], :, r:] = np.nan
    q = rng.standard_normal((B, Hq, 1, d))
    tq, tk, tv = dev(q, dt), dev(kp, dt), dev(vp, dt)
    tt, tl = torch.as_tensor(table).to(DEV), torch.as_tensor(lens).to(DEV)
    out, extra = _peak_extra(lambda: paged_flash_attention(tq, tk, tv, tt, tl))
    pool_bytes = tk.numel() * tk.element_size()
    assert extra < pool_bytes // 4, f"call allocated {extra} bytes beside a {pool_bytes}-byte pool"
    check_fwd(host(out), paged_ref(host(tq), np.nan_to_num(host(tk)), np.nan_to_num(host(tv)), table, lens), dt)


def test_decode_head_dim_copy_path_warns():
    """A head_dim the kernels cannot read in place (100 in bfloat16: rows of
    200 bytes) still computes correctly through the padded copy, and says so
    once."""
    note("shapes: decode head_dim=100 bf16 copy path")
    import warnings
    from pallas_flash import _shape
    _shape._warned.discard("flash_attention_decode")
    rng = np.random.default_rng(100)
    q = rng.standard_normal((2, 4, 1, 100))
    kc = rng.standard_normal((2, 2, 64, 100))
    vc = rng.standard_normal((2, 2, 64, 100))
    tq, tk, tv = dev(q, "bf16"), dev(kc, "bf16"), dev(vc, "bf16")
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        out = flash_attention_decode(tq, tk, tv, 50)
        flash_attention_decode(tq, tk, tv, 50)
    assert sum("copied on every call" in str(x.message) for x in w) == 1
    check_fwd(host(out), decode_ref(host(tq), host(tk)[:, :, :50], host(tv)[:, :, :50], 50), "bf16")


def test_rope_head_dim_96_forward_backward():
    note("shapes: rope head_dim=96 f32 causal")
    rng = np.random.default_rng(96)
    B, Hq, Hkv, S, d = 1, 4, 2, 130, 96
    q, k, v, do = (rng.standard_normal(s) for s in ((B, Hq, S, d), (B, Hkv, S, d), (B, Hkv, S, d),
                                                   (B, Hq, S, d)))
    cos, sin = precompute_rope_ref(S, d)
    tq, tk, tv = (dev(x, "f32").requires_grad_(True) for x in (q, k, v))
    tcos, tsin = _t(cos, torch.float32), _t(sin, torch.float32)
    out = flash_attention_rope(tq, tk, tv, tcos, tsin, causal=True)
    out.backward(dev(do, "f32"))
    torch.cuda.synchronize()
    check_fwd(host(out), rope_attention_ref(q, k, v, cos, sin, causal=True), "f32")
    want = rope_attention_bwd_ref(q, k, v, do, cos, sin, causal=True)
    for name, t, w in zip("qkv", (tq, tk, tv), want):
        check_grad(host(t.grad), w, "f32", f"d{name}")


def test_rope_head_dim_96_bf16_inference():
    note("shapes: rope head_dim=96 bf16 inference")
    rng = np.random.default_rng(97)
    q, k, v = (rng.standard_normal((1, 4, 200, 96)) for _ in range(3))
    cos, sin = precompute_rope_ref(200, 96)
    tq, tk, tv = (dev(x, "bf16") for x in (q, k, v))
    with torch.no_grad():
        out = flash_attention_rope(tq, tk, tv, _t(cos, torch.float32), _t(sin, torch.float32),
                                   causal=True)
    torch.cuda.synchronize()
    check_fwd(host(out), rope_attention_ref(host(tq), host(tk), host(tv), cos, sin, causal=True), "bf16")

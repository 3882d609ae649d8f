#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (one JSON line on stdout).

Headline ("value"): flash_attention forward+backward at BASELINE config 3
(bf16, causal, GQA, B=2, Hq=16, Hkv=4, S=8192, D=128) in algorithmic
TFLOP/s: 4*B*Hq*D*S(S+1)/2 per forward, x3.5 for forward+backward
(recomputation not credited). One step = one forward + backward over the
resident synthetic batch: pf_attn_fwd, then pf_attn_bwd_dq (which also
computes delta = rowsum(o * do)) and pf_attn_bwd_dkv, called through the C
ABI on torch's current stream with HIP events between the launches
(per-kernel durations).

Secondary figures in the same line (each timed with HIP events; medians
over the timed launches, after at least as many untimed ones as --warmup):
  fwd_tflops    config 3 forward alone (the pf_attn_fwd launches of the steps,
                each between the previous step's dK/dV and the next dQ; mean)
  fwd_loop_tflops  config 3 forward as back-to-back forward launches after the
                steps (the reference's benchmark_attention.py timing; mean)
  rope_tflops   config 2 fused-RoPE prefill, bf16 causal GQA B=4 Hq=32 Hkv=8 S=4096
                (K rotation + attention); fwd_cfg2_shape_ms is the plain forward
                at that shape, timed in alternation (rope_over_plain_fwd)
  decode_gbs    config 4 decode, B=64 Hq=32 Hkv=8, cache 8192 with kv_len 6000
                (slots past 6000 NaN); algorithmic bytes = valid K/V once + q + o
  decode_step_gbs  config 4's shape as one fused decode step (RoPE of the new
                token at position 5999, cache-slot write, attention over 6000
                slots; position in device memory), timed in alternation with
                the config 4 decode on the same cache
  paged_gbs     config 5 paged decode, 128 seqs, page 64, lens U[512, 8192] from
                np.random.default_rng(0), 16384-page pool, -1-padded table,
                unreferenced pages and tails NaN; bytes = valid K/V + q + o +
                used table entries + lens
  hbm_read_ceiling_gbs  a plain streaming read of 2 GiB (the best of three
                load forms -- non-temporal and temporal register loads and
                direct global->LDS loads -- over a few launch shapes; each form's best
                in hbm_read_by_form_gbs): what a read-only HBM stream reaches on
                this device; *_frac_read_ceiling relate decode/paged to it
  mfma_stream_ceiling_tflops  back-to-back bf16 32x32x16 MFMAs on register
                operands (no memory traffic), the best of a few launch shapes:
                the matrix-core rate this box sustains under a pure MFMA load;
                *_frac_mfma_ceiling relate the prefill kernels to it (beside
                *_frac_mfma, against the 2.5 PFLOP/s specification), so a slow
                box and a slow kernel can be told apart
  dq_tflops, dkv_tflops  the config 3 dQ and dK/dV kernels at their credits
                (dQ 1 matmul, dK/dV 4 of the 7 the step credits)

Synthetic inputs: N(0,1) from torch's CUDA generator seeded 0 (config 5's
lengths and page permutation from numpy's default_rng(0)), cast to bf16.

CPU baselines (reported, not targets; the float32 numpy oracle, timed on this
host's cores on a bounded sample of each workload): "cpu_baseline" for config
3 forward+backward (a quarter of the heads, median of three passes after a
warm-up), and secondary.cpu_baselines for config 2 (fused RoPE),
config 4 (decode, per sequence on the sliced prefix) and config 5 (paged,
per sequence on the gathered pages). "cores" is the number of host cores
this process may run on; "blas_threads" numpy's BLAS thread count.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "tpu-native-pallas-flashattention_amd")
for _p in (ROOT, PKG_DIR):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "attn TFLOP/s fwd & fwd+bwd at S=8K D=128; decode/paged HBM GB/s (1 GPU)"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def causal_pairs(S: int) -> int:
    return S * (S + 1) // 2


def fwd_flops(B, Hq, D, pairs) -> float:
    return 4.0 * B * Hq * D * pairs


class Events:
    """Pairs of HIP events recorded on the current stream."""

    def __init__(self, n_marks: int, n_iters: int):
        import torch
        self.ev = [[torch.cuda.Event(enable_timing=True) for _ in range(n_marks)] for _ in range(n_iters)]

    def mark(self, it: int, j: int):
        self.ev[it][j].record()

    def mean_ms(self, j0: int, j1: int) -> float:
        return float(np.mean([e[j0].elapsed_time(e[j1]) for e in self.ev]))

    def median_ms(self, j0: int, j1: int) -> float:
        return float(np.median([e[j0].elapsed_time(e[j1]) for e in self.ev]))


def ok(status: int, what: str):
    if status != 0:
        raise RuntimeError(f"{what} failed with status {status}")


def bench_cfg3(L, _lib, torch, steps, warmup):
    B, Hq, Hkv, S, D = 2, 16, 4, 8192, 128
    g = torch.Generator(device="cuda").manual_seed(0)
    mk = lambda *shape: torch.randn(shape, generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    q, k, v, do = mk(B, Hq, S, D), mk(B, Hkv, S, D), mk(B, Hkv, S, D), mk(B, Hq, S, D)
    o = torch.empty_like(q)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device="cuda")
    delta = torch.empty_like(lse)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    scale = 1.0 / D ** 0.5
    fa = _lib.FwdArgs(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                      B, Hq, Hkv, S, S, D, S, 1, scale, 1)
    ba = _lib.BwdArgs(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
                      lse.data_ptr(), delta.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                      B, Hq, Hkv, S, S, D, S, 1, scale, 1)
    st = torch.cuda.current_stream().cuda_stream

    def step(ev=None, it=0):
        if ev: ev.mark(it, 0)
        ok(L.pf_attn_fwd(fa, st), "pf_attn_fwd")
        if ev: ev.mark(it, 1)
        ok(L.pf_attn_bwd_dq(ba, st), "pf_attn_bwd_dq")  # also writes delta
        if ev: ev.mark(it, 2)
        ok(L.pf_attn_bwd_dkv(ba, st), "pf_attn_bwd_dkv")
        if ev: ev.mark(it, 3)

    for _ in range(warmup):
        step()
    ev = Events(4, steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(ev, i)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    kern_ms = {"pf_attn_fwd_kernel": ev.mean_ms(0, 1), "pf_attn_bwd_dq_kernel": ev.mean_ms(1, 2),
               "pf_attn_bwd_dkv_kernel": ev.mean_ms(2, 3)}
    # The forward alone as the reference's benchmark_attention.py:28-36 times
    # it: back-to-back forward calls (here each launch between two events).
    for _ in range(warmup):
        ok(L.pf_attn_fwd(fa, st), "pf_attn_fwd")
    fev = Events(2, steps)
    for i in range(steps):
        fev.mark(i, 0)
        ok(L.pf_attn_fwd(fa, st), "pf_attn_fwd")
        fev.mark(i, 1)
    torch.cuda.synchronize()
    fwd_loop_ms = fev.mean_ms(0, 1)
    F = fwd_flops(B, Hq, D, causal_pairs(S))
    # algorithmic credit per launch: fwd = 2 matmuls; dkv = S, dP, dV, dK (4); dq = dQ (1)
    credit = {"pf_attn_fwd_kernel": F, "pf_attn_bwd_dq_kernel": 0.5 * F, "pf_attn_bwd_dkv_kernel": 2.0 * F}
    host = {"q": q, "k": k, "v": v, "do": do}
    return dict(B=B, Hq=Hq, Hkv=Hkv, S=S, D=D, wall_ms=wall_ms, kern_ms=kern_ms, F=F, credit=credit,
                host=host, fwd_loop_ms=fwd_loop_ms)


def bench_rope(L, _lib, torch, iters, warmup):
    from pallas_flash import precompute_rope
    B, Hq, Hkv, S, D = 4, 32, 8, 4096, 128
    g = torch.Generator(device="cuda").manual_seed(1)
    mk = lambda *shape: torch.randn(shape, generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    q, k, v = mk(B, Hq, S, D), mk(B, Hkv, S, D), mk(B, Hkv, S, D)
    cos, sin = precompute_rope(S, D, 10000.0, device="cuda")
    o = torch.empty_like(q)
    base = _lib.FwdArgs(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), None,
                        B, Hq, Hkv, S, S, D, S, 1, 1.0 / D ** 0.5, 1)
    ra = _lib.FwdRopeArgs(base, cos.data_ptr(), sin.data_ptr(), cos.data_ptr(), sin.data_ptr(), None, 0)
    ws = torch.empty(L.pf_attn_fwd_rope_workspace_size(ra), dtype=torch.uint8, device="cuda")
    ra.workspace, ra.workspace_bytes = ws.data_ptr(), ws.numel()
    # the plain forward at the same shape (no LSE, as the fused kernel), timed
    # in alternation: what the rotation costs
    o2 = torch.empty_like(q)
    plain = _lib.FwdArgs(q.data_ptr(), k.data_ptr(), v.data_ptr(), o2.data_ptr(), None,
                         B, Hq, Hkv, S, S, D, S, 1, 1.0 / D ** 0.5, 1)
    st = torch.cuda.current_stream().cuda_stream
    run = {"rope": lambda: ok(L.pf_attn_fwd_rope(ra, st), "pf_attn_fwd_rope"),
           "plain": lambda: ok(L.pf_attn_fwd(plain, st), "pf_attn_fwd")}
    for _ in range(max(3, warmup)):
        for f in run.values():
            f()
    ev = {k_: Events(2, iters) for k_ in run}
    for i in range(iters):
        for k_, f in run.items():
            ev[k_].mark(i, 0)
            f()
            ev[k_].mark(i, 1)
    torch.cuda.synchronize()
    ms = ev["rope"].median_ms(0, 1)
    plain_ms = ev["plain"].median_ms(0, 1)
    return ms, plain_ms, fwd_flops(B, Hq, D, causal_pairs(S)), {"q": q, "k": k, "v": v, "cos": cos, "sin": sin}


def _decode_args_and_ws(L, _lib, torch, args, size_fn):
    ws_bytes = size_fn(args)
    ws = torch.empty(max(int(ws_bytes), 256), dtype=torch.uint8, device="cuda")
    args.workspace = ws.data_ptr()
    args.workspace_bytes = ws.numel()
    return ws


def bench_decode(L, _lib, torch, iters, warmup):
    """Config 4 decode (pf_attn_decode) and, on the same cache, config 4's
    shape as one fused decode step (pf_attn_decode_step: RoPE of the new
    token's q/k at position 5999, cache-slot write, attention over the 6000
    live slots, position in device memory). The two are timed in alternation
    (same clocks, same cache); medians. Step bytes = the decode bytes + the
    new k/v rows read and written + the two table rows."""
    from pallas_flash import precompute_rope
    B, Hq, Hkv, cap, D, kv_len = 64, 32, 8, 8192, 128, 6000
    pos = kv_len - 1
    g = torch.Generator(device="cuda").manual_seed(2)
    q = torch.randn((B, Hq, 1, D), generator=g, device="cuda").to(torch.bfloat16)
    kc = torch.empty((B, Hkv, cap, D), dtype=torch.bfloat16, device="cuda")
    vc = torch.empty_like(kc)
    for t in (kc, vc):
        t[:, :, :kv_len].copy_(torch.randn((B, Hkv, kv_len, D), generator=g, device="cuda"))
        t[:, :, kv_len:].fill_(float("nan"))
    kn = torch.randn((B, Hkv, 1, D), generator=g, device="cuda").to(torch.bfloat16)
    vn = torch.randn((B, Hkv, 1, D), generator=g, device="cuda").to(torch.bfloat16)
    cos, sin = precompute_rope(cap, D, 10000.0, device="cuda")
    positions = torch.full((B,), pos, dtype=torch.int32, device="cuda")
    o, o_step = torch.empty_like(q), torch.empty_like(q)
    args = _lib.DecodeArgs(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), o.data_ptr(), B, Hq, Hkv, cap,
                           D, kv_len, 1.0 / D ** 0.5, 1, None, 0)
    ws = _decode_args_and_ws(L, _lib, torch, args, L.pf_attn_decode_workspace_size)
    sargs = _lib.DecodeStepArgs(q.data_ptr(), kn.data_ptr(), vn.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                o_step.data_ptr(), positions.data_ptr(), 1, cos.data_ptr(), sin.data_ptr(), cap,
                                B, Hq, Hkv, cap, D, 0, 1.0 / D ** 0.5, 1, None, 0)
    ws_step = _decode_args_and_ws(L, _lib, torch, sargs, L.pf_attn_decode_step_workspace_size)
    st = torch.cuda.current_stream().cuda_stream
    run = {"decode": lambda: ok(L.pf_attn_decode(args, st), "pf_attn_decode"),
           "step": lambda: ok(L.pf_attn_decode_step(sargs, st), "pf_attn_decode_step")}
    for _ in range(max(3, warmup)):
        for f in run.values():
            f()
    ev = {k: Events(2, iters) for k in run}
    for i in range(iters):
        for k, f in run.items():
            ev[k].mark(i, 0)
            f()
            ev[k].mark(i, 1)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all(), "decode output not finite"
    assert torch.isfinite(o_step.float()).all(), "decode step output not finite"
    nbytes = B * Hkv * kv_len * D * 2 * 2 + 2 * B * Hq * D * 2
    nbytes_step = nbytes + 2 * 2 * B * Hkv * D * 2 + 2 * D * 4
    del ws, ws_step
    return ({"decode": (ev["decode"].median_ms(0, 1), nbytes), "step": (ev["step"].median_ms(0, 1), nbytes_step)},
            {"q": q, "k": kc, "v": vc, "kv_len": kv_len})


def bench_d256(L, _lib, torch, steps, warmup, iters):
    """head_dim 256 (bf16): config 3's prefill shape (forward, dQ, dK/dV as
    one training step; mean per-kernel times over `steps` steps) and config
    4's decode shape (median over `iters` launches). Not a north-star
    configuration: the reference's callers all use head_dim 128."""
    B, Hq, Hkv, S, D = 2, 16, 4, 8192, 256
    g = torch.Generator(device="cuda").manual_seed(3)
    mk = lambda *shape: torch.randn(shape, generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    q, k, v, do = mk(B, Hq, S, D), mk(B, Hkv, S, D), mk(B, Hkv, S, D), mk(B, Hq, S, D)
    o = torch.empty_like(q)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device="cuda")
    delta = torch.empty_like(lse)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    scale = 1.0 / D ** 0.5
    fa = _lib.FwdArgs(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                      B, Hq, Hkv, S, S, D, S, 1, scale, 1)
    ba = _lib.BwdArgs(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
                      lse.data_ptr(), delta.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                      B, Hq, Hkv, S, S, D, S, 1, scale, 1)
    st = torch.cuda.current_stream().cuda_stream
    calls = [lambda: ok(L.pf_attn_fwd(fa, st), "pf_attn_fwd"),
             lambda: ok(L.pf_attn_bwd_dq(ba, st), "pf_attn_bwd_dq"),
             lambda: ok(L.pf_attn_bwd_dkv(ba, st), "pf_attn_bwd_dkv")]
    for _ in range(warmup):
        for c in calls:
            c()
    ev = Events(4, steps)
    for i in range(steps):
        for j, c in enumerate(calls):
            ev.mark(i, j)
            c()
        ev.mark(i, 3)
    torch.cuda.synchronize()
    assert torch.isfinite(dk.float()).all() and torch.isfinite(dq.float()).all(), "head_dim 256 gradients"
    F = fwd_flops(B, Hq, D, causal_pairs(S))
    prefill = {"fwd_ms": ev.mean_ms(0, 1), "dq_ms": ev.mean_ms(1, 2), "dkv_ms": ev.mean_ms(2, 3),
               "step_ms": ev.mean_ms(0, 3), "F": F}
    del q, k, v, do, o, lse, delta, dq, dk, dv
    # decode: config 4's shape at head_dim 256 (generic split-KV kernel)
    B, Hq, Hkv, cap, kv_len = 64, 32, 8, 8192, 6000
    qd = torch.randn((B, Hq, 1, D), generator=g, device="cuda").to(torch.bfloat16)
    kc = torch.empty((B, Hkv, cap, D), dtype=torch.bfloat16, device="cuda")
    vc = torch.empty_like(kc)
    for t in (kc, vc):
        t[:, :, :kv_len].copy_(torch.randn((B, Hkv, kv_len, D), generator=g, device="cuda"))
        t[:, :, kv_len:].fill_(float("nan"))
    od = torch.empty_like(qd)
    args = _lib.DecodeArgs(qd.data_ptr(), kc.data_ptr(), vc.data_ptr(), od.data_ptr(), B, Hq, Hkv, cap,
                           D, kv_len, 1.0 / D ** 0.5, 1, None, 0)
    ws = _decode_args_and_ws(L, _lib, torch, args, L.pf_attn_decode_workspace_size)
    for _ in range(max(3, warmup)):
        ok(L.pf_attn_decode(args, st), "pf_attn_decode")
    dev_ = Events(2, iters)
    for i in range(iters):
        dev_.mark(i, 0)
        ok(L.pf_attn_decode(args, st), "pf_attn_decode")
        dev_.mark(i, 1)
    torch.cuda.synchronize()
    assert torch.isfinite(od.float()).all(), "head_dim 256 decode output"
    nbytes = B * Hkv * kv_len * D * 2 * 2 + 2 * B * Hq * D * 2
    del ws, kc, vc
    return prefill, (dev_.median_ms(0, 1), nbytes)


def cfg5_layout():
    """Config 5's sequences and pool: lengths U[512, 8192] and the page
    permutation from np.random.default_rng(0), pages dealt out in order, table
    [128, 128] padded with -1; also the mask of pages some sequence uses."""
    B, page, npages, pps = 128, 64, 16384, 128
    rng = np.random.default_rng(0)
    lens = rng.integers(512, 8193, B)
    perm = rng.permutation(npages)
    table = np.full((B, pps), -1, np.int32)
    used = np.zeros(npages, bool)
    cur = 0
    for b in range(B):
        n = -(-int(lens[b]) // page)
        table[b, :n] = perm[cur:cur + n]
        used[perm[cur:cur + n]] = True
        cur += n
    return lens, table, used


def bench_paged(L, _lib, torch, iters, warmup):
    B, Hq, Hkv, D, page, npages, pps = 128, 32, 8, 128, 64, 16384, 128
    lens, table, used = cfg5_layout()
    g = torch.Generator(device="cuda").manual_seed(3)
    q = torch.randn((B, Hq, 1, D), generator=g, device="cuda").to(torch.bfloat16)
    kp = torch.randn((npages, Hkv, page, D), generator=g, device="cuda").to(torch.bfloat16)
    vp = torch.randn((npages, Hkv, page, D), generator=g, device="cuda").to(torch.bfloat16)
    unused = torch.as_tensor(np.nonzero(~used)[0], device="cuda")
    for t in (kp, vp):
        t[unused] = float("nan")
        for b in range(B):  # beyond-length tail of each sequence's last page
            n = -(-int(lens[b]) // page)
            tail = int(lens[b]) - (n - 1) * page
            if tail < page:
                t[int(table[b, n - 1]), :, tail:] = float("nan")
    tt = torch.as_tensor(table, device="cuda")
    tl = torch.as_tensor(lens.astype(np.int32), device="cuda")
    o = torch.empty_like(q)
    args = _lib.PagedArgs(q.data_ptr(), kp.data_ptr(), vp.data_ptr(), tt.data_ptr(), tl.data_ptr(),
                          o.data_ptr(), B, Hq, Hkv, npages, page, D, pps, 1.0 / D ** 0.5, 1, None, 0)
    ws = _decode_args_and_ws(L, _lib, torch, args, L.pf_paged_attn_workspace_size)
    st = torch.cuda.current_stream().cuda_stream
    for _ in range(max(3, warmup)):
        ok(L.pf_paged_attn(args, st), "pf_paged_attn")
    ev = Events(2, iters)
    for i in range(iters):
        ev.mark(i, 0)
        ok(L.pf_paged_attn(args, st), "pf_paged_attn")
        ev.mark(i, 1)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all(), "paged output not finite"
    npg = -(-lens // page)
    nbytes = int(lens.sum()) * Hkv * D * 2 * 2 + 2 * B * Hq * D * 2 + 4 * int(npg.sum()) + 4 * B
    del ws
    return ev.median_ms(0, 1), nbytes, {"q": q, "k": kp, "v": vp, "table": table, "lens": lens}


def bench_aux(L, _lib, torch, iters, warmup):
    """The rows around the hot path, each at a configuration's own shape:
    the contiguous cache write (model.py _cache_write :257-262 as prefill and
    decode steps call it; the ring slot scatter :447-448, :487) at config 4,
    the paged page-write (paged.py:205-223, batched) into config 5's pool,
    and the RoPE-aware VJP at config 2 (the inverse rotation pf_rope applies
    to dQ and dK, and the whole RoPE training step beside the plain one).
    Median ms per launch over back-to-back launches; bytes = rows read once
    and written once (+ the tables for the rotation)."""
    from pallas_flash import precompute_rope
    st = torch.cuda.current_stream().cuda_stream
    g = torch.Generator(device="cuda").manual_seed(4)
    mk = lambda *shape: torch.randn(shape, generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)

    def timed(fns):
        for _ in range(max(3, warmup)):
            for f in fns.values():
                f()
        ev = {k_: Events(2, iters) for k_ in fns}
        for i in range(iters):
            for k_, f in fns.items():
                ev[k_].mark(i, 0)
                f()
                ev[k_].mark(i, 1)
        torch.cuda.synchronize()
        return {k_: e.median_ms(0, 1) for k_, e in ev.items()}

    res, cpu_in = {}, {}
    # contiguous cache at config 4's shape: a 6000-token prefill write, then
    # a one-token ring step at position 15000 (slot 15000 % 8192 = 6808, past
    # the prefill's slots)
    B, Hkv, C, D, Lp = 64, 8, 8192, 128, 6000
    kn, vn = mk(B, Hkv, Lp, D), mk(B, Hkv, Lp, D)
    kc = torch.zeros((B, Hkv, C, D), dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    pos0 = torch.zeros(B, dtype=torch.int32, device="cuda")
    k1, v1 = mk(B, Hkv, 1, D), mk(B, Hkv, 1, D)
    posr = torch.full((B,), 15000, dtype=torch.int32, device="cuda")
    wa = _lib.KvWriteArgs(kn.data_ptr(), vn.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos0.data_ptr(), 1,
                          B, Hkv, Lp, C, D, 0, 1)
    wr = _lib.KvWriteArgs(k1.data_ptr(), v1.data_ptr(), kc.data_ptr(), vc.data_ptr(), posr.data_ptr(), 1,
                          B, Hkv, 1, C, D, 1, 1)
    t = timed({"prefill": lambda: ok(L.pf_kv_cache_write(wa, st), "pf_kv_cache_write"),
               "ring": lambda: ok(L.pf_kv_cache_write(wr, st), "pf_kv_cache_write ring")})
    assert torch.equal(kc[:, :, :Lp], kn) and torch.equal(vc[:, :, :Lp], vn), "cache write"
    assert torch.equal(kc[:, :, 15000 % C], k1[:, :, 0]) and torch.equal(vc[:, :, 15000 % C], v1[:, :, 0])
    res["kv_write_prefill"] = (t["prefill"], 2 * 2 * B * Hkv * Lp * D * 2)
    res["kv_write_ring_step"] = (t["ring"], 2 * 2 * B * Hkv * D * 2)
    cpu_in["kv"] = {"rows": kn[:8], "C": C}
    del kn, vn, kc, vc, k1, v1

    # paged: config 5's pool and table; a 512-token prefill chunk per
    # sequence at position 0, then one token per sequence at its last
    # position (lens - 1, always inside a mapped page)
    lens, table, _ = cfg5_layout()
    B5, npages, page, pps, Lc = 128, 16384, 64, 128, 512
    kp = torch.zeros((npages, Hkv, page, D), dtype=torch.bfloat16, device="cuda")
    vp = torch.zeros_like(kp)
    tt = torch.as_tensor(table, device="cuda")
    kn, vn = mk(B5, Hkv, Lc, D), mk(B5, Hkv, Lc, D)
    k1, v1 = mk(B5, Hkv, 1, D), mk(B5, Hkv, 1, D)
    p0 = torch.zeros(B5, dtype=torch.int32, device="cuda")
    plast = torch.as_tensor((lens - 1).astype(np.int32), device="cuda")
    pa = _lib.PagedWriteArgs(kn.data_ptr(), vn.data_ptr(), kp.data_ptr(), vp.data_ptr(), tt.data_ptr(),
                             p0.data_ptr(), 1, B5, Hkv, Lc, npages, page, D, pps, 1)
    ps = _lib.PagedWriteArgs(k1.data_ptr(), v1.data_ptr(), kp.data_ptr(), vp.data_ptr(), tt.data_ptr(),
                             plast.data_ptr(), 1, B5, Hkv, 1, npages, page, D, pps, 1)
    t = timed({"prefill": lambda: ok(L.pf_paged_cache_write(pa, st), "pf_paged_cache_write"),
               "step": lambda: ok(L.pf_paged_cache_write(ps, st), "pf_paged_cache_write step")})
    for b in (0, B5 - 1):
        pg0 = int(table[b, 0])
        assert torch.equal(kp[pg0], kn[b, :, :page]) and torch.equal(vp[pg0], vn[b, :, :page]), "paged write"
        last = int(lens[b]) - 1
        pgl = int(table[b, last // page])
        assert torch.equal(kp[pgl, :, last % page], k1[b, :, 0]), "paged step write"
    res["paged_write_prefill"] = (t["prefill"], 2 * 2 * B5 * Hkv * Lc * D * 2)
    res["paged_write_step"] = (t["step"], 2 * 2 * B5 * Hkv * D * 2)
    cpu_in["paged"] = {"rows": kn[:64], "page": page}
    del kp, vp, kn, vn, k1, v1

    # RoPE-aware VJP at config 2's shape
    B2, Hq2, Hkv2, S2 = 4, 32, 8, 4096
    cos, sin = precompute_rope(S2, D, 10000.0, device="cuda")
    q, k, v, do = mk(B2, Hq2, S2, D), mk(B2, Hkv2, S2, D), mk(B2, Hkv2, S2, D), mk(B2, Hq2, S2, D)
    buf = {n: torch.empty_like(t_) for n, t_ in (("qr", q), ("kr", k), ("o", q), ("dqr", q), ("dkr", k),
                                                  ("dv", v), ("dq", q), ("dk", k))}
    lse = torch.empty((B2, Hq2, S2), dtype=torch.float32, device="cuda")
    delta = torch.empty_like(lse)
    P = lambda t_: t_.data_ptr()
    rope = lambda x, y, H, inv: _lib.RopeArgs(P(x), P(y), P(cos), P(sin), B2, H, S2, D, S2, inv, 1)
    r_q, r_k = rope(q, buf["qr"], Hq2, 0), rope(k, buf["kr"], Hkv2, 0)
    r_dq, r_dk = rope(buf["dqr"], buf["dq"], Hq2, 1), rope(buf["dkr"], buf["dk"], Hkv2, 1)
    sc = 1.0 / D ** 0.5

    def attn_args(qq, kk):
        fa = _lib.FwdArgs(P(qq), P(kk), P(v), P(buf["o"]), P(lse), B2, Hq2, Hkv2, S2, S2, D, S2, 1, sc, 1)
        ba = _lib.BwdArgs(P(qq), P(kk), P(v), P(buf["o"]), P(do), P(lse), P(delta), P(buf["dqr"]), P(buf["dkr"]),
                          P(buf["dv"]), B2, Hq2, Hkv2, S2, S2, D, S2, 1, sc, 1)
        return fa, ba

    fa_r, ba_r = attn_args(buf["qr"], buf["kr"])
    fa_p, ba_p = attn_args(q, k)

    def rope_step():
        ok(L.pf_rope(r_q, st), "pf_rope q")
        ok(L.pf_rope(r_k, st), "pf_rope k")
        ok(L.pf_attn_fwd(fa_r, st), "pf_attn_fwd")
        ok(L.pf_attn_bwd(ba_r, st), "pf_attn_bwd")
        ok(L.pf_rope(r_dq, st), "pf_rope dq (inverse)")
        ok(L.pf_rope(r_dk, st), "pf_rope dk (inverse)")

    def plain_step():
        ok(L.pf_attn_fwd(fa_p, st), "pf_attn_fwd")
        ok(L.pf_attn_bwd(ba_p, st), "pf_attn_bwd")

    t = timed({"vjp": lambda: ok(L.pf_rope(r_dq, st), "pf_rope dq (inverse)"),
               "rope_step": rope_step, "plain_step": plain_step})
    res["rope_vjp"] = (t["vjp"], 2 * q.numel() * 2 + 2 * S2 * D * 4)
    res["rope_train_step_ms"] = t["rope_step"]
    res["plain_train_step_ms"] = t["plain_step"]
    cpu_in["rope"] = {"g": buf["dqr"][0:1], "cos": cos, "sin": sin}
    return res, cpu_in


def cpu_baseline_aux(a):
    """The aux rows on the CPU, each the oracle on a bounded sample: the
    cache write (cache_write_ref, 2 of config 4's sequences, 6000 rows into a
    zeroed 8192-slot cache, K only), the page write (paged_write_ref, 8 of
    config 5's sequences, 512 rows each into a zeroed pool copy of 8192 pages)
    and the inverse rotation (apply_rope_vjp_ref in float32, batch 0, 8 heads).
    GB/s with the GPU's byte credit for the same rows (host copies untimed)."""
    from oracle import apply_rope_vjp_ref, cache_write_ref, paged_write_ref
    cores, blas = _host_cores()
    out = {}
    rows = a["kv"]["rows"].float().cpu().numpy()
    B, H, Lp, D = rows.shape
    cache = np.zeros((B, H, a["kv"]["C"], D), np.float32)
    t0 = time.perf_counter()
    cache_write_ref(cache, rows, 0)
    dt = time.perf_counter() - t0
    out["kv_write"] = {"value": 2 * B * H * Lp * D * 2 / dt / 1e9, "unit": "GB/s", "cores": cores,
                       "blas_threads": blas, "kind": "port",
                       "sample": f"numpy oracle (cache_write_ref) on {B} config-4 sequences x {H} kv heads, "
                                 f"{Lp} rows at position 0 (K only), {dt:.2f} s"}
    rows = a["paged"]["rows"].float().cpu().numpy()
    B, H, Lc, D = rows.shape
    page = a["paged"]["page"]
    npg = Lc // page  # pages per sequence the rows fill
    # a compact pool holding just the sample's pages (sequence b's page j at
    # b * npg + j): the oracle copies the whole pool, whose size is not work
    pool = np.zeros((B * npg, H, page, D), np.float32)
    table = np.arange(B * npg, dtype=np.int32).reshape(B, npg)
    t0 = time.perf_counter()
    paged_write_ref(pool, rows, table, np.zeros(B, np.int64))
    dt = time.perf_counter() - t0
    out["paged_write"] = {"value": 2 * B * H * Lc * D * 2 / dt / 1e9, "unit": "GB/s", "cores": cores,
                          "blas_threads": blas, "kind": "port",
                          "sample": f"numpy oracle (paged_write_ref) on {B} config-5 sequences x {H} kv heads, "
                                    f"{Lc} rows at position 0 into a pool of their {B * npg} pages (K only), "
                                    f"{dt:.2f} s"}
    gq = a["rope"]["g"].float().cpu().numpy()
    cos, sin = a["rope"]["cos"].cpu().numpy(), a["rope"]["sin"].cpu().numpy()
    t0 = time.perf_counter()
    apply_rope_vjp_ref(gq, cos, sin, dtype=np.float32)
    dt = time.perf_counter() - t0
    out["rope_vjp"] = {"value": 2 * gq.size * 2 / dt / 1e9, "unit": "GB/s", "cores": cores,
                       "blas_threads": blas, "kind": "port",
                       "sample": f"numpy float32 oracle (apply_rope_vjp_ref) on config 2's dQ, batch 0, "
                                 f"{gq.shape[1]} of 32 heads, {dt:.2f} s"}
    return out


def _probe_lib():
    import ctypes
    probe = ctypes.CDLL(os.path.join(PKG_DIR, "pallas_flash", "libpf_bench_probe.so"))
    probe.pf_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_void_p]
    probe.pf_probe_read.restype = ctypes.c_int
    probe.pf_probe_mfma.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    probe.pf_probe_mfma.restype = ctypes.c_int
    return probe


READ_FORMS = {0: "16-byte non-temporal register loads", 1: "16-byte temporal register loads",
              2: "direct global->LDS loads (buffer_load_dwordx4 ... lds)",
              3: "non-temporal direct global->LDS loads (the streaming decode's form)"}


def _median_launch_ms(torch, call, iters, warm=3):
    for _ in range(warm):
        call()
    ev = Events(2, iters)
    for i in range(iters):
        ev.mark(i, 0)
        call()
        ev.mark(i, 1)
    torch.cuda.synchronize()
    return ev.median_ms(0, 1)


def bench_read_ceiling(torch, iters):
    """The practical HBM read ceiling: a plain streaming read of a 2 GiB
    buffer (grid-stride over 2048-16384 workgroups of 256 threads, 4 or 8
    loads in flight per thread or wave) in four load forms: non-temporal and
    temporal 16-byte register loads and direct global->LDS loads. Returns
    (best GB/s, its description, {form: best GB/s})."""
    probe = _probe_lib()
    nbytes = 2 << 30
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    buf.fill_(1)
    sink = torch.zeros(16384, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    best, per_form = None, {}
    for form, what in READ_FORMS.items():
        for unroll in (4, 8):
            for blocks in (2048, 4096, 8192, 16384):
                call = lambda: ok(probe.pf_probe_read(buf.data_ptr(), nbytes, sink.data_ptr(), blocks, unroll,
                                                      form, st), "probe read")
                gbs = nbytes / (_median_launch_ms(torch, call, iters) * 1e-3) / 1e9
                per_form[form] = max(per_form.get(form, 0.0), gbs)
                if best is None or gbs > best[0]:
                    best = (gbs, f"{what}, {blocks} workgroups x 256 threads, {unroll} in flight, 2 GiB buffer, "
                                 f"median of {iters}")
    del buf, sink
    return best[0], best[1], {READ_FORMS[f].split(" (")[0]: round(g, 1) for f, g in per_form.items()}


def bench_mfma_ceiling(torch, iters):
    """The same-run matrix-core ceiling: back-to-back 32x32x16 bf16 MFMAs on
    register operands (four independent accumulators per wave, no memory
    traffic) over 256-2048 workgroups of 256 threads; the best launch shape's
    median TFLOP/s. Reads a box's sustained MFMA rate (its clock under a full
    MFMA load included), against which the prefill kernels' rates are also
    stated."""
    probe = _probe_lib()
    it = 8192
    best = None
    for blocks in (256, 512, 1024, 2048):
        out = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
        st = torch.cuda.current_stream().cuda_stream
        call = lambda: ok(probe.pf_probe_mfma(out.data_ptr(), blocks, it, st), "probe mfma")
        ms = _median_launch_ms(torch, call, iters)
        tflops = blocks * 4 * it * 8 * 32768 / (ms * 1e-3) / 1e12
        if best is None or tflops > best[0]:
            best = (tflops, f"{blocks} workgroups x 4 waves, {8 * it} MFMAs per wave, median of {iters}")
        del out
    return best


def bench_copy(torch, iters):
    """A plain device-to-device copy of 1 GiB (torch's copy kernel): the
    calibration workload for the HBM byte counters (its FETCH_SIZE and
    WRITE_SIZE per dispatch are each 1 GiB of algorithmic traffic)."""
    nbytes = 1 << 30
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    ev = Events(2, iters)
    for i in range(iters):
        ev.mark(i, 0)
        dst.copy_(src)
        ev.mark(i, 1)
    torch.cuda.synchronize()
    return ev.mean_ms(0, 1), nbytes


def _host_cores():
    """Host cores this process may run on, and numpy's BLAS thread count."""
    cores = len(os.sched_getaffinity(0))
    try:
        from threadpoolctl import threadpool_info
        blas = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:  # pragma: no cover
        blas = 1
    return cores, int(blas)


def cpu_baseline(c3, n_kv=2, reps=3):
    """The float32 numpy restatement of the reference algorithm (oracle/),
    forward + backward on a bounded sample of config 3: batch 0, KV heads
    [0, n_kv) with their 4 query heads each (8 of 32 (b, h) heads), full
    S=8192 causal. One untimed warm-up pass, then the median of `reps` timed
    passes. Credited FLOPs of the sample (3.5 forwards, as on the GPU) / wall
    time; the oracle's backward recomputes the attention to get P and the LSE,
    so the CPU executes 9 S-sized matmuls per pass for the 7 credited."""
    import torch
    from oracle import attention_bwd_ref, attention_ref
    cores, blas = _host_cores()
    S, D = c3["S"], c3["D"]
    h = c3["host"]
    g = c3["Hq"] // c3["Hkv"]
    f32 = lambda t: t.float().cpu().numpy()
    q = f32(h["q"][0:1, :n_kv * g])
    k = f32(h["k"][0:1, :n_kv])
    v = f32(h["v"][0:1, :n_kv])
    do = f32(h["do"][0:1, :n_kv * g])
    if torch.cuda.is_available():
        torch.cuda.synchronize()

    def one():
        t0 = time.perf_counter()
        o, _ = attention_ref(q, k, v, causal=True, dtype=np.float32)
        attention_bwd_ref(q, k, v, do, causal=True, o=o, dtype=np.float32)
        return time.perf_counter() - t0

    one()  # warm-up: first-touch of the sample's buffers, BLAS thread start-up
    times = [one() for _ in range(reps)]
    dt = float(np.median(times))
    flops = 3.5 * fwd_flops(1, q.shape[1], D, causal_pairs(S))
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": cores, "blas_threads": blas,
            "kind": "port",
            "sample": f"numpy float32 restatement (oracle/attention.py) of reference.py + its "
                      f"backward, fwd+bwd of config 3 batch 0, kv heads 0-{n_kv - 1} ({q.shape[1]} of 32 (b, h) "
                      f"heads) at S={S}: median of {reps} passes after one warm-up "
                      f"({', '.join(f'{t:.2f}' for t in times)} s); the oracle's backward recomputes "
                      f"P and the LSE (9 S-sized matmuls per pass, 7 credited); matmuls on {blas} BLAS "
                      f"threads, elementwise ops on 1 thread, {cores} host cores available"}


def cpu_baseline_rope(r, n_kv=4):
    """Config 2 on the CPU: the oracle's fused-RoPE restatement (rotation in
    float32, then naive attention) for batch 0, KV heads [0, n_kv) (4 query
    heads each, of 128 (b, h) in all) at S=4096, causal. Credited FLOPs of
    the sample / wall time (the oracle calls only; host copies untimed)."""
    from oracle import rope_attention_ref
    cores, blas = _host_cores()
    f32 = lambda t: t.float().cpu().numpy()
    cos, sin = f32(r["cos"]), f32(r["sin"])
    g = r["q"].shape[1] // r["k"].shape[1]
    S, D = r["q"].shape[2], r["q"].shape[3]
    dt = 0.0
    for h in range(n_kv):
        q = f32(r["q"][0:1, h * g:(h + 1) * g])
        k, v = f32(r["k"][0:1, h:h + 1]), f32(r["v"][0:1, h:h + 1])
        t0 = time.perf_counter()
        rope_attention_ref(q, k, v, cos, sin, causal=True, dtype=np.float32)
        dt += time.perf_counter() - t0
    flops = fwd_flops(1, n_kv * g, D, causal_pairs(S))
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": cores, "blas_threads": blas,
            "kind": "port",
            "sample": f"numpy float32 oracle (rope_attention_ref) on config 2 batch 0, kv heads "
                      f"0-{n_kv - 1} ({n_kv * g} of 128 query heads) at S={S}, {dt:.2f} s"}


def cpu_baseline_decode(d):
    """Config 4 on the CPU, per sequence on the sliced prefix (the reference's
    decode oracle, tests/test_decode.py:33): the float32 oracle over every
    sequence's [0, kv_len) slots. Algorithmic (bf16) bytes / time (the oracle
    calls only; host copies untimed)."""
    from oracle import decode_ref
    cores, blas = _host_cores()
    L = d["kv_len"]
    f32 = lambda t: t.float().cpu().numpy()
    B, Hq, _, D = d["q"].shape
    Hkv = d["k"].shape[1]
    dt = 0.0
    for b in range(B):
        q, k, v = f32(d["q"][b:b + 1]), f32(d["k"][b:b + 1, :, :L]), f32(d["v"][b:b + 1, :, :L])
        t0 = time.perf_counter()
        decode_ref(q, k, v, L, dtype=np.float32)
        dt += time.perf_counter() - t0
    nbytes = B * (Hkv * L * D * 2 * 2 + 2 * Hq * D * 2)
    return {"value": nbytes / dt / 1e9, "unit": "GB/s", "cores": cores, "blas_threads": blas,
            "kind": "port",
            "sample": f"numpy float32 oracle (decode_ref) per sequence on the sliced prefix, all "
                      f"{B} config-4 sequences (kv_len {L}), {dt:.2f} s; bytes credited as the "
                      f"GPU's (bf16 K/V once + q + o)"}


def cpu_baseline_paged(pg):
    """Config 5 on the CPU, per sequence on the gathered pages (the
    reference's paged oracle, tests/test_paged.py:25-28): the float32 oracle
    (paged_ref: gather, then attend) over every sequence. Algorithmic (bf16)
    bytes / time (the oracle calls only; host copies untimed)."""
    import torch
    from oracle import paged_ref
    cores, blas = _host_cores()
    table, lens = pg["table"], pg["lens"]
    page = pg["k"].shape[2]
    B, Hq, _, D = pg["q"].shape
    Hkv = pg["k"].shape[1]
    f32 = lambda t: t.float().cpu().numpy()
    dt = 0.0
    for b in range(B):
        n = -(-int(lens[b]) // page)
        sel = torch.as_tensor(table[b, :n].astype(np.int64), device=pg["k"].device)
        q, kp, vp = f32(pg["q"][b:b + 1]), f32(pg["k"][sel]), f32(pg["v"][sel])
        sub = np.arange(n, dtype=np.int32)[None]  # the sequence's pages, gathered in order
        t0 = time.perf_counter()
        paged_ref(q, kp, vp, sub, lens[b:b + 1], dtype=np.float32)
        dt += time.perf_counter() - t0
    n_pages = int(sum(-(-int(x) // page) for x in lens))
    nbytes = int(lens.sum()) * Hkv * D * 2 * 2 + 2 * B * Hq * D * 2 + 4 * n_pages + 4 * B
    return {"value": nbytes / dt / 1e9, "unit": "GB/s", "cores": cores, "blas_threads": blas,
            "kind": "port",
            "sample": f"numpy float32 oracle (paged_ref) per sequence on its gathered pages, all "
                      f"{B} config-5 sequences ({int(lens.sum())} tokens), {dt:.2f} s; bytes "
                      f"credited as the GPU's"}


def load_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (profiles/traffic.json: FETCH_SIZE and WRITE_SIZE per dispatch,
    each scaled by what the counter reads for a 1 GiB copy), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            recs = json.load(f).get(workload, {})
    except (OSError, ValueError):
        return None
    # keys are kernel names with their template arguments ("name<bf16, 128, ...>");
    # the workload runs one instantiation of each kernel
    hits = [r for k, r in recs.items() if k == kernel or k.startswith(kernel + "<")]
    return int(hits[0]["bytes"]) if len(hits) == 1 else None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", choices=["all", "cfg3", "rope", "decode", "paged", "aux", "stream", "mfma", "copy",
                                       "d256"], default="all")
    ap.add_argument("--skip-cpu", action="store_true", help="omit the CPU baseline leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for "
              f"--gpus {args.gpus}). Prefill would shard over (batch, KV-head group) units with no "
              f"exchange, decode and paged decode over sequences.", file=sys.stderr)
        sys.exit(2)

    import torch
    from pallas_flash import _lib
    L = _lib.lib()
    torch.cuda.set_device(0)
    iters = max(args.steps, 5)
    sec = {}

    c3 = None
    if args.only in ("all", "cfg3"):
        log("cfg3 fwd+bwd ...")
        c3 = bench_cfg3(L, _lib, torch, args.steps, args.warmup)
        sec["fwd_tflops"] = c3["F"] / (c3["kern_ms"]["pf_attn_fwd_kernel"] * 1e-3) / 1e12
        sec["kernel_ms"] = {k: round(v, 4) for k, v in c3["kern_ms"].items()}
        sec["fwd_loop_ms"] = c3["fwd_loop_ms"]
        sec["fwd_loop_tflops"] = c3["F"] / (c3["fwd_loop_ms"] * 1e-3) / 1e12
    cpu_sec = {}
    if args.only in ("all", "rope"):
        log("cfg2 rope ...")
        ms, plain_ms, F, rin = bench_rope(L, _lib, torch, iters, args.warmup)
        sec["rope_tflops"] = F / (ms * 1e-3) / 1e12
        sec["rope_ms"] = ms
        sec["fwd_cfg2_shape_ms"] = plain_ms
        sec["rope_over_plain_fwd"] = ms / plain_ms
        if not args.skip_cpu:
            log("cpu baseline cfg2 ...")
            cpu_sec["rope"] = cpu_baseline_rope(rin)
        del rin
    if args.only in ("all", "decode"):
        log("cfg4 decode and decode step ...")
        res, din = bench_decode(L, _lib, torch, iters, args.warmup)
        ms, nb = res["decode"]
        sec["decode_gbs"] = nb / (ms * 1e-3) / 1e9
        sec["decode_ms"] = ms
        ms, nb = res["step"]
        sec["decode_step_gbs"] = nb / (ms * 1e-3) / 1e9
        sec["decode_step_ms"] = ms
        if not args.skip_cpu:
            log("cpu baseline cfg4 ...")
            cpu_sec["decode"] = cpu_baseline_decode(din)
        del din
    if args.only in ("all", "paged"):
        log("cfg5 paged ...")
        ms, nb, pin = bench_paged(L, _lib, torch, iters, args.warmup)
        sec["paged_gbs"] = nb / (ms * 1e-3) / 1e9
        sec["paged_ms"] = ms
        if not args.skip_cpu:
            log("cpu baseline cfg5 ...")
            cpu_sec["paged"] = cpu_baseline_paged(pin)
        del pin

    if args.only in ("all", "aux"):
        log("cache writes and RoPE VJP ...")
        res, ain = bench_aux(L, _lib, torch, iters, args.warmup)
        for k_ in ("kv_write_prefill", "paged_write_prefill", "rope_vjp"):
            ms, nb = res[k_]
            sec[f"{k_}_gbs"] = nb / (ms * 1e-3) / 1e9
            sec[f"{k_}_ms"] = ms
            sec[f"{k_}_frac_hbm"] = sec[f"{k_}_gbs"] / PEAK_HBM_GBS
        for k_ in ("kv_write_ring_step", "paged_write_step"):
            sec[f"{k_}_us"] = res[k_][0] * 1e3
        sec["rope_train_step_ms"] = res["rope_train_step_ms"]
        sec["plain_train_step_cfg2_shape_ms"] = res["plain_train_step_ms"]
        sec["rope_train_over_plain"] = res["rope_train_step_ms"] / res["plain_train_step_ms"]
        if not args.skip_cpu:
            log("cpu baselines aux ...")
            cpu_sec.update(cpu_baseline_aux(ain))
        del ain

    if args.only in ("all", "d256"):
        log("head_dim 256 prefill and decode ...")
        pre, (ms, nb) = bench_d256(L, _lib, torch, args.steps, args.warmup, iters)
        sec["d256_kernel_ms"] = {k: round(pre[k], 4) for k in ("fwd_ms", "dq_ms", "dkv_ms")}
        sec["d256_fwd_tflops"] = pre["F"] / (pre["fwd_ms"] * 1e-3) / 1e12
        sec["d256_step_tflops"] = 3.5 * pre["F"] / (pre["step_ms"] * 1e-3) / 1e12
        sec["d256_decode_gbs"] = nb / (ms * 1e-3) / 1e9
        sec["d256_config"] = ("bf16 head_dim 256: prefill at config 3's shape (B=2 Hq=16 Hkv=4 S=8192 causal), "
                              "decode at config 4's (B=64 Hq=32 Hkv=8 cache 8192, kv_len 6000)")

    if args.only in ("all", "stream"):
        log("hbm read ceiling ...")
        gbs, how, forms = bench_read_ceiling(torch, iters)
        sec["hbm_read_ceiling_gbs"] = gbs
        sec["hbm_read_ceiling_config"] = how
        sec["hbm_read_by_form_gbs"] = forms

    if args.only in ("all", "mfma"):
        log("mfma stream ceiling ...")
        tf, how = bench_mfma_ceiling(torch, iters)
        sec["mfma_stream_ceiling_tflops"] = tf
        sec["mfma_stream_ceiling_config"] = how

    if args.only == "copy":
        log("copy calibration ...")
        ms, nb = bench_copy(torch, iters)
        sec["copy_gbs"] = 2 * nb / (ms * 1e-3) / 1e9
        sec["copy_ms"] = ms

    line = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic N(0,1) (torch CUDA generator, seed 0)"}
    if c3 is not None:
        step_ms = c3["wall_ms"]
        line.update({
            "value": round(3.5 * c3["F"] / (step_ms * 1e-3) / 1e12, 2),
            "unit": "TFLOP/s",
            "ms_per_step": round(step_ms, 4),
            "config": {"workload": "config 3: flash_attention fwd+bwd, bf16, causal GQA, B=2 Hq=16 "
                                   "Hkv=4 S=8192 D=128 (dK/dV group-summed, LSE saved)",
                       "batch": 2, "seq_len": 8192, "head_dim": 128, "num_heads": 16,
                       "num_kv_heads": 4, "causal": True},
        })
        dom = max(c3["credit"], key=lambda k: c3["kern_ms"][k])
        achieved = c3["credit"][dom] / (c3["kern_ms"][dom] * 1e-3) / 1e12
        line["roofline"] = {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 2),
                            "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                            "traffic": load_traffic(dom, "cfg3"),
                            "avg_launch_ms": round(c3["kern_ms"][dom], 4)}
        if not args.skip_cpu:
            log("cpu baseline ...")
            line["cpu_baseline"] = cpu_baseline(c3)
    line["secondary"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in sec.items()}
    if "decode_gbs" in sec:
        line["secondary"]["decode_frac_hbm"] = round(sec["decode_gbs"] / PEAK_HBM_GBS, 4)
    if "decode_step_gbs" in sec:
        line["secondary"]["decode_step_frac_hbm"] = round(sec["decode_step_gbs"] / PEAK_HBM_GBS, 4)
    if "paged_gbs" in sec:
        line["secondary"]["paged_frac_hbm"] = round(sec["paged_gbs"] / PEAK_HBM_GBS, 4)
    if "hbm_read_ceiling_gbs" in sec:
        for k in ("decode", "decode_step", "paged"):
            if f"{k}_gbs" in sec:
                line["secondary"][f"{k}_frac_read_ceiling"] = round(sec[f"{k}_gbs"] / sec["hbm_read_ceiling_gbs"], 4)
    ceil = sec.get("mfma_stream_ceiling_tflops")
    rates = {}
    if "fwd_tflops" in sec:
        rates["fwd"] = sec["fwd_tflops"]
    if "fwd_loop_tflops" in sec:
        rates["fwd_loop"] = sec["fwd_loop_tflops"]
    if c3 is not None:
        for short, kern in (("dq", "pf_attn_bwd_dq_kernel"), ("dkv", "pf_attn_bwd_dkv_kernel")):
            rates[short] = c3["credit"][kern] / (c3["kern_ms"][kern] * 1e-3) / 1e12
        line["secondary"]["dq_tflops"] = round(rates["dq"], 3)
        line["secondary"]["dkv_tflops"] = round(rates["dkv"], 3)
    if "rope_tflops" in sec:
        rates["rope"] = sec["rope_tflops"]
    for k, r in rates.items():
        line["secondary"][f"{k}_frac_mfma"] = round(r / PEAK_BF16_TFLOPS, 4)
        if ceil:
            line["secondary"][f"{k}_frac_mfma_ceiling"] = round(r / ceil, 4)
    if cpu_sec:
        line["secondary"]["cpu_baselines"] = cpu_sec
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

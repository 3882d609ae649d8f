"""GPU tier: the prefill kernels' dynamic work tail (tuning tail_dynamic_pct).

With a dynamic tail, the last share of a launch's work items is handed out at
run time by a per-stream ticket counter (whichever XCD frees a slot first
takes the next item), instead of a fixed item per workgroup. Which workgroup
computes an item must not change any result: every item is computed exactly
once, by the same code, so the outputs are bit-identical to the static
placement. Outputs are filled with NaN before every call, so an item that no
workgroup took would show. The counter is left at zero by each launch (the
workgroup drawing the last ticket resets it), which the repeated calls check;
launches on two streams use two counters; a launch captured in a graph gets
its own counter and replays correctly.

Shape B=2, Hq=32, Hkv=8, S=4096, D=128: 2048 forward and dQ items and 512
dK/dV items, above the kernels' minimums for a tail (two items per resident
workgroup slot).
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from gpu_util import DEV, note
from pallas_flash import _lib, flash_attention

pytestmark = pytest.mark.gpu

B, HQ, HKV, S, D = 2, 32, 8, 4096, 128


def _inputs(seed, dt=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    mk = lambda *s: torch.randn(s, generator=g, device=DEV).to(dt)
    return mk(B, HQ, S, D), mk(B, HKV, S, D), mk(B, HKV, S, D), mk(B, HQ, S, D)


class _Step:
    """The three prefill launches through the C ABI on given buffers."""

    def __init__(self, q, k, v, do, causal):
        self.q, self.k, self.v, self.do = q, k, v, do
        self.o = torch.empty_like(q)
        self.lse = torch.empty((B, HQ, S), device=DEV)
        self.delta = torch.empty_like(self.lse)
        self.dq, self.dk, self.dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        sc = D ** -0.5
        dtag = _lib.dtype_tag(q)
        self.fa = _lib.FwdArgs(q.data_ptr(), k.data_ptr(), v.data_ptr(), self.o.data_ptr(), self.lse.data_ptr(),
                               B, HQ, HKV, S, S, D, S, int(causal), sc, dtag)
        self.ba = _lib.BwdArgs(q.data_ptr(), k.data_ptr(), v.data_ptr(), self.o.data_ptr(), do.data_ptr(),
                               self.lse.data_ptr(), self.delta.data_ptr(), self.dq.data_ptr(), self.dk.data_ptr(),
                               self.dv.data_ptr(), B, HQ, HKV, S, S, D, S, int(causal), sc, dtag)

    def outputs(self):
        return (self.o, self.lse, self.delta, self.dq, self.dk, self.dv)

    def run(self, stream=None):
        """NaN-fill the outputs and launch the three kernels, all on `stream`
        (default: the current stream), so the fill is ordered before them."""
        L = _lib.lib()
        s = stream or torch.cuda.current_stream()
        with torch.cuda.stream(s):
            for t in self.outputs():
                t.fill_(float("nan"))
            assert L.pf_attn_fwd(ctypes.byref(self.fa), s.cuda_stream) == 0
            assert L.pf_attn_bwd_dq(ctypes.byref(self.ba), s.cuda_stream) == 0
            assert L.pf_attn_bwd_dkv(ctypes.byref(self.ba), s.cuda_stream) == 0


def _same(a, b):
    return all(torch.equal(x, y) for x, y in zip(a, b))


@pytest.mark.parametrize("causal", [True, False])
def test_tail_outputs_bit_identical_to_static(causal):
    """Forward, dQ (with delta) and dK/dV: 0% (static), 30% and 100% dynamic
    give the same bits, three calls in a row at each share."""
    note(f"work tail: bit-identical causal={causal}")
    step = _Step(*_inputs(1), causal)
    with _lib.tuning(tail_dynamic_pct=0):
        step.run()
        torch.cuda.synchronize()
        ref = [t.clone() for t in step.outputs()]
    assert all(torch.isfinite(t).all() for t in ref)
    for pct in (30, 100):
        with _lib.tuning(tail_dynamic_pct=pct):
            for rep in range(3):
                step.run()
                torch.cuda.synchronize()
                assert _same(step.outputs(), ref), f"share {pct}%, call {rep}"


def test_tail_on_two_streams():
    """Two streams launching in alternation with no synchronisation between
    the calls (each stream has its own ticket counter)."""
    note("work tail: two streams")
    a, b = _Step(*_inputs(2), True), _Step(*_inputs(3), True)
    with _lib.tuning(tail_dynamic_pct=0):
        a.run()
        b.run()
        torch.cuda.synchronize()
        ref_a = [t.clone() for t in a.outputs()]
        ref_b = [t.clone() for t in b.outputs()]
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()  # the inputs, written on the default stream, are ready
    with _lib.tuning(tail_dynamic_pct=30):
        for _ in range(4):
            a.run(sa)
            b.run(sb)
        torch.cuda.synchronize()
    assert _same(a.outputs(), ref_a)
    assert _same(b.outputs(), ref_b)


def test_tail_graph_replay():
    """flash_attention forward + backward with a dynamic tail, captured and
    replayed four times while the inputs change in place; each replay equals
    the eager step (with eager launches on the same stream between replays)."""
    note("work tail: graph replay")
    q0, k0, v0, do = _inputs(4)
    q, k, v = (t.clone().requires_grad_(True) for t in (q0, k0, v0))
    g = torch.Generator(device=DEV).manual_seed(5)

    def step():
        out = flash_attention(q, k, v, causal=True)
        return (out,) + torch.autograd.grad(out, (q, k, v), do)

    with _lib.tuning(tail_dynamic_pct=30):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            outs_g = step()
        for it in range(4):
            with torch.no_grad():
                for t in (q, k, v, do):
                    t.copy_(torch.randn(t.shape, generator=g, device=DEV).to(t.dtype))
            graph.replay()
            outs_e = step()
            torch.cuda.synchronize()
            for name, x, y in zip(("o", "dq", "dk", "dv"), outs_g, outs_e):
                assert torch.equal(x, y), f"replay {it}: {name}"

"""GPU tier: the prefill training step, paged decode, fused RoPE and decode
captured in HIP graphs (torch.cuda.graph over the C-ABI launches) and
replayed.

Every launch of these paths runs on torch's current stream, allocates only
through torch (graph-private pool under capture), issues no memset and reads
no device value on the host, so the step can be captured once and replayed
while its inputs change in place. Each replay is checked bit for bit against
the eager call on the same inputs, with eager work and synchronisations
between the replays.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import DEV, note
from pallas_flash import flash_attention, paged_flash_attention

pytestmark = pytest.mark.gpu


def _warm(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_training_step_graph_replay(dt):
    """flash_attention forward + backward (autograd) captured: o, dq, dk, dv of
    every replay equal the eager step on the inputs written in place."""
    note(f"graph: training step {dt}")
    B, Hq, Hkv, S, D = 1, 8, 2, 384, 128
    g = torch.Generator(device=DEV).manual_seed(21)
    mk = lambda *s: torch.randn(s, generator=g, device=DEV).to(dt)
    q, k, v = (mk(*s).requires_grad_(True) for s in ((B, Hq, S, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    do = mk(B, Hq, S, D)

    def step():
        out = flash_attention(q, k, v, causal=True)
        return (out,) + torch.autograd.grad(out, (q, k, v), do)

    _warm(step)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs_g = step()
    for it in range(4):
        with torch.no_grad():
            for t in (q, k, v, do):
                t.copy_(torch.randn(t.shape, generator=g, device=DEV).to(dt))
        graph.replay()
        outs_e = step()
        torch.cuda.synchronize()
        for name, a, b in zip(("o", "dq", "dk", "dv"), outs_g, outs_e):
            assert torch.equal(a, b), f"replay {it}: {name}"


def test_paged_decode_graph_replay_lengths_on_device():
    """Paged decode captured with its block table and lengths in device
    memory; the lengths grow on the GPU between replays (as a serving loop's
    would), and every replay equals the eager call."""
    note("graph: paged decode")
    rng = np.random.default_rng(22)
    B, Hq, Hkv, D, page, npages, pps = 4, 8, 2, 128, 16, 64, 8
    table = torch.as_tensor(rng.permutation(npages)[:B * pps].reshape(B, pps).astype(np.int32), device=DEV)
    lens = torch.as_tensor(np.array([1, 17, 40, 100], np.int32), device=DEV)
    g = torch.Generator(device=DEV).manual_seed(22)
    kp = torch.randn((npages, Hkv, page, D), generator=g, device=DEV).to(torch.bfloat16)
    vp = torch.randn((npages, Hkv, page, D), generator=g, device=DEV).to(torch.bfloat16)
    q = torch.randn((B, Hq, 1, D), generator=g, device=DEV).to(torch.bfloat16)
    run = lambda: paged_flash_attention(q, kp, vp, table, lens)
    _warm(run)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o_g = run()
    for it in range(6):
        graph.replay()
        o_e = run()
        torch.cuda.synchronize()
        assert torch.equal(o_g, o_e), f"replay {it}"
        lens.add_(5).clamp_(max=pps * page)
        q.copy_(torch.randn(q.shape, generator=g, device=DEV).to(q.dtype))


def test_rope_forward_and_decode_graph_replay():
    """The fused-RoPE forward (its rotated-K workspace from the graph pool)
    and the contiguous decode captured together; replays with new inputs
    equal the eager calls."""
    from pallas_flash import flash_attention_decode, flash_attention_rope, precompute_rope
    note("graph: rope forward + decode")
    g = torch.Generator(device=DEV).manual_seed(23)
    mk = lambda *s: torch.randn(s, generator=g, device=DEV).to(torch.bfloat16)
    B, Hq, Hkv, S, D = 2, 8, 2, 320, 128
    cos, sin = precompute_rope(S, D, 10000.0, device=DEV)
    q, k, v = mk(B, Hq, S, D), mk(B, Hkv, S, D), mk(B, Hkv, S, D)
    qd, kc, vc = mk(4, 8, 1, D), mk(4, 2, 512, D), mk(4, 2, 512, D)

    def run():
        with torch.no_grad():
            return (flash_attention_rope(q, k, v, cos, sin, causal=True),
                    flash_attention_decode(qd, kc, vc, 300))

    _warm(run)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs_g = run()
    for it in range(4):
        for t in (q, k, v, qd, kc):
            t.copy_(torch.randn(t.shape, generator=g, device=DEV).to(t.dtype))
        graph.replay()
        outs_e = run()
        torch.cuda.synchronize()
        for name, a, b in zip(("rope", "decode"), outs_g, outs_e):
            assert torch.equal(a, b), f"replay {it}: {name}"

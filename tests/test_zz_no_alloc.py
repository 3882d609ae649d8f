"""GPU tier: pf_paged_attn_noalloc, the paged decode that allocates nothing
(its split-KV partials live in the library's static per-device array).

Called through the C ABI, it must give bit for bit what pf_paged_attn gives
with a caller workspace, on two calls in a row where the second is smaller
(the array keeps the first call's contents), on the streaming kernel
(bf16, page 64 and page 16), on a small persistent grid that cuts sequences
across waves (partials in the array), and on the generic kernel (float32,
page size 5; bf16 at head_dim 256); sizes past the array are refused before
any launch.
A call recorded into a HIP graph replays correctly while its inputs change
in place, also when it is the process's first call of the entry point (the
array's address is then looked up during the recording).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from gpu_util import dev, note
from pallas_flash import _lib

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20  # PF_NOALLOC_SCRATCH_BYTES


def _problem(seed, B, Hq, Hkv, page, pps, num_pages, dt, max_len, D=128):
    rng = np.random.default_rng(seed)
    lens = rng.integers(1, max_len + 1, B).astype(np.int32)
    lens[0] = 0  # an empty sequence
    perm = rng.permutation(num_pages)
    table = np.full((B, pps), -1, np.int32)
    cur = 0
    for b in range(B):
        n = min(-(-int(lens[b]) // page), pps)
        table[b, :n] = perm[cur:cur + n]
        cur += n
    assert cur <= num_pages
    q = dev(rng.standard_normal((B, Hq, 1, D)), dt)
    kp = dev(rng.standard_normal((num_pages, Hkv, page, D)), dt)
    vp = dev(rng.standard_normal((num_pages, Hkv, page, D)), dt)
    return q, kp, vp, torch.as_tensor(table, device="cuda"), torch.as_tensor(lens, device="cuda")


def _args(q, kp, vp, tt, tl, o):
    B, Hq = q.shape[0], q.shape[1]
    num_pages, Hkv, page, D = kp.shape
    return _lib.PagedArgs(q.data_ptr(), kp.data_ptr(), vp.data_ptr(), tt.data_ptr(), tl.data_ptr(),
                          o.data_ptr(), B, Hq, Hkv, num_pages, page, D, tt.shape[1], 1.0 / D ** 0.5,
                          _lib.dtype_tag(q), None, 0)


def _with_workspace(L, args, q):
    ws_bytes = L.pf_paged_attn_workspace_size(ctypes.byref(args))
    assert 0 < ws_bytes <= SCRATCH_BYTES
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    st = L.pf_paged_attn(ctypes.byref(args), torch.cuda.current_stream().cuda_stream)
    assert st == _lib.PF_OK, st
    torch.cuda.synchronize()
    args.workspace, args.workspace_bytes = None, 0
    del ws


CASES = [  # (name, dt, page, Hq, Hkv, decode_waves, head_dim)
    ("stream bf16 page 64", "bf16", 64, 32, 8, 0, 128),
    ("stream bf16 page 16, 7-wave grid", "bf16", 16, 16, 2, 7, 128),
    ("generic f32 page 5", "f32", 5, 8, 2, 0, 128),
    ("generic bf16 head_dim 256 page 16", "bf16", 16, 8, 2, 0, 256),
]


@pytest.mark.parametrize("name,dt,page,Hq,Hkv,waves,D", CASES)
def test_noalloc_matches_workspace_entry_point(name, dt, page, Hq, Hkv, waves, D):
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    with _lib.tuning(decode_waves=waves):
        for call, (B, pps, max_len) in enumerate(((24, 40, 40 * page), (5, 12, 12 * page))):
            note(f"noalloc {name}: call {call + 1} B={B} pps={pps}")
            q, kp, vp, tt, tl = _problem(50 + call, B, Hq, Hkv, page, pps, B * pps, dt, max_len, D)
            want = torch.full_like(q, float("nan"))
            got = torch.full_like(q, float("nan"))
            _with_workspace(L, _args(q, kp, vp, tt, tl, want), q)
            st = L.pf_paged_attn_noalloc(ctypes.byref(_args(q, kp, vp, tt, tl, got)), stream)
            assert st == _lib.PF_OK, st
            torch.cuda.synchronize()
            assert torch.isfinite(want.float()).all()
            assert torch.equal(got, want), f"{name} call {call + 1}: differs from pf_paged_attn"
            assert not want[0].any()  # the empty sequence gives zeros


def test_noalloc_refuses_partials_past_the_array():
    """The generic kernel's partials grow with the batch: past the array the
    call is refused (PF_ERR_WORKSPACE) and the output is untouched."""
    L = _lib.lib()
    B, Hq, Hkv, page = 4096, 32, 8, 5
    q = torch.zeros((B, Hq, 1, 128), dtype=torch.float32, device="cuda")
    kp = torch.zeros((8, Hkv, page, 128), dtype=torch.float32, device="cuda")
    tt = torch.zeros((B, 2), dtype=torch.int32, device="cuda")
    tl = torch.full((B,), 7, dtype=torch.int32, device="cuda")
    o = torch.full_like(q, 3.0)
    args = _args(q, kp, kp, tt, tl, o)
    assert L.pf_paged_attn_workspace_size(ctypes.byref(args)) > SCRATCH_BYTES
    note("noalloc oversize refusal")
    st = L.pf_paged_attn_noalloc(ctypes.byref(args), torch.cuda.current_stream().cuda_stream)
    assert st == _lib.PF_ERR_WORKSPACE
    torch.cuda.synchronize()
    assert bool((o == 3.0).all())


def _graph_check(capture_first: bool) -> None:
    """Record pf_paged_attn_noalloc into a graph (torch.cuda.graph) and replay
    it four times with q and the pools rewritten in place; every replay
    equals pf_paged_attn on the same inputs, bit for bit."""
    L = _lib.lib()
    q, kp, vp, tt, tl = _problem(70, 12, 32, 8, 64, 24, 12 * 24, "bf16", 24 * 64)
    got = torch.full_like(q, float("nan"))
    want = torch.full_like(q, float("nan"))
    args = _args(q, kp, vp, tt, tl, got)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    if not capture_first:
        with torch.cuda.stream(s):
            assert L.pf_paged_attn_noalloc(ctypes.byref(args), s.cuda_stream) == _lib.PF_OK
        torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        st = L.pf_paged_attn_noalloc(ctypes.byref(args), torch.cuda.current_stream().cuda_stream)
    assert st == _lib.PF_OK, st
    g = torch.Generator(device="cuda").manual_seed(71)
    for it in range(4):
        with torch.no_grad():
            for t in (q, kp, vp):
                t.copy_(torch.randn(t.shape, generator=g, device="cuda").to(t.dtype))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _with_workspace(L, _args(q, kp, vp, tt, tl, want), q)
        assert torch.isfinite(want.float()).all()
        assert torch.equal(got, want), f"replay {it} differs from pf_paged_attn"


def test_noalloc_graph_replay():
    note("noalloc graph replay")
    _graph_check(capture_first=False)


def test_noalloc_first_call_under_capture():
    """In a fresh process whose first pf_paged_attn_noalloc call is being
    recorded into a graph."""
    note("noalloc first call under capture (child process)")
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([here, root, os.path.join(root, "tpu-native-pallas-flashattention_amd"),
                                         env.get("PYTHONPATH", "")])
    code = "import test_zz_no_alloc as t; t._graph_check(capture_first=True); print('child ok', flush=True)"
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and "child ok" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]

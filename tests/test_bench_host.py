"""CPU tier: the host side of bench.py that needs no GPU.

The roofline's `traffic` field comes from the committed rocprofv3 --pmc
summary (profiles/traffic.json); every kernel the config 3 step credits must
resolve to exactly one record there, or the bench line would carry null.
"""

from __future__ import annotations

import os
import subprocess
import sys

import pytest

from conftest import ROOT

sys.path.insert(0, ROOT)
import bench  # noqa: E402


@pytest.mark.parametrize("kernel", ["pf_attn_fwd_kernel", "pf_attn_bwd_dq_kernel",
                                    "pf_attn_bwd_dkv_kernel"])
def test_cfg3_traffic_resolves(kernel):
    b = bench.load_traffic(kernel, "cfg3")
    assert b is not None and b > 0


def test_traffic_lookup_needs_a_unique_match():
    # "pf_attn_fwd" is a prefix of a kernel name but not a kernel name
    assert bench.load_traffic("pf_attn_fwd", "cfg3") is None
    # config 2 runs the forward twice (RoPE and plain): the base name is ambiguous
    assert bench.load_traffic("pf_attn_fwd_kernel", "rope") is None
    assert bench.load_traffic("pf_attn_fwd_kernel", "no-such-workload") is None


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_cfg5_layout_matches_the_stated_workload():
    """Config 5 as the measurement contract states it: lengths from
    default_rng(0) in [512, 8192] summing to 567,626 tokens, pages dealt out
    of one permutation (no page shared), the table -1-padded past each
    sequence's ceil(len / 64) pages."""
    import numpy as np
    lens, table, used = bench.cfg5_layout()
    assert lens.shape == (128,) and lens.min() >= 512 and lens.max() <= 8192
    assert int(lens.sum()) == 567_626
    npg = -(-lens // 64)
    for b in range(128):
        assert (table[b, :npg[b]] >= 0).all() and (table[b, npg[b]:] == -1).all()
    mapped = table[table >= 0]
    assert len(np.unique(mapped)) == mapped.size == int(npg.sum()) == int(used.sum())


def test_aux_cpu_baselines_run_on_small_inputs():
    import torch
    g = torch.Generator().manual_seed(0)
    mk = lambda *s: torch.randn(s, generator=g).to(torch.bfloat16)
    cos = torch.rand(16, 64)
    sin = torch.rand(16, 64)
    a = {"kv": {"rows": mk(2, 2, 12, 64), "C": 32}, "paged": {"rows": mk(3, 2, 8, 64), "page": 4},
         "rope": {"g": mk(1, 2, 16, 64), "cos": cos, "sin": sin}}
    out = bench.cpu_baseline_aux(a)
    assert set(out) == {"kv_write", "paged_write", "rope_vjp"}
    for v in out.values():
        assert v["unit"] == "GB/s" and v["value"] > 0 and v["kind"] == "port" and v["cores"] >= 1


def test_cfg3_cpu_baseline_runs_on_a_small_sample():
    """The config 3 CPU leg (warm-up, then the median of the timed passes)
    on a tiny stand-in for config 3's inputs."""
    import torch
    g = torch.Generator().manual_seed(0)
    mk = lambda *s: torch.randn(s, generator=g).to(torch.bfloat16)
    c3 = {"S": 64, "D": 32, "Hq": 8, "Hkv": 2,
          "host": {"q": mk(2, 8, 64, 32), "k": mk(2, 2, 64, 32), "v": mk(2, 2, 64, 32), "do": mk(2, 8, 64, 32)}}
    out = bench.cpu_baseline(c3, n_kv=2, reps=3)
    assert out["unit"] == "TFLOP/s" and out["value"] > 0 and out["kind"] == "port"
    assert "median of 3" in out["sample"] and "recomputes" in out["sample"]

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

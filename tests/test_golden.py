"""Golden fixtures (tests/golden/fixtures.npz).

CPU: the oracle still reproduces the committed fixtures (guards the oracle
against silent drift). GPU: every kernel family reproduces them, in float32
and in bfloat16 (the fixture inputs are exactly bf16-representable).
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from conftest import ROOT

FIX = os.path.join(ROOT, "tests", "golden", "fixtures.npz")


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_oracle_reproduces_fixtures(fx):
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_fixtures",
                                                  os.path.join(ROOT, "tests", "golden", "make_fixtures.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    fresh = mod.build()
    assert set(fresh) == set(fx)
    for k, v in fresh.items():
        if v.dtype.kind == "f":
            np.testing.assert_allclose(fx[k], v, rtol=1e-6, atol=1e-7, err_msg=k)
        else:
            np.testing.assert_array_equal(fx[k], v, err_msg=k)


@pytest.mark.gpu
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_kernels_reproduce_fixtures(fx, dt):
    import torch
    from gpu_util import check_fwd, check_grad, dev, host, note
    from pallas_flash import (flash_attention, flash_attention_decode, flash_attention_rope,
                              flash_attention_with_lse, paged_flash_attention)

    note(f"golden fwd {dt}")
    o, lse = flash_attention_with_lse(dev(fx["fwd_q"], dt), dev(fx["fwd_k"], dt), dev(fx["fwd_v"], dt),
                                      causal=True, kv_len=83)
    check_fwd(host(o), fx["fwd_o"].astype(np.float64), dt)
    assert np.abs(host(lse) - fx["fwd_lse"]).max() < (1e-5 if dt == "f32" else 1e-3)

    note(f"golden bwd {dt}")
    q, k, v = (dev(fx[n], dt).requires_grad_(True) for n in ("bwd_q", "bwd_k", "bwd_v"))
    flash_attention(q, k, v, causal=True).backward(dev(fx["bwd_do"], dt))
    for name, t in (("dq", q), ("dk", k), ("dv", v)):
        check_grad(host(t.grad), fx["bwd_" + name].astype(np.float64), dt, name)

    note(f"golden decode {dt}")
    od = flash_attention_decode(dev(fx["dec_q"], dt), dev(fx["dec_k"], dt), dev(fx["dec_v"], dt),
                                int(fx["dec_len"]))
    check_fwd(host(od), fx["dec_o"].astype(np.float64), dt)

    note(f"golden paged {dt}")
    op = paged_flash_attention(dev(fx["pg_q"], dt), dev(fx["pg_k"], dt), dev(fx["pg_v"], dt),
                               torch.as_tensor(fx["pg_table"]), torch.as_tensor(fx["pg_lens"]))
    check_fwd(host(op), fx["pg_o"].astype(np.float64), dt)

    note(f"golden rope {dt}")
    orp = flash_attention_rope(dev(fx["rope_q"], dt), dev(fx["rope_k"], dt), dev(fx["rope_v"], dt),
                               torch.as_tensor(fx["rope_cos"]).cuda(), torch.as_tensor(fx["rope_sin"]).cuda(),
                               causal=True)
    check_fwd(host(orp), fx["rope_o"].astype(np.float64), dt)

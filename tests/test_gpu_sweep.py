"""GPU tier: a seeded random sweep of prefill shapes through the forward (with
LSE) and the backward, against the float64 oracle at the north-star bars.

The fixed-shape tests re-express the reference's own cases; this sweep adds
the combinations they leave out: every dtype with both head dims, GQA ratios
1 to 8, Sq and Sk from below one tile to a few tiles (independently, so
Sq != Sk with top-left causal masking), kv_len < Sk and a non-default scale.
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


def _inputs(seed, dt, B, Hq, Hkv, Sq, Sk, D):
    rng = np.random.default_rng(seed)
    q = dev(rng.standard_normal((B, Hq, Sq, D)), dt)
    k = dev(rng.standard_normal((B, Hkv, Sk, D)), dt)
    v = dev(rng.standard_normal((B, Hkv, Sk, D)), dt)
    do = dev(rng.standard_normal((B, Hq, Sq, D)), dt)
    return q, k, v, do


@pytest.mark.parametrize("dt,D,B,Hq,Hkv,Sq,Sk,causal,kv_len,scale", _cases(101))
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


@pytest.mark.parametrize("dt,D,B,Hq,Hkv,Sq,Sk,causal,kv_len,scale", _cases(202))
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

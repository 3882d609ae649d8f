"""GPU tier: the opt-in 64-rows-per-wave forward (tuning fwd_rows_per_wave=64,
bf16/f16, D = 128) against the float64 oracle, through the backward that
consumes its O and LSE, with fused RoPE, and against the default 32-row
kernel at larger shapes up to config 3's.

The host reads the tuning at every call, so setting it around one test routes
exactly that test's forwards through the wide kernel.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import check_fwd, check_grad, dev, host, note
from oracle import attention_bwd_ref, attention_ref
from pallas_flash import _lib, flash_attention, flash_attention_with_lse

pytestmark = pytest.mark.gpu


@pytest.fixture
def wide():
    with _lib.tuning(fwd_rows_per_wave=64):
        yield


def _cases(seed: int, n: int):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        dt = ("bf16", "f16")[i % 2]
        Hkv = int(rng.integers(1, 3))
        g = int(rng.choice([1, 2, 4, 8]))
        B = int(rng.integers(1, 3))
        Sq = int(rng.integers(1, 420))
        Sk = Sq if i % 3 == 0 else int(rng.integers(1, 420))
        causal = bool(rng.integers(0, 2))
        kv_len = int(rng.integers(1, Sk + 1)) if rng.integers(0, 2) else None
        scale = float(rng.uniform(0.05, 0.3)) if i % 5 == 4 else None
        out.append(pytest.param(dt, B, Hkv * g, Hkv, Sq, Sk, causal, kv_len, scale, id=f"w{i}-{dt}"))
    return out


def _inputs(seed, dt, B, Hq, Hkv, Sq, Sk, D=128):
    rng = np.random.default_rng(seed)
    return (dev(rng.standard_normal((B, Hq, Sq, D)), dt), dev(rng.standard_normal((B, Hkv, Sk, D)), dt),
            dev(rng.standard_normal((B, Hkv, Sk, D)), dt), dev(rng.standard_normal((B, Hq, Sq, D)), dt))


@pytest.mark.parametrize("dt,B,Hq,Hkv,Sq,Sk,causal,kv_len,scale", _cases(707, 16))
def test_wide_forward_and_lse(wide, dt, B, Hq, Hkv, Sq, Sk, causal, kv_len, scale):
    note(f"wide fwd dt={dt} B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Sk={Sk} causal={causal} kv_len={kv_len} scale={scale}")
    q, k, v, _ = _inputs(21, dt, B, Hq, Hkv, Sq, Sk)
    o, lse = flash_attention_with_lse(q, k, v, causal=causal, kv_len=kv_len, sm_scale=scale)
    want_o, want_lse = attention_ref(host(q), host(k), host(v), causal=causal, kv_len=kv_len, sm_scale=scale)
    check_fwd(host(o), want_o, dt)
    lse_err = np.abs(host(lse) - want_lse).max() / (np.abs(want_lse).max() + 1.0)
    assert lse_err <= 1e-3, f"lse error {lse_err:.3e}"


@pytest.mark.parametrize("dt,B,Hq,Hkv,Sq,Sk,causal,kv_len,scale", _cases(808, 6))
def test_wide_forward_backward(wide, dt, B, Hq, Hkv, Sq, Sk, causal, kv_len, scale):
    note(f"wide bwd dt={dt} B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Sk={Sk} causal={causal} kv_len={kv_len}")
    q, k, v, do = _inputs(22, dt, B, Hq, Hkv, Sq, Sk)
    for t in (q, k, v):
        t.requires_grad_(True)
    flash_attention(q, k, v, causal=causal, kv_len=kv_len, sm_scale=scale).backward(do)
    want = attention_bwd_ref(host(q), host(k), host(v), host(do), causal=causal, kv_len=kv_len, sm_scale=scale)
    for name, t, w in zip("qkv", (q, k, v), want):
        check_grad(host(t.grad), w, dt, "d" + name)


@pytest.mark.parametrize("dt,Sq,Sk,causal", [("bf16", 300, 300, True), ("f16", 200, 333, False)])
def test_wide_rope(wide, dt, Sq, Sk, causal):
    from oracle import rope_attention_ref
    from pallas_flash import flash_attention_rope, precompute_rope
    note(f"wide rope dt={dt} Sq={Sq} Sk={Sk} causal={causal}")
    q, k, v, _ = _inputs(23, dt, 1, 8, 2, Sq, Sk)
    cos, sin = precompute_rope(max(Sq, Sk), 128, 10000.0, device="cuda")
    qc, qs, kc, ks = cos[:Sq], sin[:Sq], cos[:Sk], sin[:Sk]
    out = flash_attention_rope(q, k, v, qc, qs, kc, ks, causal=causal)
    want = rope_attention_ref(host(q), host(k), host(v), host(qc), host(qs), host(kc), host(ks), causal=causal)
    check_fwd(host(out), want, dt)


@pytest.mark.parametrize("B,Hq,Hkv,S,causal", [(1, 8, 2, 1536, True), (1, 8, 2, 1536, False),
                                               (2, 16, 4, 8192, True)])  # last: config 3's shape
def test_wide_matches_default_kernel(B, Hq, Hkv, S, causal):
    """Both tilings compute each row with the same operations in the same
    order; they may differ only where a bf16 rounding of O flips (one ulp)."""
    note(f"wide vs default B={B} Hq={Hq} Hkv={Hkv} S={S} causal={causal}")
    g = torch.Generator(device="cuda").manual_seed(24)
    q, k, v = (torch.randn((B, h, S, 128), generator=g, device="cuda").to(torch.bfloat16) for h in (Hq, Hkv, Hkv))
    res = {}
    for rows in ("32", "64"):
        with _lib.tuning(fwd_rows_per_wave=int(rows)):
            o, lse = flash_attention_with_lse(q, k, v, causal=causal)
            torch.cuda.synchronize()
        res[rows] = (o.float(), lse.clone())
    o32, l32 = res["32"]
    o64, l64 = res["64"]
    ulp = torch.maximum(o32.abs(), o64.abs()) * 2.0 ** -7 + 1e-30
    assert bool(((o32 - o64).abs() <= ulp).all()), "O differs by more than one bf16 ulp"
    assert float((l32 - l64).abs().max()) <= 1e-5 * float(l32.abs().max())

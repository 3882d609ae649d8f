"""Helpers shared by the GPU parity tests (not a test module).

Inputs are generated on the host with ``np.random.default_rng(seed)`` in
float64, rounded to the kernel dtype on the device, and the oracle is run on
exactly the rounded values the kernel sees.
"""

from __future__ import annotations

import sys

import numpy as np
import torch

DEV = "cuda"

TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}

# Tolerances from the north star: fp32 max-abs error <= 1e-5 relative to the
# reference's max magnitude; bf16/f16 outputs <= 2e-2 absolute; bf16/f16
# gradients <= 5e-2 relative.
FWD_TOL = {"f32": 1e-5, "bf16": 2e-2, "f16": 2e-2}
GRAD_REL_TOL = {"f32": 1e-5, "bf16": 5e-2, "f16": 5e-2}


def note(msg: str) -> None:
    """Print-and-flush the case being run (names the case if the box dies)."""
    print(msg, flush=True)
    sys.stdout.flush()


def dev(x, dt: str) -> torch.Tensor:
    return torch.as_tensor(np.ascontiguousarray(x)).to(DEV).to(TORCH_DT[dt]).contiguous()


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def rel_err(a, b) -> float:
    return float(np.abs(a - b).max() / (np.abs(b).max() + 1e-9))


def max_abs(a, b) -> float:
    return float(np.abs(a - b).max())


def check_fwd(out: np.ndarray, ref: np.ndarray, dt: str) -> None:
    assert np.isfinite(out).all()
    if dt == "f32":
        err = rel_err(out, ref)
        assert err <= FWD_TOL[dt], f"f32 relative max-abs error {err:.3e}"
    else:
        err = max_abs(out, ref)
        assert err <= FWD_TOL[dt], f"{dt} max-abs error {err:.3e}"


def check_grad(got: np.ndarray, want: np.ndarray, dt: str, name: str) -> None:
    assert np.isfinite(got).all(), name
    err = rel_err(got, want)
    assert err <= GRAD_REL_TOL[dt], f"{name}: {dt} relative error {err:.3e}"


def qkv(rng, B, Hq, Hkv, Sq, Sk, D=128):
    return (rng.standard_normal((B, Hq, Sq, D)), rng.standard_normal((B, Hkv, Sk, D)),
            rng.standard_normal((B, Hkv, Sk, D)))

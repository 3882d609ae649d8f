"""CPU tier: head_dim padding and dtype selection of the Python API
(pallas_flash._shape), checked without a GPU.

The padded problem must have the same answer as the caller's: zero columns
leave q.k unchanged and give zero output columns, and RoPE's half-by-half
padding keeps every element with its rotation partner. Both are checked
against the float64 oracle on the padded and unpadded inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import apply_rope_ref, attention_ref, precompute_rope_ref
from pallas_flash._shape import (compute_dtype, decode_head_dim, kernel_head_dim, max_head_dim, pad_head_dim,
                                 pad_rope_halves, unpad_rope_halves)

BF, F16, F32 = torch.bfloat16, torch.float16, torch.float32


@pytest.mark.parametrize("d,want", [(1, 64), (32, 64), (64, 64), (65, 128), (80, 128), (128, 128)])
@pytest.mark.parametrize("dt", [BF, F16, F32])
def test_kernel_head_dim(d, want, dt):
    assert kernel_head_dim(d, dt) == want


@pytest.mark.parametrize("d,want", [(129, 256), (160, 256), (192, 256), (256, 256)])
@pytest.mark.parametrize("dt", [BF, F16])
def test_kernel_head_dim_above_128_16bit(d, want, dt):
    assert kernel_head_dim(d, dt) == want


def test_head_dim_limits():
    """256 columns for the 16-bit kernels, 128 for float32 (the compute dtype
    of float32 and mixed inputs); above that NotImplementedError."""
    assert (max_head_dim(BF), max_head_dim(F16), max_head_dim(F32)) == (256, 256, 128)
    for dt in (BF, F16):
        with pytest.raises(NotImplementedError):
            kernel_head_dim(257, dt)
    for d in (129, 256):
        with pytest.raises(NotImplementedError):
            kernel_head_dim(d, F32)
    with pytest.raises(ValueError):
        kernel_head_dim(0, BF)


@pytest.mark.parametrize("d,dt,want", [
    (96, BF, 96), (200, BF, 200), (256, F16, 256), (136, BF, 136),   # whole 16-byte chunks: in place
    (100, BF, 128), (250, BF, 256), (33, BF, 64),                   # ragged chunks: padded
    (132, F32, None),                                               # float32 above 128: unsupported
    (124, F32, 124), (126, F32, 128)])
def test_decode_head_dim(d, dt, want):
    if want is None:
        with pytest.raises(NotImplementedError):
            decode_head_dim(d, dt)
    else:
        assert decode_head_dim(d, dt) == want


def test_compute_dtype():
    f32, bf, h, f64 = (torch.zeros(1, dtype=t) for t in (torch.float32, torch.bfloat16, torch.float16,
                                                          torch.float64))
    assert compute_dtype(bf, bf, bf) == torch.bfloat16
    assert compute_dtype(h, h, h) == torch.float16
    assert compute_dtype(f32, f32, f32) == torch.float32
    assert compute_dtype(bf, f32, f32) == torch.float32       # mixed: float32, as the reference
    assert compute_dtype(bf, h, h) == torch.float32
    assert compute_dtype(f64, f64, f64) == torch.float32      # no float64 kernel


@pytest.mark.parametrize("d", [32, 80, 96, 160])
def test_zero_padding_keeps_attention(d):
    rng = np.random.default_rng(d)
    q, k, v = (rng.standard_normal((1, 2, 9, d)) for _ in range(3))
    dp = kernel_head_dim(d, BF)
    pad = lambda x: pad_head_dim(torch.from_numpy(x), dp).numpy()
    scale = 1.0 / d ** 0.5                          # the caller's head_dim sets the default scale
    o, lse = attention_ref(q, k, v, causal=True)
    op, lsep = attention_ref(pad(q), pad(k), pad(v), causal=True, sm_scale=scale)
    assert np.allclose(op[..., :d], o, atol=1e-12) and np.all(op[..., d:] == 0)
    assert np.allclose(lsep, lse, atol=1e-12)


@pytest.mark.parametrize("d", [32, 80, 96, 200])
def test_rope_half_padding_commutes_with_rotation(d):
    rng = np.random.default_rng(d + 1)
    x = rng.standard_normal((1, 2, 7, d))
    cos, sin = precompute_rope_ref(7, d)
    dp = kernel_head_dim(d, BF)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    xp, cp, sp = (pad_rope_halves(t(a), dp).numpy() for a in (x, cos, sin))
    y = apply_rope_ref(x, cos, sin)
    yp = apply_rope_ref(xp, cp, sp)
    assert np.allclose(unpad_rope_halves(t(yp), d).numpy(), y, atol=1e-12)
    # padded slots stay zero, and plain end-padding would break the pairing
    assert np.all(yp[..., d // 2:dp // 2] == 0) and np.all(yp[..., dp // 2 + d // 2:] == 0)
    xe, ce, se = (pad_head_dim(t(a), dp).numpy() for a in (x, cos, sin))
    assert not np.allclose(apply_rope_ref(xe, ce, se)[..., :d], y, atol=1e-3)


def test_unpad_inverts_pad():
    x = torch.arange(2 * 48, dtype=torch.float32).reshape(2, 48)
    assert torch.equal(unpad_rope_halves(pad_rope_halves(x, 64), 48), x)

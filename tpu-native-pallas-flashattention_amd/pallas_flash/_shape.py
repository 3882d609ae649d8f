"""Head-dim and dtype adaptation between the reference's API and the kernels.

The reference accepts any head_dim and any mix of input dtypes: its kernels
cast q, k and v to float32 on load (flash_attention.py:91-93, fused_rope.py:
70-72, paged.py:68-70) and write the output in q's dtype (flash_attention.py:
212, fused_rope.py:202, paged.py:185); gradients come back in each input's
dtype (flash_attention.py:438-442). The HIP kernels here
take head_dim 64, 128 or (bfloat16/float16) 256 and one dtype (float32,
bfloat16 or float16) for all operands. The API bridges the two on the device:

* head_dim: zero-padded to the next kernel size (<= 64 -> 64, <= 128 -> 128,
  <= 256 -> 256). Zero columns add nothing to q.k and give zero output
  columns, which are sliced off; the default scale stays 1/sqrt(head_dim) of
  the caller's head_dim. RoPE pads each half, so element i and its rotation
  partner i + head_dim/2 stay paired. Above the compute dtype's maximum
  (max_head_dim: 256 for bfloat16/float16, 128 for float32, whose 256-column
  tiles would not fit the LDS) NotImplementedError is raised.
* dtype: one supported dtype for all operands runs as is; any other
  combination (mixed dtypes, or float64) is computed in float32, as the
  reference computes, and the output is cast to q's dtype.

Decode and paged decode read any head_dim up to that maximum whose rows are
whole 16-byte chunks (a multiple of 8 for bfloat16/float16, of 4 for float32)
in place (decode_head_dim): the generic decode kernel computes at the next
kernel size with the missing columns as zeros, so the cache or page pool is
not copied. Other head dims there, and mixed dtypes, copy the padded or cast
cache or pool per call, with a one-time warning (warn_copy). Prefill pads its
operands, which are per-call inputs anyway.
"""

from __future__ import annotations

import warnings

import torch
import torch.nn.functional as F

KERNEL_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def max_head_dim(dtype: torch.dtype) -> int:
    """The largest head_dim the kernels compute in ``dtype`` (the compute dtype)."""
    return 256 if dtype in (torch.bfloat16, torch.float16) else 128


def kernel_head_dim(head_dim: int, dtype: torch.dtype) -> int:
    """The head_dim the kernels run for a caller's head_dim, computing in ``dtype``."""
    if head_dim <= 0:
        raise ValueError(f"head_dim must be positive, got {head_dim}")
    top = max_head_dim(dtype)
    if head_dim > top:
        raise NotImplementedError(
            f"head_dim {head_dim} is not supported in {dtype} (the kernels cover head_dim <= {top} there; "
            f"bfloat16/float16 inputs reach 256)")
    for dp in (64, 128, 256):
        if head_dim <= dp:
            return dp
    raise AssertionError("unreachable")


def decode_head_dim(head_dim: int, dtype: torch.dtype) -> int:
    """The head_dim the decode / paged kernels are called with: the caller's
    own when they read its rows in place (up to max_head_dim, rows of whole
    16-byte chunks), else the padded kernel size."""
    es = torch.empty((), dtype=dtype).element_size()
    if 0 < head_dim <= max_head_dim(dtype) and (head_dim * es) % 16 == 0:
        return head_dim
    return kernel_head_dim(head_dim, dtype)


_warned = set()


def warn_copy(what: str, reason: str) -> None:
    """Warn (once per process and call site) that a call copies its cache or
    pool because of its head_dim or dtypes."""
    if what not in _warned:
        _warned.add(what)
        warnings.warn(f"{what}: {reason}; the cache/pool is copied on every call (use one dtype "
                      f"and a head_dim that is a multiple of 8 (16-bit, up to 256) or 4 (float32, up to 128) "
                      f"to avoid it)",
                      RuntimeWarning, stacklevel=3)


def compute_dtype(*tensors: torch.Tensor) -> torch.dtype:
    """The dtype the kernels compute in for these operands."""
    dt = tensors[0].dtype
    if dt in KERNEL_DTYPES and all(t.dtype == dt for t in tensors):
        return dt
    return torch.float32


def pad_head_dim(x: torch.Tensor, dp: int) -> torch.Tensor:
    """x [..., d] zero-padded to [..., dp] (differentiable; x itself if d == dp)."""
    d = x.shape[-1]
    return x if d == dp else F.pad(x, (0, dp - d))


def pad_rope_halves(x: torch.Tensor, dp: int) -> torch.Tensor:
    """x [..., d] (d even) as [x1, 0, x2, 0] with halves of dp/2, so the
    rotate-half pairs (i, i + d/2) land on (i, i + dp/2)."""
    d = x.shape[-1]
    if d == dp:
        return x
    h, hp = d // 2, dp // 2
    return torch.cat([F.pad(x[..., :h], (0, hp - h)), F.pad(x[..., h:], (0, hp - h))], dim=-1)


def unpad_rope_halves(x: torch.Tensor, d: int) -> torch.Tensor:
    """Inverse of pad_rope_halves."""
    dp = x.shape[-1]
    if d == dp:
        return x
    h, hp = d // 2, dp // 2
    return torch.cat([x[..., :h], x[..., hp:hp + h]], dim=-1)


def adapt(x: torch.Tensor, dtype: torch.dtype, dp: int) -> torch.Tensor:
    """Cast to the compute dtype and pad the head dim (no-ops when they match)."""
    return pad_head_dim(x.to(dtype), dp)


def restore(o: torch.Tensor, d: int, dtype: torch.dtype) -> torch.Tensor:
    """Slice the caller's head dim back out and cast to the output dtype."""
    if o.shape[-1] != d:
        o = o[..., :d]
    return o.to(dtype)

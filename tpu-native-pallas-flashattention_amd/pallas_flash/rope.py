"""Rotary-embedding tables and the unfused rotation (torch, on device).

Counterparts of the reference's ``precompute_rope`` / ``apply_rope``
(src/pallas_flash/model.py:41-67): the producers of the cos/sin inputs that
``flash_attention_rope`` consumes, and the unfused path it must match.
"""

from __future__ import annotations

import torch


def precompute_rope(seq_len: int, head_dim: int, theta: float, *, device=None):
    """cos/sin tables ``[seq_len, head_dim]`` in rotate-half layout, float32
    (model.py:41-51): ``inv_freq = 1 / theta^(i / half)``, ``emb =
    concat(pos * inv_freq, pos * inv_freq)``."""
    half = head_dim // 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, half, dtype=torch.float32, device=device) / half))
    pos = torch.arange(seq_len, dtype=torch.float32, device=device)
    freqs = torch.outer(pos, inv_freq)
    emb = torch.cat([freqs, freqs], dim=-1)
    return torch.cos(emb), torch.sin(emb)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """``[x1, x2] -> [-x2, x1]`` over the last axis (model.py:54-57)."""
    half = x.shape[-1] // 2
    return torch.cat([-x[..., half:], x[..., :half]], dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``x * cos + rotate_half(x) * sin`` for ``x [batch, heads, seq, head_dim]``
    and tables ``[seq, head_dim]`` (model.py:60-67). Computed in the promoted
    dtype of x and the tables, as the reference's jnp broadcast does."""
    return x * cos[None, None] + rotate_half(x) * sin[None, None]


__all__ = ["precompute_rope", "apply_rope", "rotate_half"]

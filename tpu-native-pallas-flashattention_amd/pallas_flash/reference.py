"""Naive ``softmax(q k^T) v`` in torch: the materialising baseline.

Counterpart of the reference's ``reference_attention`` (src/pallas_flash/
reference.py:22-66), which plays two roles there: the correctness oracle and
the "what XLA does by default" baseline. Here it is only the baseline (the
parity oracle is the float64 restatement under ``oracle/``, used by the tests).
It materialises the full ``[Sq, Sk]`` score matrix per (batch, head).

Arithmetic follows reference.py:45-66 step by step: GQA by repeating K/V
heads (:49-53); scores = q k^T computed in the input dtype, then upcast to
float32 and scaled (:55), so bf16 inputs give bf16-rounded scores; causal
positions q_pos < k_pos set to -1e30 (:57-62); float32 softmax (:64);
weights times float32 V (:65); cast to q's dtype (:66).
"""

from __future__ import annotations

from typing import Optional

import torch


def reference_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool = False,
                        sm_scale: Optional[float] = None) -> torch.Tensor:
    """Standard scaled dot-product attention with GQA head repetition
    (reference.py:22-66). Returns q's dtype."""
    head_dim = q.shape[-1]
    if sm_scale is None:
        sm_scale = 1.0 / (head_dim ** 0.5)
    num_heads, num_kv_heads = q.shape[1], k.shape[1]
    if num_kv_heads != num_heads:
        rep = num_heads // num_kv_heads
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
    # reference.py:55: the product in the input dtype, then float32. The right
    # operand is made contiguous (a transposed view as the right operand of a
    # batched 16-bit product is avoided on this platform).
    scores = torch.matmul(q, k.transpose(-1, -2).contiguous()).float() * sm_scale
    if causal:
        sq, sk = q.shape[2], k.shape[2]
        keep = torch.arange(sq, device=q.device)[:, None] >= torch.arange(sk, device=q.device)[None, :]
        scores = torch.where(keep, scores, torch.full_like(scores, -1e30))
    weights = torch.softmax(scores, dim=-1)
    return torch.matmul(weights, v.float()).to(q.dtype)


__all__ = ["reference_attention"]

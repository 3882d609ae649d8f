"""FlashAttention with rotary position embeddings fused into the kernel.

Drop-in for the reference's ``pallas_flash.fused_rope.flash_attention_rope``
(src/pallas_flash/fused_rope.py:116-213). Rotation is float32
``x * cos + rotate_half(x) * sin``. Q is rotated in registers inside the HIP
attention kernel; K is rotated exactly once per position by a prologue kernel
into a workspace the attention kernel streams (the reference re-rotates every
K tile for every query head and query block).

Differentiable (a RoPE-aware VJP; the reference is forward-only and tells
training users to apply RoPE outside, README.md:156-157): when q, k or v
requires grad, the forward rotates q and k once (pf_rope), runs the
LSE-saving forward on the rotated tensors and saves them; the backward runs
the standard backward (pf_attn_bwd) and maps dq, dk back through the
transpose of the rotation (pf_rope, inverse): g*cos + rotate_half^T(g*sin),
rotate_half^T([y1, y2]) = [y2, -y1]. That is the VJP for any table, also one
whose halves differ (for precompute_rope's tables it equals the inverse
rotation).

Numerics: the rotated Q and K are rounded once to the input dtype before the
bf16/f16 MFMA (the reference keeps them in float32 and runs a float32 dot,
fused_rope.py:75-78); float32 inputs keep float32 throughout.

A head_dim that is not a kernel size (64, 128, or 256 for bfloat16/float16)
is zero-padded half by half to the next one (each element keeps its rotation
partner) and mixed dtypes compute in float32 (``_shape``).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from ._shape import compute_dtype, kernel_head_dim, pad_head_dim, pad_rope_halves, restore


def _table(t: torch.Tensor, device) -> torch.Tensor:
    # The kernel reads float32 tables; upcasting bf16/f16 tables is exact.
    return t.to(device=device, dtype=torch.float32).contiguous()


def _rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, inverse: bool) -> torch.Tensor:
    """Rows s of x [B, H, S, D] rotated with table row s (pf_rope)."""
    out = torch.empty_like(x)
    if x.numel() == 0:
        return out
    B, H, S, D = x.shape
    args = _lib.RopeArgs(_lib.ptr(x), _lib.ptr(out), _lib.ptr(cos), _lib.ptr(sin), B, H, S, D, cos.shape[0],
                         int(inverse), _lib.dtype_tag(x))
    with torch.cuda.device(x.device):
        _lib.check(_lib.lib().pf_rope(args, _lib.stream_of(x)), "rope")
    return out


class _RopeFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, q_cos, q_sin, k_cos, k_sin, causal, sm_scale, kv_len):
        from .flash_attention import _fwd
        B, Hq, Sq, D = q.shape
        Hkv, Sk = k.shape[1], k.shape[2]
        ctx.causal, ctx.sm_scale, ctx.kv_len = causal, sm_scale, kv_len
        if any(ctx.needs_input_grad[:3]):
            # Training path: rotate once, keep the rotated q/k, o and LSE.
            q_rot = _rope(q, q_cos, q_sin, False)
            k_rot = _rope(k, k_cos, k_sin, False)
            o, lse = _fwd(q_rot, k_rot, v, causal, sm_scale, kv_len, True)
            ctx.save_for_backward(q_rot, k_rot, v, o, lse, q_cos, q_sin, k_cos, k_sin)
            return o
        o = torch.empty_like(q)
        if o.numel() == 0:
            return o
        base = _lib.FwdArgs(
            _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), None,
            B, Hq, Hkv, Sq, Sk, D, kv_len, int(bool(causal)), float(sm_scale), _lib.dtype_tag(q))
        args = _lib.FwdRopeArgs(base, _lib.ptr(q_cos), _lib.ptr(q_sin), _lib.ptr(k_cos),
                                _lib.ptr(k_sin), None, 0)
        L = _lib.lib()
        nbytes = L.pf_attn_fwd_rope_workspace_size(args)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
        args.workspace = _lib.ptr(ws)
        args.workspace_bytes = nbytes
        with torch.cuda.device(q.device):
            _lib.check(L.pf_attn_fwd_rope(args, _lib.stream_of(q)), "flash_attention_rope")
        return o

    @staticmethod
    def backward(ctx, do):
        from .flash_attention import _bwd
        q_rot, k_rot, v, o, lse, q_cos, q_sin, k_cos, k_sin = ctx.saved_tensors
        dq_rot, dk_rot, dv = _bwd(q_rot, k_rot, v, o, lse, do, ctx.causal, ctx.sm_scale, ctx.kv_len)
        dq = _rope(dq_rot, q_cos, q_sin, True)
        dk = _rope(dk_rot, k_cos, k_sin, True)
        return dq, dk, dv, None, None, None, None, None, None, None


def flash_attention_rope(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_cos: torch.Tensor,
    q_sin: torch.Tensor,
    k_cos: Optional[torch.Tensor] = None,
    k_sin: Optional[torch.Tensor] = None,
    *,
    causal: bool = False,
    sm_scale: Optional[float] = None,
    block_q: int = 128,
    block_k: int = 128,
    kv_len: Optional[int] = None,
    interpret: bool = False,
) -> torch.Tensor:
    """Attention with RoPE applied to Q and K inside the kernel.

    Equivalent to ``flash_attention(apply_rope(q), apply_rope(k), v)`` without
    materialising the rotated Q; the rotated K lives in a transient workspace
    of K's size.

    Args:
        q: ``[batch, num_heads, seq_len_q, head_dim]``.
        k, v: ``[batch, num_kv_heads, seq_len_k, head_dim]``.
        q_cos, q_sin: ``[seq_len_q, head_dim]`` tables for the query positions.
        k_cos, k_sin: ``[seq_len_k, head_dim]``; default to the query tables
            when ``seq_len_k == seq_len_q``.
        causal, sm_scale, kv_len: as ``flash_attention``.
        block_q, block_k, interpret: accepted for compatibility; ignored.
    """
    # fused_rope.py:154-181
    if k_cos is None or k_sin is None:
        if k.shape[2] != q.shape[2]:
            raise ValueError(
                "k_cos/k_sin are required when the key sequence length differs "
                "from the query sequence length")
        k_cos, k_sin = q_cos, q_sin
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be rank-4 [batch, heads, seq, head_dim] arrays")
    batch, num_heads, seq_len_q, head_dim = q.shape
    num_kv_heads, seq_len_k = k.shape[1], k.shape[2]
    if k.shape != v.shape or k.shape[0] != batch or k.shape[3] != head_dim:
        raise ValueError("k and v must share shape, and batch/head_dim with q")
    if num_kv_heads == 0 or num_heads % num_kv_heads != 0:
        raise ValueError(
            f"num_heads ({num_heads}) must be a multiple of num_kv_heads ({num_kv_heads})")
    if head_dim % 2 != 0:
        raise ValueError(f"head_dim must be even for RoPE, got {head_dim}")
    for name, tbl, want in (("q_cos", q_cos, seq_len_q), ("q_sin", q_sin, seq_len_q),
                            ("k_cos", k_cos, seq_len_k), ("k_sin", k_sin, seq_len_k)):
        if tuple(tbl.shape) != (want, head_dim):
            raise ValueError(f"{name} must have shape {(want, head_dim)}, got {tuple(tbl.shape)}")
    if sm_scale is None:
        sm_scale = 1.0 / (head_dim ** 0.5)
    if kv_len is None:
        kv_len = seq_len_k
    elif not 0 < kv_len <= seq_len_k:
        raise ValueError(f"kv_len must be in (0, {seq_len_k}], got {kv_len}")
    _lib.require_device(q, k, v)
    dev = q.device
    cdt = compute_dtype(q, k, v)
    dp = kernel_head_dim(head_dim, cdt)
    tables = [pad_rope_halves(_table(t, dev), dp).contiguous() for t in (q_cos, q_sin, k_cos, k_sin)]
    o = _RopeFn.apply(pad_rope_halves(q.to(cdt), dp).contiguous(), pad_rope_halves(k.to(cdt), dp).contiguous(),
                      pad_head_dim(v.to(cdt), dp).contiguous(), *tables, bool(causal), float(sm_scale),
                      int(kv_len))
    return restore(o, head_dim, q.dtype)


__all__ = ["flash_attention_rope"]

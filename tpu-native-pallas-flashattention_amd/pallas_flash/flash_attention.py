"""FlashAttention forward + backward and single-query decode on MI355X.

Drop-in for the reference's ``pallas_flash.flash_attention`` module
(aabhimittal/TPU-Native-Pallas-FlashAttention,
src/pallas_flash/flash_attention.py): same function names, keyword-only
arguments, defaults and ``ValueError`` conditions. Arrays are torch tensors on
a ROCm device; the arithmetic runs in hand-written HIP kernels for gfx950
reached through the C ABI in ``include/pallas_flash_amd.h``.

* ``flash_attention`` is differentiable in q, k and v (a
  ``torch.autograd.Function``, the counterpart of the reference's
  ``jax.custom_vjp`` at flash_attention.py:448-476). Its backward runs the
  dQ kernel (which also writes delta = rowsum(o * do)) and then the dK/dV
  kernel; dK/dV are summed over each GQA group in float32 before the cast to
  the input dtype (flash_attention.py:433-442).
* ``flash_attention_decode`` (flash_attention.py:555-589) runs a split-KV
  decode kernel that reads each cached K/V byte once. When a gradient is
  requested it routes through ``flash_attention`` instead, as the reference
  does unconditionally.

``block_q``/``block_k`` are accepted for signature compatibility; tile shapes
are chosen by the kernels. ``interpret`` is accepted and ignored: there is no
CPU interpreter here, the HIP kernels always run. Any head_dim up to 256
(bfloat16/float16) or 128 (float32 compute, which mixed dtypes use) and any
mix of input dtypes are accepted (``_shape``: zero-padding to the kernels'
head_dim 64, 128 or 256, float32 compute for mixed dtypes, output in q's
dtype).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from ._shape import adapt, compute_dtype, decode_head_dim, kernel_head_dim, restore, warn_copy


def _validate(q, k, v, kv_len):
    """flash_attention.py:527-545."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be rank-4 [batch, heads, seq, head_dim] arrays")
    batch, num_heads, seq_len_q, head_dim = q.shape
    num_kv_heads, seq_len_k = k.shape[1], k.shape[2]
    if k.shape != v.shape:
        raise ValueError("k and v must have the same shape")
    if k.shape[0] != batch or k.shape[3] != head_dim:
        raise ValueError("q and k/v must share batch and head_dim")
    if num_kv_heads == 0 or num_heads % num_kv_heads != 0:
        raise ValueError(
            f"num_heads ({num_heads}) must be a multiple of num_kv_heads "
            f"({num_kv_heads}) for grouped-query attention")
    if kv_len is None:
        kv_len = seq_len_k
    elif not 0 < kv_len <= seq_len_k:
        raise ValueError(f"kv_len must be in (0, {seq_len_k}], got {kv_len}")
    return int(kv_len)


def _fwd(q, k, v, causal: bool, sm_scale: float, kv_len: int, want_lse: bool):
    B, Hq, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    o = torch.empty_like(q)
    lse = torch.empty((B, Hq, Sq), dtype=torch.float32, device=q.device) if want_lse else None
    if o.numel() == 0:
        if lse is not None:
            lse.zero_()
        return o, lse
    args = _lib.FwdArgs(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(lse),
        B, Hq, Hkv, Sq, Sk, D, kv_len, int(bool(causal)), float(sm_scale), _lib.dtype_tag(q))
    with torch.cuda.device(q.device):
        _lib.check(_lib.lib().pf_attn_fwd(args, _lib.stream_of(q)), "flash_attention forward")
    return o, lse


def _bwd(q, k, v, o, lse, do, causal: bool, sm_scale: float, kv_len: int):
    B, Hq, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    do = do.to(q.dtype).contiguous()
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    if q.numel() == 0:
        return dq.zero_(), dk.zero_(), dv.zero_()
    delta = torch.empty((B, Hq, Sq), dtype=torch.float32, device=q.device)
    args = _lib.BwdArgs(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(do), _lib.ptr(lse),
        _lib.ptr(delta), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv),
        B, Hq, Hkv, Sq, Sk, D, kv_len, int(bool(causal)), float(sm_scale), _lib.dtype_tag(q))
    with torch.cuda.device(q.device):
        _lib.check(_lib.lib().pf_attn_bwd(args, _lib.stream_of(q)), "flash_attention backward")
    return dq, dk, dv


class _FlashAttentionFn(torch.autograd.Function):
    """Counterpart of ``_flash_attention_vjp`` (flash_attention.py:448-476):
    the forward saves (q, k, v, out, lse); the backward recomputes P from LSE."""

    @staticmethod
    def forward(ctx, q, k, v, causal, sm_scale, kv_len):
        want_lse = any(ctx.needs_input_grad[:3])
        o, lse = _fwd(q, k, v, causal, sm_scale, kv_len, want_lse)
        ctx.causal, ctx.sm_scale, ctx.kv_len = causal, sm_scale, kv_len
        if want_lse:
            ctx.save_for_backward(q, k, v, o, lse)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = _bwd(q, k, v, o, lse, do, ctx.causal, ctx.sm_scale, ctx.kv_len)
        return dq, dk, dv, None, None, None


def flash_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    causal: bool = False,
    sm_scale: Optional[float] = None,
    block_q: int = 128,
    block_k: int = 128,
    kv_len: Optional[int] = None,
    interpret: bool = False,
) -> torch.Tensor:
    """FlashAttention on MI355X (reference: flash_attention.py:479-552).

    Args:
        q: ``[batch, num_heads, seq_len_q, head_dim]``.
        k, v: ``[batch, num_kv_heads, seq_len_k, head_dim]``; ``num_kv_heads``
            divides ``num_heads`` (GQA/MQA: query head h reads KV head
            ``h // (num_heads // num_kv_heads)``, never replicated).
        causal: lower-triangular mask ``q_pos >= k_pos``, top-left aligned.
        sm_scale: softmax scale, default ``1 / sqrt(head_dim)``.
        block_q, block_k: accepted for compatibility (tiles are internal).
        kv_len: valid key positions (default ``seq_len_k``); keys at or past it
            are masked and never read.
        interpret: accepted for compatibility; ignored.

    Returns:
        ``[batch, num_heads, seq_len_q, head_dim]`` in q's dtype. Differentiable
        in q, k, v (gradients in each input's dtype).
    """
    kv_len = _validate(q, k, v, kv_len)
    head_dim = q.shape[3]
    if sm_scale is None:
        sm_scale = 1.0 / (head_dim ** 0.5)
    _lib.require_device(q, k, v)
    cdt = compute_dtype(q, k, v)
    dp = kernel_head_dim(head_dim, cdt)
    q2, k2, v2 = (adapt(x, cdt, dp).contiguous() for x in (q, k, v))
    o = _FlashAttentionFn.apply(q2, k2, v2, bool(causal), float(sm_scale), kv_len)
    return restore(o, head_dim, q.dtype)


def flash_attention_with_lse(q, k, v, *, causal=False, sm_scale=None, kv_len=None):
    """Forward only, returning ``(out, lse)`` with lse ``[B, H, Sq]`` float32
    (the residual the reference's forward kernel emits, flash_attention.py:
    192-194, 213; natural log of the scaled scores)."""
    kv_len = _validate(q, k, v, kv_len)
    head_dim = q.shape[3]
    if sm_scale is None:
        sm_scale = 1.0 / (head_dim ** 0.5)
    _lib.require_device(q, k, v)
    cdt = compute_dtype(q, k, v)
    dp = kernel_head_dim(head_dim, cdt)
    q2, k2, v2 = (adapt(x, cdt, dp).contiguous() for x in (q, k, v))
    o, lse = _fwd(q2, k2, v2, bool(causal), float(sm_scale), kv_len, True)
    return restore(o, head_dim, q.dtype), lse


def _decode(q, k_cache, v_cache, cache_len: int, sm_scale: float):
    B, Hq, _, D = q.shape
    Hkv, cap = k_cache.shape[1], k_cache.shape[2]
    o = torch.empty_like(q)
    if o.numel() == 0:
        return o
    args = _lib.DecodeArgs(
        _lib.ptr(q), _lib.ptr(k_cache), _lib.ptr(v_cache), _lib.ptr(o),
        B, Hq, Hkv, cap, D, int(cache_len), float(sm_scale), _lib.dtype_tag(q), None, 0)
    L = _lib.lib()
    ws_bytes = L.pf_attn_decode_workspace_size(args)
    ws = torch.empty(max(int(ws_bytes), 1), dtype=torch.uint8, device=q.device)
    args.workspace = ws.data_ptr()
    args.workspace_bytes = ws.numel()
    with torch.cuda.device(q.device):
        _lib.check(L.pf_attn_decode(args, _lib.stream_of(q)), "flash_attention_decode")
    return o


def flash_attention_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    cache_len: int,
    *,
    sm_scale: Optional[float] = None,
    block_k: int = 128,
    interpret: bool = False,
) -> torch.Tensor:
    """Single-token decode against a fixed-size KV cache
    (reference: flash_attention.py:555-589).

    Args:
        q: ``[batch, num_heads, 1, head_dim]``.
        k_cache, v_cache: ``[batch, num_kv_heads, cache_size, head_dim]``.
        cache_len: valid (written) cache positions; slots past it are never read.
        sm_scale: default ``1 / sqrt(head_dim)``.
        block_k, interpret: accepted for compatibility; ignored.

    Returns:
        ``[batch, num_heads, 1, head_dim]``.
    """
    if q.shape[2] != 1:
        raise ValueError(f"decode expects a single query row, got seq_len_q={q.shape[2]}")
    if any(t.requires_grad for t in (q, k_cache, v_cache)) and torch.is_grad_enabled():
        return flash_attention(q, k_cache, v_cache, causal=False, sm_scale=sm_scale, block_q=1,
                               block_k=block_k, kv_len=cache_len, interpret=interpret)
    cache_len = _validate(q, k_cache, v_cache, cache_len)
    head_dim = q.shape[3]
    if sm_scale is None:
        sm_scale = 1.0 / (head_dim ** 0.5)
    _lib.require_device(q, k_cache, v_cache)
    cdt = compute_dtype(q, k_cache, v_cache)
    dp = decode_head_dim(head_dim, cdt)
    if dp != head_dim or k_cache.dtype != cdt or v_cache.dtype != cdt:
        warn_copy("flash_attention_decode", f"head_dim {head_dim} / dtypes {q.dtype}, {k_cache.dtype}, "
                  f"{v_cache.dtype} are not read in place")
    q2, k2, v2 = (adapt(x, cdt, dp).contiguous() for x in (q, k_cache, v_cache))
    return restore(_decode(q2, k2, v2, cache_len, float(sm_scale)), head_dim, q.dtype)


__all__ = ["flash_attention", "flash_attention_decode", "flash_attention_with_lse"]

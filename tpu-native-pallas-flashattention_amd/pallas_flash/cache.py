"""Decode-loop primitives on device: KV-cache writes and the fused decode step.

The reference builds its decode loop from jnp pieces around the attention
kernel (src/pallas_flash/model.py): ``_cache_write`` (:257-262), the ring slot
``pos % capacity`` and live length ``ring_kv_len`` (:405-413, :475-476), the
ring scatter of ``prefill_ring`` (:437, :447-448), RoPE at the new position
(:340-341, :485-486) and ``flash_attention_decode`` over ``pos + 1`` slots
(:344-347, :488-491). Here each of those is a HIP kernel behind the C ABI
(``pf_kv_cache_write``, ``pf_attn_decode_step``), and positions are read from
device memory: nothing on the host depends on the position, so one captured
decode step (a HIP graph) can be replayed while the caller advances the
positions on the GPU. The caches are updated in place (torch tensors are
mutable; the reference threads new cache arrays through functionally).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib


def ring_kv_len(total_tokens: int, capacity: int) -> int:
    """Live slots after ``total_tokens`` writes into a ring of ``capacity``
    (model.py:405-407)."""
    return min(total_tokens, capacity)


def _check_positions(positions, batch: int) -> Tuple[torch.Tensor, int]:
    """Positions as a 1-D integer tensor and their batch stride (0: one for
    all); raises ValueError before any device work."""
    t = positions if isinstance(positions, torch.Tensor) else torch.as_tensor(positions)
    if t.dim() > 1:
        raise ValueError(f"positions must be a scalar or [batch], got shape {tuple(t.shape)}")
    if t.dtype.is_floating_point or t.dtype.is_complex or t.dtype == torch.bool:
        raise ValueError(f"positions must be integers, got {t.dtype}")
    t = t.reshape(-1)
    if t.numel() == 1:
        return t, 0
    if t.numel() == batch:
        return t, 1
    raise ValueError(f"positions must hold 1 or batch={batch} entries, got {t.numel()}")


def _positions(positions, batch: int, device) -> Tuple[torch.Tensor, int]:
    """Device int32 positions and their batch stride (0: one for all). A
    contiguous int32 tensor already on ``device`` is used as is (no copy: the
    call stays capturable)."""
    t, stride = _check_positions(positions, batch)
    if t.device != device or t.dtype != torch.int32:
        t = t.to(device=device, dtype=torch.int32)
    return t.contiguous(), stride


def write_kv_cache(k_cache: torch.Tensor, v_cache: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   positions, *, ring: bool = False, inplace: bool = True):
    """Write rows of ``k``/``v`` into a contiguous KV cache (in place by default).

    ``_cache_write`` (model.py:257-262) for ``ring=False``: row ``i`` of batch
    ``b`` goes to slot ``positions[b] + i``; rows past the capacity are not
    written. With ``ring=True`` (prefill_ring / ring_decode_step,
    model.py:437, :447-448, :475): slot ``(positions[b] + i) % capacity``, and
    only the last ``capacity`` rows are written (the ones a ring keeps).

    Args:
        k_cache, v_cache: ``[batch, num_kv_heads, capacity, head_dim]``.
        k, v: ``[batch, num_kv_heads, seq_len, head_dim]`` (cast to the cache dtype).
        positions: absolute position of row 0: an int, or ``[batch]`` integers
            (a device tensor keeps the call free of host-side data).
        inplace: ``True`` writes into ``k_cache``/``v_cache`` and returns
            them; ``False`` leaves them unchanged and returns written copies,
            as the reference's functional ``dynamic_update_slice`` does (one
            cache-sized device copy per call).

    Returns ``(k_cache, v_cache)``: the given tensors, or the new ones.
    """
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must be [batch, num_kv_heads, capacity, head_dim] of one shape")
    if k.dim() != 4 or k.shape != v.shape:
        raise ValueError("k and v must be [batch, num_kv_heads, seq_len, head_dim] of one shape")
    batch, hkv, cap, d = k_cache.shape
    if k.shape[0] != batch or k.shape[1] != hkv or k.shape[3] != d:
        raise ValueError(f"k {tuple(k.shape)} does not match the cache {tuple(k_cache.shape)}")
    if k_cache.dtype != v_cache.dtype:
        raise ValueError("k_cache and v_cache must share a dtype")
    _check_positions(positions, batch)
    _lib.require_device(k_cache, v_cache, k, v)
    if not inplace:
        k_cache, v_cache = (t.clone(memory_format=torch.contiguous_format) for t in (k_cache, v_cache))
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("the caches are written in place and must be contiguous")
    dev = k_cache.device
    pos, stride = _positions(positions, batch, dev)
    k = k.to(k_cache.dtype).contiguous()
    v = v.to(k_cache.dtype).contiguous()
    args = _lib.KvWriteArgs(_lib.ptr(k), _lib.ptr(v), _lib.ptr(k_cache), _lib.ptr(v_cache), _lib.ptr(pos),
                            stride, batch, hkv, k.shape[2], cap, d, int(bool(ring)),
                            _lib.dtype_tag(k_cache))
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().pf_kv_cache_write(args, _lib.stream_of(k_cache)), "write_kv_cache")
    return k_cache, v_cache


def flash_attention_decode_step(
    q: torch.Tensor,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    positions,
    cos: Optional[torch.Tensor] = None,
    sin: Optional[torch.Tensor] = None,
    *,
    ring: bool = False,
    sm_scale: Optional[float] = None,
) -> torch.Tensor:
    """One decode step of a layer's attention, fused on device.

    The attention part of ``decode_step`` / ``ring_decode_step``
    (model.py:340-347, :485-491): rotate the new token's ``q`` and ``k`` with
    RoPE at its position, write ``k``/``v`` into the cache slot, and attend
    the single query over the live slots -- ``[0, pos]`` (``ring=False``) or
    the last ``min(pos + 1, capacity)`` tokens of a ring (``ring=True``, slot
    ``pos % capacity``). The caches are updated in place. The fused step is
    the streaming decode kernel's mode for bfloat16/float16 at head_dim 128
    (the reference model's); other dtypes or head dims raise
    NotImplementedError -- compose ``write_kv_cache`` (after rotating the
    new rows) and ``flash_attention_decode`` for them.

    Args:
        q: ``[batch, num_heads, 1, head_dim]``, before RoPE.
        k_new, v_new: ``[batch, num_kv_heads, 1, head_dim]``, ``k_new`` before RoPE.
        k_cache, v_cache: ``[batch, num_kv_heads, capacity, head_dim]``.
        positions: absolute position of the new token: an int, or ``[batch]``
            integers; pass a device int32 tensor to keep the step capturable.
            With ``ring=False`` a host-side position ``>= capacity`` raises
            ``ValueError`` (as decode_step, model.py:329-331); in device
            memory, an out-of-range position (``ring=False``: outside
            ``[0, capacity)``; any: negative, or past the RoPE table) writes
            nothing and yields zeros for that batch.
        cos, sin: ``[rope_len, head_dim]`` tables (``precompute_rope``), or
            both ``None`` for no rotation.
        sm_scale: default ``1 / sqrt(head_dim)``.

    Returns:
        ``[batch, num_heads, 1, head_dim]`` in q's dtype.
    """
    if q.dim() != 4 or q.shape[2] != 1:
        raise ValueError(f"decode step expects q of shape [batch, heads, 1, head_dim], got {tuple(q.shape)}")
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must be [batch, num_kv_heads, capacity, head_dim] of one shape")
    batch, hq, _, d = q.shape
    _, hkv, cap, dc = k_cache.shape
    if k_cache.shape[0] != batch or dc != d:
        raise ValueError(f"q {tuple(q.shape)} does not match the cache {tuple(k_cache.shape)}")
    if tuple(k_new.shape) != (batch, hkv, 1, d) or tuple(v_new.shape) != (batch, hkv, 1, d):
        raise ValueError(f"k_new and v_new must be [{batch}, {hkv}, 1, {d}]")
    if hkv == 0 or hq % hkv != 0:
        raise ValueError(f"num_heads ({hq}) must be a multiple of num_kv_heads ({hkv})")
    if (cos is None) != (sin is None):
        raise ValueError("pass both cos and sin, or neither")
    if cos is not None and (cos.dim() != 2 or cos.shape != sin.shape or cos.shape[1] != d):
        raise ValueError(f"cos/sin must be [rope_len, {d}] of one shape")
    for t in (k_new, v_new, k_cache, v_cache):
        if t.dtype != q.dtype:
            raise ValueError("q, k_new, v_new and the caches must share a dtype")
    if sm_scale is None:
        sm_scale = 1.0 / (d ** 0.5)
    pos_t, _ = _check_positions(positions, batch)
    if not ring and pos_t.device.type == "cpu" and pos_t.numel() and int(pos_t.max()) >= cap:
        # decode_step's host check (model.py:329-331); positions in device
        # memory are not read back (that would sync) -- the kernel skips them.
        raise ValueError(f"position {int(pos_t.max())} exceeds cache capacity {cap}")
    tensors = [q, k_new, v_new, k_cache, v_cache] + ([cos, sin] if cos is not None else [])
    _lib.require_device(*tensors)
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("the caches are written in place and must be contiguous")
    dev = q.device
    pos, stride = _positions(positions, batch, dev)
    q, k_new, v_new = q.contiguous(), k_new.contiguous(), v_new.contiguous()
    if cos is not None:
        cos = cos.to(torch.float32).contiguous()
        sin = sin.to(torch.float32).contiguous()
    o = torch.empty_like(q)
    if batch == 0:
        return o
    args = _lib.DecodeStepArgs(
        _lib.ptr(q), _lib.ptr(k_new), _lib.ptr(v_new), _lib.ptr(k_cache), _lib.ptr(v_cache), _lib.ptr(o),
        _lib.ptr(pos), stride, _lib.ptr(cos), _lib.ptr(sin), 0 if cos is None else cos.shape[0],
        batch, hq, hkv, cap, d, int(bool(ring)), float(sm_scale), _lib.dtype_tag(q), None, 0)
    L = _lib.lib()
    with torch.cuda.device(dev):
        ws_bytes = L.pf_attn_decode_step_workspace_size(args)
        if ws_bytes == 0:
            # the same validation as the launch: reports the reason
            _lib.check(L.pf_attn_decode_step(args, _lib.stream_of(q)), "flash_attention_decode_step")
        ws = torch.empty(int(ws_bytes), dtype=torch.uint8, device=dev)
        args.workspace = ws.data_ptr()
        args.workspace_bytes = ws.numel()
        _lib.check(L.pf_attn_decode_step(args, _lib.stream_of(q)), "flash_attention_decode_step")
    return o


__all__ = ["ring_kv_len", "write_kv_cache", "flash_attention_decode_step"]

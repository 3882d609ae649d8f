"""Paged attention on MI355X: single-query attention over a page pool.

Drop-in for the reference's ``pallas_flash.paged`` (src/pallas_flash/paged.py).
Layout, as in the reference:

    k_pages / v_pages : [num_pages, num_kv_heads, page_size, head_dim]
    block_tables      : [batch, pages_per_seq]  int32  (logical -> physical page)
    context_lens      : [batch]                 int32  (valid tokens per sequence)

The HIP kernel reads the block table from device memory, so page gathering is
address arithmetic inside the kernel. Each KV head's pages are streamed once
for all query heads of its GQA group (the reference re-reads them per query
head). Table entries for logical pages at or past ``ceil(len / page_size)``
are never read, so ``-1`` padding is legal (the reference documents that its
unused entries must be valid indices because its DMA address is formed
regardless, paged.py:119-121).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from ._shape import adapt, compute_dtype, decode_head_dim, restore, warn_copy


def paged_flash_attention(
    q: torch.Tensor,
    k_pages: torch.Tensor,
    v_pages: torch.Tensor,
    block_tables,
    context_lens,
    *,
    sm_scale: Optional[float] = None,
    interpret: bool = False,
) -> torch.Tensor:
    """Single-query attention over a paged KV cache (reference: paged.py:102-192).

    Args:
        q: ``[batch, num_heads, 1, head_dim]``.
        k_pages, v_pages: ``[num_pages, num_kv_heads, page_size, head_dim]``.
        block_tables: ``[batch, pages_per_seq]`` integer table (cast to int32).
        context_lens: ``[batch]`` valid tokens per sequence (cast to int32). A
            sequence attends ``min(len, pages_per_seq * page_size)`` tokens;
            a non-positive length yields zeros.
        sm_scale: default ``1 / sqrt(head_dim)``.
        interpret: accepted for compatibility; ignored.

    Returns:
        ``[batch, num_heads, 1, head_dim]`` in q's dtype. Any head_dim up to
        256 that is a multiple of 8 (bfloat16/float16), or up to 128 that is
        a multiple of 4 (float32), is read in place; other head dims and
        mixed dtypes copy the pool padded/cast per call, with a one-time
        warning (``_shape``).
    """
    # paged.py:129-149
    if q.dim() != 4 or q.shape[2] != 1:
        raise ValueError(
            f"paged attention expects q of shape [batch, heads, 1, head_dim], got {tuple(q.shape)}")
    if k_pages.shape != v_pages.shape:
        raise ValueError("k_pages and v_pages must have the same shape")
    if k_pages.dim() != 4:
        raise ValueError("k_pages must be [num_pages, num_kv_heads, page_size, head_dim]")
    batch, num_heads, _, head_dim = q.shape
    num_pages, num_kv_heads, page_size, k_head_dim = k_pages.shape
    if k_head_dim != head_dim:
        raise ValueError("q and pages must share head_dim")
    if num_kv_heads == 0 or num_heads % num_kv_heads != 0:
        raise ValueError(
            f"num_heads ({num_heads}) must be a multiple of num_kv_heads ({num_kv_heads})")
    block_tables = torch.as_tensor(block_tables)
    context_lens = torch.as_tensor(context_lens)
    if block_tables.dim() != 2 or block_tables.shape[0] != batch:
        raise ValueError(
            f"block_tables must be [batch, pages_per_seq], got {tuple(block_tables.shape)}")
    if tuple(context_lens.shape) != (batch,):
        raise ValueError(f"context_lens must be [batch], got {tuple(context_lens.shape)}")
    if sm_scale is None:
        sm_scale = 1.0 / (head_dim ** 0.5)
    _lib.require_device(q, k_pages, v_pages)
    dev = q.device
    tables = block_tables.to(device=dev, dtype=torch.int32).contiguous()
    lens = context_lens.to(device=dev, dtype=torch.int32).contiguous()
    out_dtype = q.dtype
    cdt = compute_dtype(q, k_pages, v_pages)
    dp = decode_head_dim(head_dim, cdt)
    if dp != head_dim or k_pages.dtype != cdt or v_pages.dtype != cdt:
        warn_copy("paged_flash_attention", f"head_dim {head_dim} / dtypes {q.dtype}, {k_pages.dtype}, "
                  f"{v_pages.dtype} are not read in place")
    q, k_pages, v_pages = (adapt(x, cdt, dp).contiguous() for x in (q, k_pages, v_pages))
    o = torch.empty_like(q)
    if batch == 0:
        return restore(o, head_dim, out_dtype)
    args = _lib.PagedArgs(
        _lib.ptr(q), _lib.ptr(k_pages), _lib.ptr(v_pages), _lib.ptr(tables), _lib.ptr(lens),
        _lib.ptr(o), batch, num_heads, num_kv_heads, num_pages, page_size, dp,
        tables.shape[1], float(sm_scale), _lib.dtype_tag(q), None, 0)
    L = _lib.lib()
    ws_bytes = L.pf_paged_attn_workspace_size(args)
    ws = torch.empty(max(int(ws_bytes), 1), dtype=torch.uint8, device=dev)
    args.workspace = ws.data_ptr()
    args.workspace_bytes = ws.numel()
    with torch.cuda.device(dev):
        _lib.check(L.pf_paged_attn(args, _lib.stream_of(q)), "paged_flash_attention")
    return restore(o, head_dim, out_dtype)


def init_paged_cache(num_pages: int, num_kv_heads: int, page_size: int, head_dim: int,
                     dtype=torch.float32, device=None):
    """Allocate an empty page pool ``(k_pages, v_pages)`` (paged.py:198-202)."""
    shape = (num_pages, num_kv_heads, page_size, head_dim)
    return (torch.zeros(shape, dtype=dtype, device=device),
            torch.zeros(shape, dtype=dtype, device=device))


def write_to_paged_cache(k_pages, v_pages, k, v, block_table, position, *, inplace: bool = True):
    """Write token K/V into the pages holding their positions
    (paged.py:205-223), on device (pf_paged_cache_write), in place by default.

    The reference writes one token of one sequence: ``k``/``v``
    ``[1, num_kv_heads, 1, head_dim]``, ``block_table`` ``[pages_per_seq]``,
    ``position`` an int. The same call also takes a batch: ``k``/``v``
    ``[batch, num_kv_heads, seq_len, head_dim]``, ``block_table``
    ``[batch, pages_per_seq]`` and ``position`` an int or ``[batch]``
    integers (row ``i`` of sequence ``b`` goes to position
    ``position[b] + i``). A row whose position falls outside the table, or
    whose table entry is not a page of the pool (e.g. ``-1`` padding), is not
    written (the reference's dynamic_update_slice would clamp it onto a valid
    slot).

    Returns the updated ``(k_pages, v_pages)``: with ``inplace=True``
    (default) the same tensors, written in place, so the reference's
    functional call pattern keeps working without a pool copy; with
    ``inplace=False`` written copies, the given pools left unchanged, as the
    reference's functional update leaves them (one pool-sized device copy
    per call: for callers that keep the pre-write pool, e.g. to roll back
    speculative tokens).
    """
    from .cache import _check_positions, _positions
    if k_pages.dim() != 4 or k_pages.shape != v_pages.shape:
        raise ValueError("k_pages and v_pages must be [num_pages, num_kv_heads, page_size, head_dim] of one shape")
    if k.dim() != 4 or k.shape != v.shape:
        raise ValueError("k and v must be [batch, num_kv_heads, seq_len, head_dim] of one shape")
    num_pages, hkv, page_size, d = k_pages.shape
    batch = k.shape[0]
    if k.shape[1] != hkv or k.shape[3] != d:
        raise ValueError(f"k {tuple(k.shape)} does not match the pool {tuple(k_pages.shape)}")
    if k_pages.dtype != v_pages.dtype:
        raise ValueError("k_pages and v_pages must share a dtype")
    table = torch.as_tensor(block_table)
    if table.dim() == 1:
        table = table.unsqueeze(0)
    if table.dim() != 2 or table.shape[0] != batch:
        raise ValueError(f"block_table must be [pages_per_seq] or [batch, pages_per_seq], got {tuple(table.shape)}")
    _check_positions(position, batch)
    _lib.require_device(k_pages, v_pages, k, v)
    if not inplace:
        k_pages, v_pages = (t.clone(memory_format=torch.contiguous_format) for t in (k_pages, v_pages))
    if not (k_pages.is_contiguous() and v_pages.is_contiguous()):
        raise ValueError("the page pools are written in place and must be contiguous")
    dev = k_pages.device
    table = table.to(device=dev, dtype=torch.int32).contiguous()
    pos, stride = _positions(position, batch, dev)
    k = k.to(k_pages.dtype).contiguous()
    v = v.to(k_pages.dtype).contiguous()
    args = _lib.PagedWriteArgs(_lib.ptr(k), _lib.ptr(v), _lib.ptr(k_pages), _lib.ptr(v_pages), _lib.ptr(table),
                               _lib.ptr(pos), stride, batch, hkv, k.shape[2], num_pages, page_size, d,
                               table.shape[1], _lib.dtype_tag(k_pages))
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().pf_paged_cache_write(args, _lib.stream_of(k_pages)), "write_to_paged_cache")
    return k_pages, v_pages


__all__ = ["paged_flash_attention", "init_paged_cache", "write_to_paged_cache"]

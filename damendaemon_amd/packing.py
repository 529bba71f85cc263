"""GPU ragged-batch packer and K/V page writer.

``pack_batch`` replaces the host-side packing of damendaemon/paged.py:149-159
(flat ``positions``/``slot_ids`` built by list comprehensions), the
``accumulate(lengths)`` segment ends of paged.py:118-120 and the physical
slot computation of kernels.py:279-281: the host uploads one (3, n) int64
array of (length, start, slot) per segment and the GPU expands it.
"""
from dataclasses import dataclass

import numpy as np
import torch

from . import _native
from ._native import call, ptr


@dataclass
class PackedBatch:
    """Device outputs of ``pack_batch`` (int64 unless noted) plus host sizes."""
    cu_seqlens: torch.Tensor      # (n+1,)
    ends: torch.Tensor            # (n,)  last token of each segment
    context_lens: torch.Tensor    # (n,)  start + length
    positions: torch.Tensor       # (T,)
    slot_ids: torch.Tensor        # (T,)
    slot_map: torch.Tensor        # (T,)  physical page * P + offset, or None
    cu_pages: torch.Tensor        # (n+1,) int32, or None
    gather_pages: torch.Tensor    # (total_pages,) int32, or None
    lengths: list
    starts: list
    slots: list
    total_tokens: int
    page_size: int


def pack_batch(lengths, starts, slots, page_table=None, page_size=16, device='cuda', gather=True):
    """Pack n segments (len_i tokens appended after start_i cached tokens of slot_i).

    ``lengths``, ``starts`` and ``slots`` are host integer sequences (the
    scheduler's own lists).  With a ``page_table`` the slot map and the page
    gather lists are produced too.
    """
    try:
        host = np.array((lengths, starts, slots), dtype=np.int64)
    except (TypeError, ValueError, OverflowError):
        raise ValueError('invalid packing request') from None
    if host.ndim != 2 or page_size <= 0 or (host[:2] < 0).any():
        raise ValueError('invalid packing request')
    n = host.shape[1]
    lengths, starts, slots = host.tolist()
    total = int(host[0].sum())
    pages = int(((host[0] + host[1] + (page_size - 1)) // page_size).sum())
    dev = torch.device(device)
    meta = torch.from_numpy(host)
    meta = _native.upload(meta, dev) if dev.type == 'cuda' else meta.to(dev)
    _native.require_device(meta, page_table)
    if page_table is not None and (page_table.dtype != torch.int32 or not page_table.is_contiguous()):
        raise ValueError('page table must be a contiguous int32 matrix')
    i64 = dict(dtype=torch.int64, device=dev)
    out = PackedBatch(
        cu_seqlens=torch.empty(n + 1, **i64), ends=torch.empty(n, **i64), context_lens=torch.empty(n, **i64),
        positions=torch.empty(total, **i64), slot_ids=torch.empty(total, **i64),
        slot_map=torch.empty(total, **i64) if page_table is not None else None,
        cu_pages=torch.empty(n + 1, dtype=torch.int32, device=dev) if page_table is not None and gather else None,
        gather_pages=torch.empty(pages, dtype=torch.int32, device=dev) if page_table is not None and gather else None,
        lengths=lengths, starts=starts, slots=slots, total_tokens=total, page_size=page_size)
    call('dd_pack_batch', ptr(meta[0]), ptr(meta[1]), ptr(meta[2]), n, total, pages if out.gather_pages is not None else 0,
         ptr(page_table), 0 if page_table is None else page_table.shape[0],
         0 if page_table is None else page_table.shape[1], page_size,
         ptr(out.cu_seqlens), ptr(out.ends), ptr(out.context_lens), ptr(out.positions), ptr(out.slot_ids),
         ptr(out.slot_map), ptr(out.cu_pages), ptr(out.gather_pages), _native.stream_of(meta))
    out._meta = meta  # keep the uploaded metadata alive until the kernels ran
    return out


def store_kv_pages(key, value, slot_map, cache_k, cache_v, k_scale=None, v_scale=None):
    """Write (T, KH, D) keys/values into their page slots.

    bf16/fp16/fp32 caches take the rows as they are (cast to the cache dtype
    first); int8 caches (with fp16 ``k_scale``/``v_scale`` (..., page, D/group))
    quantise each row group to Q8_0 on the way in.
    """
    tokens, kv_heads, dim = key.shape
    capacity, kvh, page, cdim = cache_k.shape
    if (value.shape != key.shape or kvh != kv_heads or cdim != dim or slot_map.shape != (tokens,)
            or cache_v.shape != cache_k.shape or not cache_k.is_contiguous() or not cache_v.is_contiguous()):
        raise ValueError('incompatible K/V page write shapes')
    _native.require_device(key, value, slot_map, cache_k, cache_v)
    slot_map = slot_map.to(torch.int64)
    if cache_k.dtype == torch.int8:
        if k_scale is None or v_scale is None or k_scale.shape[:-1] != cache_k.shape[:-1] or dim % k_scale.shape[-1]:
            raise ValueError('int8 pages need fp16 scales (..., page, dim/group)')
        key, value = key.contiguous(), value.contiguous()
        call('dd_store_kv_pages_q8', ptr(key), ptr(value), _native.DTYPE_CODES[key.dtype], ptr(slot_map), tokens,
             kv_heads, dim, dim // k_scale.shape[-1], page, capacity, ptr(cache_k), ptr(cache_v), ptr(k_scale),
             ptr(v_scale), _native.stream_of(key))
        return
    key = key.to(cache_k.dtype).contiguous()
    value = value.to(cache_k.dtype).contiguous()
    call('dd_store_kv_pages', ptr(key), ptr(value), cache_k.element_size(), ptr(slot_map), tokens, kv_heads, dim,
         page, capacity, ptr(cache_k), ptr(cache_v), _native.stream_of(key))

"""Bulk copy between physical KV pages and dense snapshots (damendaemon/paged_kernels.py:28-47)."""
import torch

from . import _native
from ._native import call, ptr


def copy_pages(cache, table, slot, tokens, snapshot=None):
    """Gather when ``snapshot`` is absent; otherwise restore exactly its live tokens.

    cache (2, capacity, KH, page, D); returns the (2, KH, tokens, D) dense
    gather, or writes ``snapshot`` back into the pages and returns it.  The
    executor owns page admission and must allocate all destination pages
    before calling; unused entries and the tail of the last page are untouched.
    """
    if (cache.ndim != 5 or cache.shape[0] != 2 or not cache.is_contiguous()
            or type(slot) is not int or not 0 <= slot < table.shape[0]
            or type(tokens) is not int or not 0 < tokens <= table.shape[1] * cache.shape[-2]):
        raise ValueError('invalid paged copy shape')
    shape = (2, cache.shape[2], tokens, cache.shape[4])
    restore = snapshot is not None
    if restore:
        if (snapshot.shape != shape or snapshot.dtype != cache.dtype or snapshot.device != cache.device
                or not snapshot.is_contiguous()):
            raise ValueError('invalid KV snapshot')
    else:
        snapshot = torch.empty(shape, dtype=cache.dtype, device=cache.device)
    _native.require_device(cache, table)
    if table.dtype != torch.int32 or not table.is_contiguous():
        raise ValueError('page table must be a contiguous int32 matrix')
    call('dd_copy_pages', ptr(cache), ptr(table), table.shape[0], table.shape[1], ptr(snapshot),
         cache.element_size(), slot, tokens, cache.shape[1], cache.shape[2], cache.shape[3], cache.shape[4],
         int(restore), _native.stream_of(cache))
    return snapshot

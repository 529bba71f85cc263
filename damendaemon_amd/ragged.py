"""Attention over one packed continuous batch: chunked prefill + decode rows.

The reference runs a prefill chunk as copy_pages (gather start+len tokens
into a dense tensor, damendaemon/paged.py:101-104) followed by torch SDPA
with a lower-right causal mask (qwen2.py:756-770), and decodes through
``kernels.attention`` in a separate forward pass (scheduler.py:822-873).
Here one packed token buffer (from ``packing.pack_batch``) is attended in
place: multi-token segments by the paged MFMA prefill kernel, the trailing
run of single-token segments by the split-KV decode kernel.  Both read the
pages directly; nothing is gathered.
"""
import ctypes
import math
import os

import numpy as np
import torch

from . import _native, kernels
from ._native import DTYPE_CODES, call, ptr


def _check(query, cache_k, cache_v, page_table):
    if query.ndim == 4:
        query = query.reshape(query.shape[0], query.shape[1], query.shape[3])
    T, H, D = query.shape
    capacity, KH, page, kd = cache_k.shape
    if (kd != D or cache_v.shape != cache_k.shape or H % KH or cache_k.dtype != query.dtype
            or cache_v.dtype != query.dtype or query.dtype not in (torch.bfloat16, torch.float16, torch.float32)):
        raise ValueError('prefill attention needs bf16/fp16/fp32 query and pages of one dtype and head size')
    if not (query.is_contiguous() and cache_k.is_contiguous() and cache_v.is_contiguous()):
        raise ValueError('prefill attention needs contiguous tensors')
    if page_table.dtype != torch.int32 or page_table.ndim != 2 or not page_table.is_contiguous():
        raise ValueError('page table must be a contiguous int32 matrix')
    _native.require_device(query, cache_k, cache_v, page_table)
    return query


def _has_mfma_geometry(dim, group):
    """Whether the 16-bit MFMA prefill kernels take this head size and number
    of query heads per KV head (then the call carries a workgroup plan)."""
    cols, keys = ctypes.c_int(0), ctypes.c_int(0)
    ok = _native.library().dd_prefill_geometry(int(dim), ctypes.byref(cols), ctypes.byref(keys)) == 0
    return ok and cols.value >= group


def prefill_plan(lengths, starts, heads, kv_heads, dim, window=0, slots=None, workgroups=0):
    """Schedule of the prefill kernel for these segments: a host int32 array
    (entries, 8), each row (item or -1, first packed token, length, start,
    slot, rounds, 0, 0); entry r * G + b is round r of workgroup b.

    Balances (segment, KV head, query tile) items over the XCDs, longest
    first, from the host copies of the segment lengths, starts and slots
    (slots default to 0 .. n-1).  ``workgroups`` > 0 (the number of CUs)
    gives each of at most that many workgroups a list of items to run in
    turn; 0 gives one item per workgroup.
    """
    lengths = np.ascontiguousarray(lengths, dtype=np.int64)
    starts = np.ascontiguousarray(starts, dtype=np.int64)
    slots = np.ascontiguousarray(np.arange(len(lengths)) if slots is None else slots, dtype=np.int64)
    if lengths.shape != starts.shape or lengths.shape != slots.shape or lengths.ndim != 1:
        raise ValueError('lengths, starts and slots must be matching 1-D sequences')
    lib = _native.library()
    args = (lengths.ctypes.data_as(ctypes.c_void_p), starts.ctypes.data_as(ctypes.c_void_p),
            slots.ctypes.data_as(ctypes.c_void_p), len(lengths), heads, kv_heads, dim, int(window or 0),
            int(workgroups))
    need = lib.dd_prefill_plan(*args, None, 0)
    if need < 0:
        raise _native.NativeError(f'dd_prefill_plan failed: {lib.dd_error_string(-need).decode()} ({-need})')
    plan = np.empty((max(need, 1), PLAN_INTS), dtype=np.int32)
    got = lib.dd_prefill_plan(*args, plan.ctypes.data_as(ctypes.c_void_p), len(plan))
    if got != need:
        raise _native.NativeError('dd_prefill_plan returned an inconsistent length')
    return plan[:need]


PLAN_INTS = 8   # DD_PREFILL_PLAN_INTS


def prefill_attention(query, cache_k, cache_v, packed, page_table, window=0, scale=None, out=None,
                      segments=None, flags=None):
    """Causal attention of every packed query token over its slot's pages.

    query (T, H, D) or (T, H, 1, D); ``packed`` from ``pack_batch``; the
    chunk's own K/V must already be in the pages.  ``segments`` (a, b)
    restricts the work to segments a..b-1 (their tokens only).  ``flags``
    (optional, int32 on the device, at least ``prefill_flag_count`` entries)
    receives the bf16 kernel's per-item re-run flags; by default the call
    allocates them.
    """
    return prepare_prefill(query, cache_k, cache_v, packed, page_table, window, scale, out, segments, flags).run()


def prepare_prefill(query, cache_k, cache_v, packed, page_table, window=0, scale=None, out=None, segments=None,
                    flags=None):
    """Validate a prefill call, compute and upload its workgroup plan, and
    return a ``PrefillLaunch`` whose ``run()`` only enqueues the kernels
    (arguments and errors as ``prefill_attention``)."""
    q = _check(query, cache_k, cache_v, page_table)
    T, H, D = q.shape
    scale = float(D ** -.5 if scale is None else scale)
    if not math.isfinite(scale):
        raise ValueError('prefill attention needs a finite scale')
    if out is None:
        out = torch.empty_like(q)
    else:
        if (out.dtype != q.dtype or out.device != q.device or out.numel() != q.numel()
                or not out.is_contiguous()):
            raise ValueError('out must be a contiguous tensor of the query dtype, device and size')
        out = out.view(q.shape)
    a, b = segments if segments is not None else (0, len(packed.lengths))
    if b <= a:
        return PrefillLaunch(out, None)
    max_len = max(packed.lengths[a:b])
    max_context = max(s + n for s, n in zip(packed.starts[a:b], packed.lengths[a:b]))
    plan_dev, plan_len = None, 0
    if q.dtype != torch.float32 and scale != 0.0 and _has_mfma_geometry(D, H // cache_k.shape[1]):
        # the MFMA kernel's XCD-balanced workgroup order (the fp32 / other-D
        # kernel takes none)
        plan = prefill_plan(packed.lengths[a:b], packed.starts[a:b], H, cache_k.shape[1], D, window,
                            packed.slots[a:b], _persistent_workgroups(q.device, D))
        if len(plan) == 0:
            return PrefillLaunch(out, None)
        plan_dev = _native.upload(torch.from_numpy(plan), q.device)
        plan_len = len(plan) // int(plan[0, 5])     # workgroups
    n_flags = prefill_flag_count(b - a, max_len, H, cache_k.shape[1], D, q.dtype)
    # per-item exactness flags of the bf16 kernel (written by the kernel itself)
    if flags is not None:
        if flags.dtype != torch.int32 or flags.device != q.device or flags.numel() < n_flags:
            raise ValueError(f'flags must be int32 on the query device with at least {n_flags} entries')
    elif n_flags:
        flags = torch.empty(n_flags, dtype=torch.int32, device=q.device)
    args = (ptr(q), ptr(cache_k), ptr(cache_v), DTYPE_CODES[q.dtype],
            ptr(packed.cu_seqlens[a:]), ptr(packed.context_lens[a:]), ptr(packed._meta[2, a:]), b - a, max_len,
            max_context, ptr(page_table), page_table.shape[0], page_table.shape[1], H, cache_k.shape[1], D,
            cache_k.shape[2], cache_k.shape[0], int(window or 0), scale,
            ptr(plan_dev) if plan_dev is not None else None, plan_len, ptr(flags), ptr(out))
    return PrefillLaunch(out, args, keep=(q, cache_k, cache_v, packed, page_table, plan_dev, flags))


class PrefillLaunch:
    """One validated prefill launch (plan uploaded, output and flags
    allocated); ``run()`` enqueues it on the current stream and returns the
    output.  Repeated runs reuse the same buffers."""

    def __init__(self, out, args, keep=()):
        self.out, self._args, self._keep = out, args, keep

    def run(self):
        if self._args is not None:
            call('dd_prefill_attention', *self._args,
                 ctypes.c_void_p(torch.cuda.current_stream(self.out.device).cuda_stream))
        return self.out

    def phase(self, which):
        """Enqueue one launch of the call: 1 the attention kernel, 2 the exact
        re-run of the items the bf16 kernel flagged (both together = run())."""
        if self._args is not None:
            call('dd_prefill_attention_phase', *self._args, int(which),
                 ctypes.c_void_p(torch.cuda.current_stream(self.out.device).cuda_stream))
        return self.out


_CU_COUNT = {}


def _persistent_workgroups(device, dim):
    """Workgroup count for a persistent prefill schedule: one per CU for the
    kernel that runs its items in turn (head sizes up to 128, and 256), else 0."""
    if dim > 256:
        return 0
    forced = os.environ.get('DAMENDAEMON_AMD_PREFILL_WORKGROUPS')   # tuning: 0 = one item per workgroup
    if forced is not None:
        return int(forced)
    index = torch.device(device).index
    index = torch.cuda.current_device() if index is None else index
    if index not in _CU_COUNT:
        _CU_COUNT[index] = torch.cuda.get_device_properties(index).multi_processor_count
    return _CU_COUNT[index]


def prefill_flag_count(segments, max_len, heads, kv_heads, dim, dtype):
    """Entries of the re-run flag workspace a prefill call needs (0: none)."""
    lib = _native.library()
    n = lib.dd_prefill_flag_count(segments, max_len, heads, kv_heads, dim, DTYPE_CODES[dtype])
    if n < 0:
        raise _native.NativeError(f'dd_prefill_flag_count failed: {lib.dd_error_string(-n).decode()} ({-n})')
    return n


def ragged_attention(query, cache_k, cache_v, packed, page_table, window=0, scale=None):
    """Mixed batch: the trailing single-token segments decode, the rest prefill.

    Returns (T, H, D) in the query dtype.
    """
    q = _check(query, cache_k, cache_v, page_table)
    T, H, D = q.shape
    out = torch.empty_like(q)
    lengths = packed.lengths
    n = len(lengths)
    first_decode = n
    while first_decode > 0 and lengths[first_decode - 1] == 1:
        first_decode -= 1
    t_decode = sum(lengths[:first_decode])

    def decode():
        rows = slice(t_decode, T)
        kernels.prepare_attention(q[rows].unsqueeze(2), cache_k, cache_v, packed.positions[rows],
                                  packed.slot_ids[rows], window=window, scale=scale, page_table=page_table,
                                  out=out[rows].unsqueeze(2)).run()

    if first_decode > 0 and first_decode < n:
        # The decode rows (HBM-bound) run on a side stream beside the prefill
        # chunks (matrix cores): C4 526 us vs 586 us one after the other.  The
        # two write disjoint rows of `out`; the caller's stream waits for both.
        main = torch.cuda.current_stream(q.device)
        side = _side_stream(q.device)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            decode()
        prefill_attention(q, cache_k, cache_v, packed, page_table, window, scale, out, (0, first_decode))
        main.wait_stream(side)
    elif first_decode > 0:
        prefill_attention(q, cache_k, cache_v, packed, page_table, window, scale, out, (0, first_decode))
    elif first_decode < n:
        decode()
    return out


_SIDE_STREAMS = {}


def _side_stream(device):
    """One extra stream per device, default priority, for the decode half of a mixed batch."""
    key = torch.device(device).index
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = torch.cuda.Stream(device=device)
    return _SIDE_STREAMS[key]

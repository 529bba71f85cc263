"""Q8_0 KV codec on the GPU, with the reference API of damendaemon/kv_quant.py.

``quantize_kv``/``dequantize_kv`` keep the reference signatures and the
reference format by default (one fp16 scale per gcd(dim, 32) channels,
kv_quant.py:23-31); the ``group`` keyword extends them to any channel group
that divides the head (``group=dim`` is one scale per (token, KV head)).
Arithmetic is bit-identical to the reference (see csrc/quant.hip).
"""
import math

import torch

from . import _native
from ._native import DTYPE_CODES, call, ptr, stream_of

GROUP = 32


def group_for(dim):
    """Channel group of the reference format: gcd(dim, 32)."""
    return math.gcd(int(dim), GROUP)


def allocate_kv(max_batch, kv_heads, context, dim, device, group=None):
    """(data, scales) of one layer: (2, batch, KH, context, dim) int8 and
    (2, batch, KH, context, dim/group) fp16, zero-filled (kv_quant.py:34-45)."""
    group = group or group_for(dim)
    if dim % group or context <= 0 or max_batch <= 0 or kv_heads <= 0:
        raise ValueError('invalid quantized KV geometry')
    data = torch.zeros((2, max_batch, kv_heads, context, dim), dtype=torch.int8, device=device)
    scales = torch.zeros((2, max_batch, kv_heads, context, dim // group), dtype=torch.float16, device=device)
    return data, scales


def quantize_kv(values, group=None):
    """int8 values and fp16 scales (..., dim/group) of ``values`` (..., tokens, dim)."""
    dim = values.shape[-1]
    group = group or group_for(dim)
    if values.ndim < 2 or dim % group:
        raise ValueError('quantized KV requires a valid channel-group geometry')
    _native.require_device(values)
    if values.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError('quantized KV input must be fp32, fp16 or bf16')
    x = values.contiguous()
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    s = torch.empty((*x.shape[:-1], dim // group), dtype=torch.float16, device=x.device)
    call('dd_quantize_q8', ptr(x), DTYPE_CODES[x.dtype], x.numel() // dim, dim, group, ptr(q), ptr(s),
         stream_of(x))
    return q, s


def dequantize_kv(data, scales, dtype):
    """int8 * float(scale), rounded once to ``dtype`` (kv_quant.py:67-76)."""
    if data.dtype != torch.int8 or scales.dtype != torch.float16:
        raise ValueError('quantized KV requires int8 values with FP16 scales')
    dim = data.shape[-1]
    if scales.shape[:-1] != data.shape[:-1] or dim % scales.shape[-1]:
        raise ValueError('incompatible quantized KV shapes')
    _native.require_device(data, scales)
    group = dim // scales.shape[-1]
    d, s = data.contiguous(), scales.contiguous()
    out = torch.empty(d.shape, dtype=dtype, device=d.device)
    call('dd_dequantize_q8', ptr(d), ptr(s), d.numel() // dim, dim, group, ptr(out), DTYPE_CODES[dtype],
         stream_of(d))
    return out


def store_kv(cache, slots, positions, k, v):
    """Quantise K/V (batch, KH, tokens, dim) into (slot, position) rows of the
    dense resident pair (the contract of kv_quant.py:79-107).

    One GPU quantisation of K and V together and one indexed write each for
    the int8 rows and the scales.  When (slot, position) pairs repeat, the
    last one in (row, token) order wins, as in the reference's row-by-row
    loop (kv_quant.py:99-106): every duplicate writes the winner's values,
    so the result does not depend on the order the GPU applies the writes.
    """
    data, scales = cache
    if positions.ndim != 2 or positions.shape[0] != k.shape[0] or positions.shape[1] != k.shape[2]:
        raise ValueError('quantized KV store requires (batch, tokens) positions')
    group = data.shape[-1] // scales.shape[-1]
    if k.ndim != 4 or v.shape != k.shape or k.shape[0] != len(slots) or k.shape[-1] % group:
        raise ValueError('quantized KV store requires matching batch-major K/V')
    if positions.numel() and int(positions.max()) >= data.shape[3]:
        raise ValueError('KV store position exceeds the cache context')
    codes, steps = quantize_kv(torch.stack((k, v)), group)        # (2, B, KH, T, ...)
    slot_of_token = torch.as_tensor(slots, device=data.device).long()[:, None].expand(positions.shape)
    pos = positions.to(data.device).long()
    winner = _last_writer(slot_of_token * data.shape[3] + pos)
    where = (slot_of_token, slice(None), pos)
    # destination rows data[:, b-slot, :, position] are (B, T, 2, KH, ...)
    rows = codes.permute(1, 3, 0, 2, 4)
    row_scales = steps.permute(1, 3, 0, 2, 4)
    data[(slice(None),) + where] = rows.reshape((-1,) + rows.shape[2:])[winner].view(rows.shape)
    scales[(slice(None),) + where] = row_scales.reshape((-1,) + row_scales.shape[2:])[winner].view(row_scales.shape)


def _last_writer(keys):
    """For each element of ``keys`` (any shape, flattened in order), the flat
    index of the last element with the same key.  Sort-based, no host sync."""
    flat = keys.reshape(-1)
    ordered, perm = torch.sort(flat, stable=True)
    last = torch.searchsorted(ordered, ordered, right=True) - 1
    winner = torch.empty_like(perm)
    winner[perm] = perm[last]
    return winner


def read_kv(cache, slots, end, dtype=torch.float32):
    """Dequantised (slots, KH, end, dim) K and V of the populated prefix (the
    contract of kv_quant.py:110-122); duplicate slots give duplicate rows."""
    data, scales = cache
    rows = torch.as_tensor(slots, device=data.device).long()
    both = dequantize_kv(data[:, rows, :, :end], scales[:, rows, :, :end], dtype)
    return both[0], both[1]

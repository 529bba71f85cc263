"""Causal index plans for full-prefill and single-token ring-cache attention, on the GPU.

Same API, validation order and outputs as damendaemon/cache_indices.py:24-80:
every argument is validated (and the 1,048,576-element plan budget enforced)
before anything is allocated; the plans are then filled by one HIP kernel.
"""
import torch

from . import _native
from ._native import call, ptr

MAX_INDEX_ELEMENTS = 1_048_576


def _integer(value, name, minimum=1):
    if type(value) is not int or not minimum <= value < 2 ** 31:
        raise ValueError(f'{name} must be an integer in {minimum}..2147483647')


def _options(window, ratio, batch, rows, columns):
    _integer(window, 'window')
    _integer(ratio, 'compression ratio', 0)
    _integer(batch, 'batch')
    if batch * rows * columns > MAX_INDEX_ELEMENTS:
        raise ValueError('cache index plan exceeds 1048576 elements; split query rows')


def prefill_indices(sequence_length, *, window, ratio=0, batch=1, query_start=0, query_stop=None, device='cuda'):
    """(batch, rows, keys + compressed) int64 indices into [sequence KV, completed compressed blocks]."""
    _integer(sequence_length, 'sequence length')
    _integer(query_start, 'query start', 0)
    query_stop = sequence_length if query_stop is None else query_stop
    _integer(query_stop, 'query stop')
    _integer(window, 'window')
    _integer(ratio, 'compression ratio', 0)
    if not query_start < query_stop <= sequence_length:
        raise ValueError('prefill query range must be nonempty and within the full sequence')
    keys = min(window, sequence_length)
    compressed = query_stop // ratio if ratio else 0
    _options(window, ratio, batch, query_stop - query_start, keys + compressed)
    out = torch.empty((query_stop - query_start, keys + compressed), dtype=torch.int64, device=device)
    _native.require_device(out)
    call('dd_prefill_indices', sequence_length, window, ratio, query_start, query_stop, ptr(out),
         _native.stream_of(out))
    return out.unsqueeze(0).expand(batch, -1, -1)


def ring_decode_indices(positions, *, window, ratio=0, device='cuda'):
    """(slots, 1, window + compressed) int64 indices into [window ring KV, compressed blocks]."""
    if not isinstance(positions, (tuple, list)) or not positions:
        raise ValueError('ring decode requires a nonempty list/tuple of logical positions')
    for position in positions:
        _integer(position, 'logical position', 0)
    _integer(window, 'window')
    _integer(ratio, 'compression ratio', 0)
    compressed = (max(positions) + 1) // ratio if ratio else 0
    _options(window, ratio, len(positions), 1, window + compressed)
    logical = torch.tensor(positions, dtype=torch.int64, device=device)
    _native.require_device(logical)
    out = torch.empty((len(positions), window + compressed), dtype=torch.int64, device=device)
    call('dd_ring_decode_indices', ptr(logical), len(positions), window, ratio, compressed, ptr(out),
         _native.stream_of(out))
    return out.unsqueeze(1)

"""ctypes binding of the gfx950 shared library (the C ABI in include/).

Mirrors the reference's native-library convention
(damendaemon/native_q4.py:9-47): the library is opened once, its ABI
version is checked, functions take plain device pointers, ints and a
stream, and a non-zero return code becomes an exception here.

There is no CPU fallback: every op in this package runs on the HIP
kernels, and a missing or stale library raises instead of silently
computing something else.
"""
import ctypes
import threading
import os
from functools import lru_cache
from pathlib import Path

import torch

ABI_VERSION = 5
LIBRARY = Path(__file__).resolve().parent / '_lib' / 'libdamendaemon_amd.so'

F32, F16, BF16, I8 = 0, 1, 2, 3
DTYPE_CODES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.int8: I8}

_p, _i, _i64, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float

# name -> argtypes (restype is always c_int)
SIGNATURES = {
    'dd_abi_version': [],
    'dd_decode_splits': [_i, _i, ctypes.POINTER(_i)],
    'dd_decode_splits_for': [_i, _i, _i, _i, ctypes.POINTER(_i)],
    'dd_decode_attention': [_p, _i, _p, _p, _i, _p, _p, _i,   # q .. group
                            _p, _p, _p, _i, _i,               # positions, slots, table, rows, width
                            _i, _i, _i, _i, _i, _i64, _i, _f,  # B H KH D page cap window scale
                            _p, _p, _i, _f, _p,               # alibi rel buckets denom sinks
                            _p, _p, _p, _i, _i, _p],          # out part lse splits split_tokens stream
}
SIGNATURES['dd_quantize_q8'] = [_p, _i, _i64, _i, _i, _p, _p, _p]
SIGNATURES['dd_dequantize_q8'] = [_p, _p, _i64, _i, _i, _p, _i, _p]
SIGNATURES['dd_pack_batch'] = [_p, _p, _p, _i, _i64, _i64, _p, _i, _i, _i] + [_p] * 9
SIGNATURES['dd_store_kv_pages'] = [_p, _p, _i, _p, _i64, _i, _i, _i, _i64, _p, _p, _p]
SIGNATURES['dd_store_kv_pages_q8'] = [_p, _p, _i, _p, _i64, _i, _i, _i, _i, _i64, _p, _p, _p, _p, _p]
SIGNATURES['dd_copy_pages'] = [_p, _p, _i, _i, _p, _i, _i64, _i64, _i64, _i, _i, _i, _i, _p]
SIGNATURES['dd_rope_batch'] = [_p, _i, _p, _p, _i, _i, _p, _p, _i64, _i, _i, _i, _p, _p, _i, _f, _i,
                               _p, _i, _i, _p, _p, _p, _i, _i64, _i, _p, _p, _p]
SIGNATURES['dd_prefill_attention'] = [_p, _p, _p, _i, _p, _p, _p, _i, _i, _i, _p, _i, _i, _i, _i, _i, _i, _i64, _i,
                                      _f, _p, _i, _p, _p, _p]
SIGNATURES['dd_prefill_flag_count'] = [_i, _i, _i, _i, _i, _i]
SIGNATURES['dd_prefill_attention_phase'] = SIGNATURES['dd_prefill_attention'][:-1] + [_i, _p]
SIGNATURES['dd_prefill_plan'] = [_p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _i]
SIGNATURES['dd_prefill_geometry'] = [_i, ctypes.POINTER(_i), ctypes.POINTER(_i)]
SIGNATURES['dd_prefill_indices'] = [_i64, _i, _i, _i64, _i64, _p, _p]
SIGNATURES['dd_ring_decode_indices'] = [_p, _i64, _i, _i, _i, _p, _p]
SIGNATURES['dd_decode_partials'] = SIGNATURES['dd_decode_attention']
SIGNATURES['dd_decode_merge'] = SIGNATURES['dd_decode_attention']
# the allocation-free variant: no partial / lse arguments
SIGNATURES['dd_decode_attention_static'] = SIGNATURES['dd_decode_attention'][:-5] + [_i, _i, _p]


class NativeError(RuntimeError):
    pass


@lru_cache(maxsize=1)
def library():
    path = os.environ.get('DAMENDAEMON_AMD_LIBRARY', str(LIBRARY))
    if not Path(path).exists():
        raise NativeError(f'{path} is missing: build it with '
                          '`python -m damendaemon_amd.build` (no CPU fallback exists)')
    handle = ctypes.CDLL(path)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    handle.dd_error_string.argtypes = [_i]
    handle.dd_error_string.restype = ctypes.c_char_p
    if handle.dd_abi_version() != ABI_VERSION:
        raise NativeError('unsupported damendaemon_amd library ABI')
    return handle


def call(name, *args):
    lib = library()
    code = getattr(lib, name)(*args)
    if code:
        raise NativeError(f'{name} failed: {lib.dd_error_string(code).decode()} ({code})')


def ptr(tensor):
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


def stream_of(tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(tensor.device).cuda_stream)


def require_device(*tensors):
    for t in tensors:
        if t is not None and t.device.type != 'cuda':
            raise ValueError('damendaemon_amd kernels need tensors on the GPU '
                             '(there is no CPU path)')


class _Staging:
    """Pinned host buffers for the small per-call uploads (segment metadata,
    prefill plans), reused round-robin instead of pinning fresh memory on
    every call: pinning costs far more than the copy.  Each slot remembers
    the event of its last copy and waits for it before being rewritten."""

    SLOTS = 8

    def __init__(self):
        self._slots = {}   # device index -> list of [pinned uint8 buffer, event or None]
        self._next = {}
        # slot choice, the wait on the slot's last copy, the host copy into it
        # and the enqueue of its device copy happen under one lock, so that two
        # host threads never fill the same pinned slot at once
        self._lock = threading.Lock()

    def upload(self, host, device):
        """Asynchronous copy of the contiguous CPU tensor ``host`` to ``device``
        on the current stream; returns the device tensor.  Not under graph
        capture: a replay would copy whatever the reused pinned slot holds by
        then (prepare the call outside the capture and capture its run())."""
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError('host upload during HIP graph capture: prepare the call (prepare_prefill, '
                               'pack_batch) before capturing and capture only the launch')
        host = host.contiguous()
        with self._lock:
            return self._upload(host, torch.device(device))

    def _upload(self, host, dev):
        nbytes = host.numel() * host.element_size()
        index = dev.index if dev.index is not None else torch.cuda.current_device()
        slots = self._slots.setdefault(index, [[None, None] for _ in range(self.SLOTS)])
        k = self._next.get(index, 0)
        self._next[index] = (k + 1) % self.SLOTS
        slot = slots[k]
        if slot[1] is not None:
            slot[1].synchronize()
        if slot[0] is None or slot[0].numel() < nbytes:
            slot[0] = torch.empty(max(nbytes, 4096), dtype=torch.uint8, pin_memory=True)
        staged = slot[0][:nbytes].view(host.dtype).view(host.shape)
        staged.copy_(host)
        out = torch.empty(host.shape, dtype=host.dtype, device=dev)
        out.copy_(staged, non_blocking=True)
        if slot[1] is None:
            slot[1] = torch.cuda.Event()
        slot[1].record(torch.cuda.current_stream(dev))
        return out


_staging = _Staging()


def upload(host, device):
    """Copy a small CPU tensor to the GPU through the reusable pinned buffers."""
    return _staging.upload(host, device)

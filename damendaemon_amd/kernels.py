"""Drop-in replacement for the attention entry points of ``damendaemon.kernels``.

``PagedExecutor`` reaches its kernels through the module object
(damendaemon/qwen2.py:458-461, damendaemon/paged.py:90-95), so this module
exposes the same functions with the same signatures and keyword defaults;
every call runs hand-written gfx950 HIP kernels through the C ABI in
``include/damendaemon_amd.h``.
"""
import ctypes
import math
import os

import torch

from . import _native
from ._native import DTYPE_CODES, call, ptr


def _splits(max_context, batch_kv, dim, kv_dtype):
    """Split count and tokens per split: the library's policy for this head
    size and page dtype, or a fixed split size from
    DAMENDAEMON_AMD_SPLIT_TOKENS (a multiple of 64; tuning)."""
    forced = os.environ.get('DAMENDAEMON_AMD_SPLIT_TOKENS')
    if forced:
        tokens = int(forced)
        if tokens <= 0 or tokens % 64:
            raise ValueError('DAMENDAEMON_AMD_SPLIT_TOKENS must be a positive multiple of 64')
        return -(-int(max_context) // tokens), tokens
    tokens = ctypes.c_int(0)
    splits = _native.library().dd_decode_splits_for(int(max_context), int(batch_kv), int(dim), DTYPE_CODES[kv_dtype],
                                                     ctypes.byref(tokens))
    if splits <= 0:
        raise ValueError('invalid decode geometry')
    return splits, tokens.value


def attention(query, cache_k, cache_v, positions, slots=None, window=0, scale=None, alibi=None, page_table=None,
              relative_bias=None, relative_max_distance=128, sinks=None, scratch_bytes=None,
              *, k_scale=None, v_scale=None):
    """Decode attention of one query row per sequence over a paged or slotted cache.

    Same contract as damendaemon/kernels.py:213-267:
      query (B, H, 1, D); cache_k/cache_v (capacity, KH, page, D) with
      ``page_table`` (rows, W) int32, or (slots, KH, context, D) without;
      positions (B,) index of the current token (keys 0..pos are live);
      returns a new (B, H, 1, D) tensor in the query dtype.
    Extension (no reference counterpart): int8 pages with fp16 scales
    ``k_scale``/``v_scale`` shaped (..., page, D/group), the Q8_0 layout of
    damendaemon/kv_quant.py:48-64 generalised to any group that is a
    multiple of 32 or the whole head.
    """
    if scratch_bytes is not None:
        from .attention_budget import query_rows
        batch, heads, _, dim = query.shape
        context = cache_k.shape[2] * (1 if page_table is None else page_table.shape[1])
        splits, _ = _splits(context, batch * cache_k.shape[1], dim, cache_k.dtype)
        rows = query_rows(heads, dim, splits, scratch_bytes, query.element_size())
        if batch > rows:
            # Partition only independent query rows (kernels.py:237-252); each
            # row still attends its whole history.
            out = torch.empty_like(query)
            for start in range(0, batch, rows):
                end = min(start + rows, batch)
                out[start:end].copy_(attention(
                    query[start:end], cache_k, cache_v, positions[start:end],
                    None if slots is None else slots[start:end], window=window, scale=scale,
                    alibi=alibi, page_table=page_table, relative_bias=relative_bias,
                    relative_max_distance=relative_max_distance, sinks=sinks,
                    k_scale=k_scale, v_scale=v_scale))
            return out
    return prepare_attention(query, cache_k, cache_v, positions, slots, window, scale, alibi, page_table,
                             relative_bias, relative_max_distance, sinks, k_scale=k_scale, v_scale=v_scale).run()


def prepare_attention(query, cache_k, cache_v, positions, slots=None, window=0, scale=None, alibi=None,
                      page_table=None, relative_bias=None, relative_max_distance=128, sinks=None,
                      *, k_scale=None, v_scale=None, out=None):
    """Validate a decode call once and return its ``DecodeLaunch``.

    ``out`` (optional) is a preallocated (B, H, 1, D) contiguous output.

    Arguments and errors are those of ``attention`` (damendaemon/kernels.py:213-229).
    """
    batch, heads, _, dim = query.shape
    if alibi is not None and (alibi.shape != (heads,) or alibi.dtype != torch.float32
                              or alibi.device != query.device or not alibi.is_contiguous()):
        raise ValueError('ALiBi needs one contiguous FP32 slope per query head on the same device')
    if sinks is not None and (sinks.shape != (heads,) or sinks.dtype != torch.float32
                              or sinks.device != query.device or not sinks.is_contiguous()):
        raise ValueError('attention sinks require one contiguous FP32 logit per query head')
    buckets = 0
    if relative_bias is not None:
        if (relative_bias.ndim != 2 or relative_bias.shape[0] != heads or relative_bias.shape[1] < 2
                or relative_bias.shape[1] % 2 or relative_bias.dtype != torch.float32
                or relative_bias.device != query.device or not relative_bias.is_contiguous()
                or type(relative_max_distance) is not int
                or relative_max_distance <= relative_bias.shape[1] // 2):
            raise ValueError('invalid relative attention bias')
        buckets = relative_bias.shape[1]
    capacity, kv_heads, page_size, kdim = cache_k.shape
    if (cache_v.shape != cache_k.shape or kdim != dim or heads % kv_heads
            or query.shape[2] != 1 or positions.shape != (batch,)):
        raise ValueError('incompatible attention shapes')
    quantized = k_scale is not None or v_scale is not None
    group = 0
    if quantized:
        if (k_scale is None or v_scale is None or cache_k.dtype != torch.int8 or cache_v.dtype != torch.int8
                or k_scale.dtype != torch.float16 or v_scale.dtype != torch.float16
                or k_scale.shape != v_scale.shape or k_scale.shape[:-1] != cache_k.shape[:-1]
                or dim % k_scale.shape[-1] or not k_scale.is_contiguous() or not v_scale.is_contiguous()):
            raise ValueError('int8 KV pages need fp16 scales shaped (..., page, dim/group)')
        group = dim // k_scale.shape[-1]
    elif cache_k.dtype != query.dtype or cache_v.dtype != query.dtype:
        raise ValueError('KV cache dtype must match the query dtype')
    if not (query.is_contiguous() and cache_k.is_contiguous() and cache_v.is_contiguous()):
        raise ValueError('attention needs contiguous query and cache tensors')
    _native.require_device(query, cache_k, cache_v, positions, slots, page_table)
    if positions.dtype != torch.int64:
        positions = positions.to(torch.int64)
    if slots is not None and slots.dtype != torch.int64:
        slots = slots.to(torch.int64)
    if page_table is not None:
        if page_table.dtype != torch.int32 or page_table.ndim != 2 or not page_table.is_contiguous():
            raise ValueError('page table must be a contiguous int32 matrix')
        context = page_table.shape[1] * page_size
    else:
        context = page_size
    splits, split_tokens = _splits(context, batch * kv_heads, dim, cache_k.dtype)
    return DecodeLaunch(query, cache_k, cache_v, positions, slots, page_table, kv_heads, page_size, capacity,
                        group, k_scale, v_scale, window, scale, alibi, relative_bias, buckets,
                        relative_max_distance, sinks, splits, split_tokens, out)


class DecodeLaunch:
    """One validated decode launch with its output and split scratch allocated.

    ``run()`` enqueues the split kernel and the merge on the current stream;
    ``partials()`` / ``merge()`` enqueue one phase each.  Buffers and
    arguments stay fixed, so repeated runs (or a HIP-graph capture of them)
    see stable pointers, as the reference's per-batch-size graphs require
    (damendaemon/batch.py:25-46).
    """

    def __init__(self, query, cache_k, cache_v, positions, slots, page_table, kv_heads, page_size, capacity,
                 group, k_scale, v_scale, window, scale, alibi, relative_bias, buckets, relative_max_distance,
                 sinks, splits, split_tokens, out=None):
        batch, heads, _, dim = query.shape
        if out is not None and (out.shape != query.shape or out.dtype != query.dtype or not out.is_contiguous()):
            raise ValueError('out must be a contiguous tensor shaped and typed like the query')
        self.out = torch.empty_like(query) if out is None else out
        if splits > 1:
            self.partial = torch.empty((batch * heads, splits, dim), device=query.device, dtype=torch.float32)
            self.lse = torch.empty((batch * heads, splits), device=query.device, dtype=torch.float32)
        else:
            self.partial = self.lse = None
        self.splits, self.split_tokens = splits, split_tokens
        # keep every tensor argument alive as long as the launch object
        self._keep = (query, cache_k, cache_v, positions, slots, page_table, k_scale, v_scale, alibi,
                      relative_bias, sinks)
        self._device = query.device
        self._args = (
            ptr(query), DTYPE_CODES[query.dtype], ptr(cache_k), ptr(cache_v), DTYPE_CODES[cache_k.dtype],
            ptr(k_scale), ptr(v_scale), group,
            ptr(positions), ptr(slots), ptr(page_table),
            0 if page_table is None else page_table.shape[0], 0 if page_table is None else page_table.shape[1],
            batch, heads, kv_heads, dim, page_size, capacity, int(window or 0),
            float(dim ** -.5 if scale is None else scale),
            ptr(alibi), ptr(relative_bias), buckets,
            math.log(relative_max_distance / (buckets // 2)) if buckets else 1.0,
            ptr(sinks), ptr(self.out), ptr(self.partial), ptr(self.lse), splits, split_tokens)

    def _call(self, name):
        call(name, *self._args, ctypes.c_void_p(torch.cuda.current_stream(self._device).cuda_stream))

    def run(self):
        self._call('dd_decode_attention')
        return self.out

    def partials(self):
        self._call('dd_decode_partials')

    def merge(self):
        self._call('dd_decode_merge')


def rope_batch(qkv, cos, sin, positions, slots, cache_k, cache_v, heads, q_norm=None, k_norm=None, eps=1e-6,
               precise=False, page_table=None, materialize=False):
    """Rotary embedding + K/V cache write, same contract as damendaemon/kernels.py:325-340.

    qkv (T, (heads + 2*KH)*D); cos/sin (positions, RD); writes rotated keys
    and raw values into ``cache_k``/``cache_v`` at each token's position
    (through ``page_table`` when given) and returns the rotated queries
    (T, heads, 1, D), or (query, key, value) with dense (T, KH, D) copies
    when ``materialize``.
    """
    _, kv_heads, context, dim = cache_k.shape
    rotary_dim = cos.shape[-1]
    if not 0 < rotary_dim <= dim or rotary_dim % 2 or (q_norm is not None and rotary_dim != dim):
        raise ValueError('unsupported rotary table width')
    tokens = qkv.shape[0]
    if (qkv.ndim != 2 or qkv.shape[1] != (heads + 2 * kv_heads) * dim or cache_v.shape != cache_k.shape
            or positions.shape != (tokens,) or slots.shape != (tokens,) or sin.shape != cos.shape):
        raise ValueError('incompatible rope_batch shapes')
    _native.require_device(qkv, cos, sin, positions, slots, cache_k, cache_v, q_norm, k_norm, page_table)
    qkv, cos, sin = qkv.contiguous(), cos.contiguous(), sin.contiguous()
    if not cache_k.is_contiguous() or not cache_v.is_contiguous():
        raise ValueError('rope_batch writes contiguous caches only')
    norm = q_norm if q_norm is not None else k_norm
    if (q_norm is None) != (k_norm is None):
        raise ValueError('q_norm and k_norm go together')
    if norm is not None and (q_norm.dtype != k_norm.dtype or q_norm.numel() != dim or k_norm.numel() != dim):
        raise ValueError('norm weights must be (dim,) of one dtype')
    positions = positions.to(torch.int64)
    slots = slots.to(torch.int64)
    if page_table is not None and (page_table.dtype != torch.int32 or not page_table.is_contiguous()):
        raise ValueError('page table must be a contiguous int32 matrix')
    query = torch.empty((tokens, heads, 1, dim), device=qkv.device, dtype=qkv.dtype)
    key = torch.empty((tokens, kv_heads, dim), device=qkv.device, dtype=cache_k.dtype) if materialize else None
    value = torch.empty_like(key) if materialize else None
    call('dd_rope_batch', ptr(qkv), DTYPE_CODES[qkv.dtype], ptr(cos), ptr(sin), DTYPE_CODES[cos.dtype], rotary_dim,
         ptr(positions), ptr(slots), tokens, heads, kv_heads, dim,
         ptr(None if norm is None else q_norm.contiguous()), ptr(None if norm is None else k_norm.contiguous()),
         DTYPE_CODES[norm.dtype] if norm is not None else 0, float(eps), int(bool(precise)),
         ptr(page_table), 0 if page_table is None else page_table.shape[0],
         0 if page_table is None else page_table.shape[1],
         ptr(query), ptr(cache_k), ptr(cache_v), DTYPE_CODES[cache_k.dtype], cache_k.shape[0], context,
         ptr(key), ptr(value), _native.stream_of(qkv))
    return (query, key, value) if materialize else query


# The functions of this module that replace the reference's kernels-module
# entry points one for one (damendaemon/kernels.py:213 attention, :325
# rope_batch).  The executor's kernels module also supplies rms, swiglu,
# rope_store and linear_fp32 (damendaemon/kernels.py:29,48,121,356; called at
# qwen2.py:606,678,684 and paged.py:114); those are not attention and stay
# the module's own.
HOT_PATH = ('attention', 'rope_batch')


def install(module):
    """Point ``module.attention`` and ``module.rope_batch`` at this package.

    ``module`` is the kernels module an executor already holds
    (``self.kernels``, damendaemon/qwen2.py:458-461).  Only the two hot-path
    attributes are replaced; every other attribute (rms, swiglu, rope_store,
    linear_fp32, ...) is left as it was.  Returns ``module``.
    """
    missing = [name for name in HOT_PATH if not hasattr(module, name)]
    if missing:
        raise ValueError(f'{module!r} has no {", ".join(missing)}: not a kernels module')
    for name in HOT_PATH:
        setattr(module, name, globals()[name])
    return module


def overlay(module):
    """A new module object with every attribute of ``module``, except that
    ``attention`` and ``rope_batch`` come from this package; ``module`` itself
    is not changed (for one executor: ``self.kernels = overlay(self.kernels)``)."""
    import types
    view = types.ModuleType(getattr(module, '__name__', 'kernels') + '+damendaemon_amd')
    view.__dict__.update({k: v for k, v in vars(module).items() if k not in ('__name__', '__spec__', '__loader__')})
    return install(view)

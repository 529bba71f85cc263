"""Seeded synthetic inputs for the benchmark configurations and the parity tests.

Each builder returns plain tensors in the reference layouts: per-layer KV
pages (capacity, KV heads, 16, D) for K and V (damendaemon/paged.py:31-34),
an int32 page table (rows, W) with -1 for unused entries (paged.py:20-21),
int64 positions and slots.  Random values come from a torch Generator on
the target device, so the same seed gives the same inputs on every run on
that device type.
"""
import math

import torch

PAGE = 16


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def paged_decode_case(contexts, heads, kv_heads, dim, dtype, *, seed=0, device='cpu', capacity=None,
                      pool_factor=1.25, page=PAGE, table_width=None, nan_fill=False, outlier_frac=0.0,
                      outlier_scale=8.0):
    """Ragged decode over scattered pages.

    ``contexts[b]`` tokens are live for sequence b (keys 0..ctx-1, so
    ``positions = ctx - 1``).  Physical pages are a seeded permutation of the
    pool handed out in logical order.  Unused pool pages are NaN when
    ``nan_fill`` (they must never be read).  ``outlier_frac`` of K entries
    are multiplied by ``outlier_scale`` (the long-context config's outlier
    channels).
    """
    g = _gen(device, seed)
    counts = [math.ceil(c / page) for c in contexts]
    total = sum(counts)
    capacity = capacity or max(1, math.ceil(total * pool_factor))
    if capacity < total:
        raise ValueError('pool too small for the requested contexts')
    width = table_width or max(counts)
    order = torch.randperm(capacity, generator=g, device=device).cpu()
    table = torch.full((len(contexts), width), -1, dtype=torch.int32)
    used = torch.zeros(capacity, dtype=torch.bool)
    k = 0
    for b, n in enumerate(counts):
        table[b, :n] = order[k:k + n].to(torch.int32)
        used[order[k:k + n]] = True
        k += n
    shape = (capacity, kv_heads, page, dim)
    cache_k = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    cache_v = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    if outlier_frac:
        hit = torch.rand(shape, generator=g, device=device) < outlier_frac
        cache_k = torch.where(hit, cache_k * outlier_scale, cache_k)
    query = torch.randn((len(contexts), heads, 1, dim), generator=g, device=device, dtype=torch.float32)
    if nan_fill:
        unused = (~used).to(device)
        cache_k[unused] = float('nan')
        cache_v[unused] = float('nan')
        # tails of each sequence's last page are not live either
        for b, c in enumerate(contexts):
            if c % page:
                last = int(table[b, counts[b] - 1])
                cache_k[last, :, c % page:] = float('nan')
                cache_v[last, :, c % page:] = float('nan')
    return {
        'query': query.to(dtype), 'cache_k': cache_k.to(dtype), 'cache_v': cache_v.to(dtype),
        'page_table': table.to(device), 'positions': torch.tensor([c - 1 for c in contexts], device=device),
        'slots': torch.arange(len(contexts), device=device), 'contexts': list(contexts),
        'capacity': capacity,
    }


def quantize_pages(case, group, kv_quant):
    """Replace the bf16/fp32 pages of ``case`` by int8 pages + fp16 scales.

    ``kv_quant`` is the module providing ``quantize_kv(values, group)``
    (the GPU codec for device cases).
    """
    out = dict(case)
    out['cache_k'], out['k_scale'] = kv_quant.quantize_kv(case['cache_k'], group=group)
    out['cache_v'], out['v_scale'] = kv_quant.quantize_kv(case['cache_v'], group=group)
    return out


def uniform_contexts(n, lo, hi, seed):
    """n context lengths uniform in [lo, hi] from a CPU generator (seeded)."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (n,), generator=g).tolist()


# Benchmark configurations (BASELINE.json "configs").
def config_c1(device='cpu', seed=1):
    return paged_decode_case([17, 128, 300, 1000], 8, 2, 128, torch.float32, seed=seed, device=device,
                             capacity=128)


def config_c2(device='cuda', seed=2, dtype=torch.bfloat16):
    contexts = uniform_contexts(64, 512, 8192, seed)
    return paged_decode_case(contexts, 32, 8, 128, dtype, seed=seed, device=device,
                             table_width=8192 // PAGE)


def config_c5(device='cuda', seed=5):
    return paged_decode_case([32768] * 16, 16, 2, 256, torch.bfloat16, seed=seed, device=device,
                             capacity=16 * 32768 // PAGE, outlier_frac=0.01)


def config_c4(device='cuda', seed=4, dtype=torch.bfloat16, chunks=8, chunk=512, decodes=120, dim=128):
    """Mixed continuous batch: ``chunks`` prefill chunks of ``chunk`` tokens appended
    to contexts U[0,4096], then ``decodes`` single-token rows with contexts U[256,8192].

    Returns the paged case (history already in the pages), plus the packed
    segment lists and new query / K / V rows for every packed token.
    """
    g = torch.Generator().manual_seed(seed)
    chunk_starts = torch.randint(0, 4097, (chunks,), generator=g).tolist()
    decode_ctx = torch.randint(256, 8193, (decodes,), generator=g).tolist()
    lengths = [chunk] * chunks + [1] * decodes
    starts = chunk_starts + [c - 1 for c in decode_ctx]
    contexts = [s + n for s, n in zip(starts, lengths)]
    case = paged_decode_case(contexts, 32, 8, dim, dtype, seed=seed, device=device)
    gd = _gen(device, seed + 100)
    T = sum(lengths)
    case.update(lengths=lengths, starts=starts, seg_slots=list(range(len(lengths))),
                q=torch.randn((T, 32, dim), generator=gd, device=device).to(dtype),
                k_new=torch.randn((T, 8, dim), generator=gd, device=device).to(dtype),
                v_new=torch.randn((T, 8, dim), generator=gd, device=device).to(dtype))
    return case

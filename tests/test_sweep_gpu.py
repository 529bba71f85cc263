"""Seeded random sweeps of decode and chunked-prefill attention against the oracle.

Each case draws its own combination of KV dtype, head size, GQA width, page
size, batch shape, window, ALiBi / sinks / T5 bias and softmax scale, so the
kernels' dispatch paths (streamed and generic decode, int8 groupings, MFMA and
vector-ALU prefill) are crossed with each other instead of one axis at a time.
Bounds are those of test_decode_gpu.py and test_prefill_gpu.py: max
|gpu - oracle| <= atol + rtol*|ref| + half an ulp of ref in the output dtype.
"""
import random

import pytest
import torch

from _bounds import excess
from damendaemon_amd import kernels, packing, ragged
from damendaemon_amd.workloads import paged_decode_case
from oracle import paged_oracle as O

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def check(actual, expected, atol, rtol, out_dtype, what):
    worst, err = excess(actual, expected, atol, out_dtype, rtol)
    print(f'{what}: max abs err {err:.3e}')
    assert worst <= 0, f'{what}: max abs err {err:.3e} exceeds the bound by {worst:.3e}'


def decode_case(seed):
    rng = random.Random(seed)
    kind = rng.choice(['fp32', 'f16', 'bf16', 'i8g32', 'i8row'])
    dim = rng.choice([64, 96, 128, 256])
    kvh = rng.choice([1, 2, 4])
    group = rng.choice([1, 2, 4, 7, 8, 16, 20])
    page = rng.choice([16, 32, 64])
    n = rng.randint(1, 6)
    contexts = [rng.choice([1, rng.randint(2, 40), rng.randint(41, 700), rng.randint(701, 3000),
                            rng.randint(3001, 12000)]) for _ in range(n)]
    heads = kvh * group
    base = torch.float32 if kind.startswith('i8') else {'fp32': torch.float32, 'f16': torch.float16,
                                                       'bf16': torch.bfloat16}[kind]
    case = paged_decode_case(contexts, heads, kvh, dim, base, seed=seed, page=page, nan_fill=rng.random() < 0.5)
    if kind.startswith('i8'):
        g = 32 if kind == 'i8g32' else dim
        qk, ks = O.quantize_q8(case['cache_k'], g)
        qv, vs = O.quantize_q8(case['cache_v'], g)
        case.update(cache_k=qk, cache_v=qv, k_scale=ks, v_scale=vs,
                    query=case['query'].to(rng.choice([torch.bfloat16, torch.float16])))
    kw = {}
    if rng.random() < 0.3:
        kw['window'] = rng.randint(1, 800)
    if rng.random() < 0.3:
        kw['scale'] = rng.choice([0.05, 0.3, dim ** -.5 * 2])
    g = torch.Generator().manual_seed(seed)
    if rng.random() < 0.25:
        kw['alibi'] = -torch.rand(heads, generator=g) * 0.02
    if rng.random() < 0.25:
        kw['sinks'] = torch.randn(heads, generator=g)
    if rng.random() < 0.2:
        kw['relative_bias'] = torch.randn(heads, 32, generator=g)
        kw['relative_max_distance'] = rng.choice([64, 128])
    atol, rtol = {'fp32': (2e-5, 1e-5), 'f16': (2e-3, 0.0), 'bf16': (2e-3, 0.0)}.get(kind, (5e-3, 0.0))
    what = (f'decode seed {seed}: {kind} D{dim} KH{kvh} G{group} page {page} ctx {contexts} '
            f'{sorted(kw)} scale {kw.get("scale")}')
    return case, kw, atol, rtol, what


@pytest.mark.parametrize('seed', range(150))
def test_decode_sweep(seed):
    case, kw, atol, rtol, what = decode_case(1000 + seed)
    print(what, flush=True)
    d = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    dkw = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in kw.items()}
    out = kernels.attention(d['query'], d['cache_k'], d['cache_v'], d['positions'], d['slots'],
                            page_table=d['page_table'], k_scale=d.get('k_scale'), v_scale=d.get('v_scale'), **dkw)
    exp = O.decode_attention(case['query'], case['cache_k'], case['cache_v'], case['positions'], case['slots'],
                             page_table=case['page_table'], k_scale=case.get('k_scale'),
                             v_scale=case.get('v_scale'), **kw)
    check(out, exp, atol, rtol, out.dtype, what)


@pytest.mark.parametrize('seed', range(100))
def test_prefill_sweep(seed):
    rng = random.Random(2000 + seed)
    dtype = rng.choice([torch.bfloat16, torch.float16, torch.float32])
    dim = rng.choice([64, 80, 96, 128, 256])
    kvh = rng.choice([1, 2, 4])
    group = rng.choice([1, 2, 4, 7, 8])
    heads = kvh * group
    page = rng.choice([16, 32])
    n = rng.randint(1, 4)
    lengths = [rng.choice([1, rng.randint(2, 64), rng.randint(65, 300)]) for _ in range(n)]
    starts = [rng.choice([0, rng.randint(1, 100), rng.randint(101, 2000)]) for _ in range(n)]
    window = rng.choice([0, 0, 0, rng.randint(1, 400)])
    scale = rng.choice([None, None, 0.05, -dim ** -.5])
    contexts = [s + l for s, l in zip(starts, lengths)]
    case = paged_decode_case(contexts, heads, kvh, dim, dtype, seed=2000 + seed, page=page,
                             nan_fill=rng.random() < 0.5)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(sum(lengths), heads, dim, generator=g).to(dtype)
    slots = list(range(n))
    what = (f'prefill seed {2000 + seed}: {dtype} D{dim} KH{kvh} G{group} page {page} lengths {lengths} '
            f'starts {starts} window {window} scale {scale}')
    print(what, flush=True)
    table = case['page_table'].to(DEV)
    packed = packing.pack_batch(lengths, starts, slots, table, page_size=page)
    out = ragged.prefill_attention(q.to(DEV), case['cache_k'].to(DEV), case['cache_v'].to(DEV), packed, table,
                                   window=window, scale=scale)
    exp = O.prefill_attention(q, case['cache_k'], case['cache_v'], lengths, starts, slots, case['page_table'],
                              window=window, scale=scale)
    atol = 2e-5 if dtype == torch.float32 else 2e-3
    check(out, exp, atol, 0.0, dtype, what)

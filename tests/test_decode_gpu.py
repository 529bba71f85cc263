"""Decode attention on the GPU against the CPU oracle.

Cases restate the reference's GPU verification recipes as our own tests:
fragmented paging with NaN-filled pools (scripts/verify_paged_kernels.py:9-69),
slotted caches with reordered slots, NaN tails and expired windows
(scripts/verify_kernels.py:33-90), plus the BASELINE configurations.

Tolerances (max |gpu - oracle|, oracle in float64), each plus half an ulp of
the reference value in the output dtype (the output's own final rounding):
  fp32 KV: 2e-5 + 1e-5*|ref|;  fp16/bf16 KV: 2e-3;  int8 KV: 5e-3.
"""
import math

import pytest
import torch

from _bounds import excess
from damendaemon_amd import kernels
from damendaemon_amd.workloads import paged_decode_case, uniform_contexts
from oracle import paged_oracle as oracle

pytestmark = pytest.mark.gpu
DEV = 'cuda'
TOL = {torch.float32: (2e-5, 1e-5), torch.float16: (2e-3, 0.0), torch.bfloat16: (2e-3, 0.0),
       torch.int8: (5e-3, 0.0)}


def check(actual, expected, kind, rows=None):
    atol, rtol = TOL[kind]
    a = actual.detach().cpu()
    e = expected.double()
    if rows is not None:
        a, e = a[rows], e[rows]
    out_dtype = a.dtype
    worst, err = excess(a, e, atol, out_dtype, rtol)
    assert worst <= 0, f'max abs err {err:.3e} exceeds {atol} + {rtol}*|ref| + half-ulp ({worst:.3e} over)'
    return err


def to_dev(case):
    return {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}


def run_case(case, **kw):
    d = to_dev(case)
    return kernels.attention(d['query'], d['cache_k'], d['cache_v'], d['positions'], d['slots'],
                             page_table=d['page_table'], k_scale=d.get('k_scale'),
                             v_scale=d.get('v_scale'), **kw)


def oracle_case(case, **kw):
    return oracle.decode_attention(case['query'], case['cache_k'], case['cache_v'], case['positions'],
                                   case['slots'], page_table=case['page_table'],
                                   k_scale=case.get('k_scale'), v_scale=case.get('v_scale'), **kw)


def test_config_c1_fp32():
    case = paged_decode_case([17, 128, 300, 1000], 8, 2, 128, torch.float32, seed=1, capacity=128)
    check(run_case(case), oracle_case(case), torch.float32)


@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize('dim', [64, 96, 128])
@pytest.mark.parametrize('window', [0, 33])
def test_fragmented_pages_nan_pool(dtype, dim, window):
    """verify_paged_kernels.py recipe: 80-page NaN pool, table (4,33), slots [3,0,2]."""
    torch.manual_seed(2026)
    heads, kh, page, cap = 8, 2, 16, 80
    slots = torch.tensor([3, 0, 2])
    pos = torch.tensor([15, 256, 512])
    table = torch.full((4, 33), -1, dtype=torch.int32)
    k = torch.full((cap, kh, page, dim), float('nan'))
    v = torch.full_like(k, float('nan'))
    free = torch.randperm(cap).tolist()
    for slot, p in zip(slots.tolist(), pos.tolist()):
        for first in range(0, p + 1, page):
            block = free.pop()
            table[slot, first // page] = block
            n = min(page, p + 1 - first)
            k[block, :, :n] = torch.randn(kh, n, dim)
            v[block, :, :n] = torch.randn(kh, n, dim)
    q = torch.randn(3, heads, 1, dim)
    case = {'query': q.to(dtype), 'cache_k': k.to(dtype), 'cache_v': v.to(dtype), 'page_table': table,
            'positions': pos, 'slots': slots}
    check(run_case(case, window=window), oracle_case(case, window=window), dtype)


@pytest.mark.parametrize('dim', [64, 96, 128])
@pytest.mark.parametrize('context', [256, 513, 1024])
def test_slotted_positions_gqa7(dim, context):
    """verify_kernels.py:33-55: 14 query heads over 2 KV heads, several positions."""
    torch.manual_seed(7)
    heads, kvh = 14, 2
    k = torch.randn(1, kvh, context, dim).half()
    v = torch.randn_like(k)
    q = torch.randn(1, heads, 1, dim).half()
    kd, vd, qd = k.to(DEV), v.to(DEV), q.to(DEV)
    for position in sorted({0, 1, 31, min(255, context - 1), min(256, context - 1), context - 1}):
        pos = torch.tensor([position])
        out = kernels.attention(qd, kd, vd, pos.to(DEV))
        check(out, oracle.decode_attention(q, k, v, pos), torch.float16)
    # entries past the live prefix must not influence the output
    k[:, :, 1:] = float('nan')
    v[:, :, 1:] = float('nan')
    pos = torch.tensor([0])
    out = kernels.attention(q.to(DEV), k.to(DEV), v.to(DEV), pos.to(DEV))
    expected = v[:, :, :1].repeat_interleave(heads // kvh, dim=1)
    assert torch.equal(out.cpu(), expected)


def test_slotted_reordered_slots_nan_tails():
    """verify_kernels.py:56-70."""
    torch.manual_seed(11)
    context, dim, heads, kvh = 1024, 64, 14, 2
    k = torch.randn(5, kvh, context, dim).half()
    v = torch.randn_like(k)
    q = torch.randn(4, heads, 1, dim).half()
    slots = torch.tensor([4, 1, 3, 0])
    pos = torch.tensor([0, 256, 512, 1023])
    for s, p in zip(slots.tolist(), pos.tolist()):
        k[s, :, p + 1:] = float('nan')
        v[s, :, p + 1:] = float('nan')
    out = kernels.attention(q.to(DEV), k.to(DEV), v.to(DEV), pos.to(DEV), slots.to(DEV))
    check(out, oracle.decode_attention(q, k, v, pos, slots), torch.float16)


@pytest.mark.parametrize('dtype', [torch.float16, torch.float32])
@pytest.mark.parametrize('window', [1, 127, 256, 512])
def test_window_skips_expired_nan(dtype, window):
    """verify_kernels.py:72-90: D=256, one KV head, expired keys are NaN."""
    torch.manual_seed(window)
    dim, heads, context = 256, 4, 2048
    k = torch.randn(4, 1, context, dim, dtype=dtype)
    v = torch.randn_like(k)
    q = torch.randn(4, heads, 1, dim, dtype=dtype)
    slots = torch.tensor([3, 0, 2, 1])
    pos = torch.tensor([0, 511, 512, 2047])
    expected = oracle.decode_attention(q, k, v, pos, slots, window=window, scale=.07)
    for s, p in zip(slots.tolist(), pos.tolist()):
        start = max(0, p - window + 1)
        k[s, :, :start] = float('nan')
        v[s, :, :start] = float('nan')
        k[s, :, p + 1:] = float('nan')
        v[s, :, p + 1:] = float('nan')
    out = kernels.attention(q.to(DEV), k.to(DEV), v.to(DEV), pos.to(DEV), slots.to(DEV), window=window, scale=.07)
    check(out, expected, dtype)


@pytest.mark.parametrize('heads,kvh', [(4, 4), (6, 3), (16, 1), (24, 8), (32, 8), (12, 4), (40, 2), (34, 1)])
def test_group_sizes(heads, kvh):
    case = paged_decode_case([1, 15, 16, 17, 700, 2049], heads, kvh, 128, torch.bfloat16, seed=heads * 10 + kvh,
                             nan_fill=True)
    check(run_case(case), oracle_case(case), torch.bfloat16)


@pytest.mark.parametrize('group', [32, 128])
@pytest.mark.parametrize('qdtype', [torch.bfloat16, torch.float16])
def test_int8_pages(group, qdtype):
    case = paged_decode_case([5, 64, 333, 1500, 4000], 32, 8, 128, torch.float32, seed=group, nan_fill=False)
    qk, ks = oracle.quantize_q8(case['cache_k'], group)
    qv, vs = oracle.quantize_q8(case['cache_v'], group)
    case.update(cache_k=qk, cache_v=qv, k_scale=ks, v_scale=vs, query=case['query'].to(qdtype))
    check(run_case(case), oracle_case(case), torch.int8)


@pytest.mark.parametrize('qmag', [3e4, 1e-5])
@pytest.mark.parametrize('group', [128, 32])
def test_int8_query_and_value_ranges(qmag, group):
    """The int8 path feeds the matrix cores fp16: queries far outside fp16's
    comfortable range (x3e4, x1e-5, softmax scale compensating), and V rows
    whose magnitudes span 1e-6 .. 1e4 within one sequence (so p * v_scale
    spans ~2^33), must stay inside the int8 bound."""
    case = paged_decode_case([7, 200, 1500], 16, 4, 128, torch.float32, seed=int(qmag * 10) + group, nan_fill=False)
    g = torch.Generator().manual_seed(group)
    mag = torch.exp(torch.empty(case['cache_v'].shape[:3] + (1,)).uniform_(math.log(1e-6), math.log(1e4),
                                                                             generator=g))
    case['cache_v'] = case['cache_v'] * mag
    qk, ks = oracle.quantize_q8(case['cache_k'], group)
    qv, vs = oracle.quantize_q8(case['cache_v'], group)
    query = (case['query'] * qmag).to(torch.bfloat16)
    scale = 128 ** -.5 / qmag
    case.update(cache_k=qk, cache_v=qv, k_scale=ks, v_scale=vs, query=query)
    out = run_case(case, scale=scale)
    exp = oracle_case(case, scale=scale)
    # the outputs span the V magnitudes: the int8 bound is taken relative to
    # each row's largest value, plus the bf16 output's own half ulp (2^-9)
    a = out.cpu().double()
    assert torch.isfinite(a).all()
    row_mag = exp.abs().amax(dim=-1, keepdim=True).clamp_min(1e-300)
    err = ((a - exp).abs() / row_mag).max().item()
    assert err <= 5e-3 + 2 ** -9, f'max error {err:.3e} of the row magnitude'


def test_int8_dim256_group32():
    case = paged_decode_case([40, 900, 3000], 16, 2, 256, torch.float32, seed=3)
    qk, ks = oracle.quantize_q8(case['cache_k'], 32)
    qv, vs = oracle.quantize_q8(case['cache_v'], 32)
    case.update(cache_k=qk, cache_v=qv, k_scale=ks, v_scale=vs, query=case['query'].to(torch.bfloat16))
    check(run_case(case), oracle_case(case), torch.int8)


@pytest.mark.parametrize('dim,group', [(64, 64), (64, 32), (128, 128), (128, 32), (256, 256)])
@pytest.mark.parametrize('window', [0, 77])
def test_int8_nan_scales_and_expired_rows(dim, group, window):
    """Q8 pages whose unused rows (pool, page tails) and expired rows (before
    the window) carry NaN scales and arbitrary bytes: none may be read."""
    contexts = [1, 15, 17, 300, 1111, 2500]
    case = paged_decode_case(contexts, 12, 3, dim, torch.float32, seed=dim + group + window, nan_fill=True)
    qk, ks = oracle.quantize_q8(case['cache_k'], group)
    qv, vs = oracle.quantize_q8(case['cache_v'], group)
    expected = oracle.decode_attention(case['query'].to(torch.bfloat16), qk, qv, case['positions'], case['slots'],
                                       page_table=case['page_table'], k_scale=ks, v_scale=vs, window=window)
    ks[~torch.isfinite(ks)] = float('nan')
    vs[~torch.isfinite(vs)] = float('nan')
    if window:
        for b, c in enumerate(contexts):
            for t in range(max(0, c - window)):
                page = int(case['page_table'][b, t // 16])
                qk[page, :, t % 16] = 127
                qv[page, :, t % 16] = -127
                ks[page, :, t % 16] = float('nan')
                vs[page, :, t % 16] = float('nan')
    case.update(cache_k=qk, cache_v=qv, k_scale=ks, v_scale=vs, query=case['query'].to(torch.bfloat16))
    check(run_case(case, window=window), expected, torch.int8)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize('dim', [8, 16, 24, 32, 40, 48, 72, 80, 112, 144, 160, 192, 200, 224, 240])
def test_other_head_sizes(dtype, dim):
    """Head sizes (multiples of 8) other than 64/96/128/256: 16-bit and fp32 pages on the
    streamed kernel in the smallest of its 64/96/128/160/192/224/256 layouts that holds
    them (the extra dims zeros), rows of the real length; NaN-filled pools, several
    splits, 4 query heads per KV head, with and without a window."""
    contexts = [1, 17, 300, 2100]
    case = paged_decode_case(contexts, 12, 3, dim, dtype, seed=dim, nan_fill=True)
    check(run_case(case), oracle_case(case), dtype)
    check(run_case(case, window=45), oracle_case(case, window=45), dtype)


@pytest.mark.parametrize('dim,group', [(48, 48), (80, 80), (96, 96), (160, 160), (160, 32), (192, 32), (224, 224)])
@pytest.mark.parametrize('window', [0, 90])
def test_int8_other_head_sizes(dim, group, window):
    """Q8 pages at head sizes without a streamed kernel, NaN scales on unused rows."""
    contexts = [1, 15, 17, 300, 1111]
    case = paged_decode_case(contexts, 12, 3, dim, torch.float32, seed=dim + group, nan_fill=True)
    qk, ks = oracle.quantize_q8(case['cache_k'], group)
    qv, vs = oracle.quantize_q8(case['cache_v'], group)
    expected = oracle.decode_attention(case['query'].to(torch.bfloat16), qk, qv, case['positions'], case['slots'],
                                       page_table=case['page_table'], k_scale=ks, v_scale=vs, window=window)
    ks[~torch.isfinite(ks)] = float('nan')
    vs[~torch.isfinite(vs)] = float('nan')
    case.update(cache_k=qk, cache_v=qv, k_scale=ks, v_scale=vs, query=case['query'].to(torch.bfloat16))
    check(run_case(case, window=window), expected, torch.int8)


def test_unsupported_head_size_refused():
    """A head size that is not a multiple of 8 (or above 256) is refused before any launch."""
    for dim in (36, 272):
        case = paged_decode_case([5, 40], 4, 2, dim, torch.bfloat16, seed=dim)
        with pytest.raises(Exception, match='unsupported'):
            run_case(case)


@pytest.mark.parametrize('page', [32, 64])
@pytest.mark.parametrize('kind', ['bf16', 'int8'])
def test_larger_pages(page, kind):
    """Pages of 32 / 64 tokens: a page holds several 16-token chunks."""
    contexts = [3, 31, 32, 33, 700, 2049]
    dtype = torch.bfloat16 if kind == 'bf16' else torch.float32
    case = paged_decode_case(contexts, 16, 4, 128, dtype, seed=page, page=page, nan_fill=True)
    if kind == 'int8':
        qk, ks = oracle.quantize_q8(case['cache_k'], 128)
        qv, vs = oracle.quantize_q8(case['cache_v'], 128)
        case.update(cache_k=qk, cache_v=qv, k_scale=ks, v_scale=vs, query=case['query'].to(torch.bfloat16))
    check(run_case(case), oracle_case(case), torch.bfloat16 if kind == 'bf16' else torch.int8)


def test_alibi_sinks_relative_bias_with_splits():
    torch.manual_seed(3)
    case = paged_decode_case([3, 600, 2500, 5000], 8, 2, 128, torch.float16, seed=9)
    heads = 8
    alibi = torch.linspace(-0.01, -0.001, heads)
    sinks = torch.randn(heads)
    rel = torch.randn(heads, 32)
    for kw in ({'alibi': alibi}, {'sinks': sinks}, {'relative_bias': rel, 'relative_max_distance': 128},
               {'alibi': alibi, 'sinks': sinks, 'window': 300}):
        dev_kw = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in kw.items()}
        check(run_case(case, **dev_kw), oracle_case(case, **kw), torch.float16)


@pytest.mark.parametrize('dim,dtype', [(80, torch.bfloat16), (200, torch.float16), (40, torch.float32), (160, torch.bfloat16),
                                       (192, torch.float16), (224, torch.bfloat16)])
def test_other_head_sizes_bias_terms(dim, dtype):
    """Head sizes outside 64/96/128/256 with ALiBi, sinks, T5 bias and a window, over
    several splits and 16 query heads per KV head (MQA-like)."""
    g = torch.Generator().manual_seed(dim)
    case = paged_decode_case([2, 333, 1800, 4100], 16, 1, dim, dtype, seed=dim, nan_fill=True)
    heads = 16
    for kw in ({'alibi': -torch.rand(heads, generator=g) * 0.02, 'sinks': torch.randn(heads, generator=g)},
               {'relative_bias': torch.randn(heads, 32, generator=g), 'relative_max_distance': 128},
               {'alibi': -torch.rand(heads, generator=g) * 0.02, 'window': 250}):
        dev_kw = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in kw.items()}
        check(run_case(case, **dev_kw), oracle_case(case, **kw), dtype)


@pytest.mark.parametrize('dim,dtype', [(80, torch.bfloat16), (176, torch.float16), (48, torch.float32)])
def test_other_head_sizes_wide_groups(dim, dtype):
    """Head sizes below their streamed layout's with more than 16 query heads per KV head
    (40 on one KV head: three workgroups of up to 16 heads over the same keys)."""
    case = paged_decode_case([5, 700, 3000], 40, 1, dim, dtype, seed=dim + 40, nan_fill=True)
    check(run_case(case), oracle_case(case), dtype)
    check(run_case(case, window=100), oracle_case(case, window=100), dtype)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16])
@pytest.mark.parametrize('window', [0, 200])
def test_dim96_streamed_padded_rows(dtype, window):
    """D = 96 on the streamed kernel (LDS rows padded by 16 bytes, the pad
    lanes of the DMA reading out of range): NaN-filled unused pages, a page
    boundary inside every split, ALiBi + sinks and T5 bias."""
    g = torch.Generator().manual_seed(96 + window)
    case = paged_decode_case([1, 17, 300, 1409, 2900, 6000], 12, 3, 96, dtype, seed=96, nan_fill=True)
    heads = 12
    for kw in ({}, {'alibi': -torch.rand(heads, generator=g) * 0.02, 'sinks': torch.randn(heads, generator=g)},
               {'relative_bias': torch.randn(heads, 32, generator=g), 'relative_max_distance': 128}):
        if window:
            kw = dict(kw, window=window)
        dev_kw = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in kw.items()}
        check(run_case(case, **dev_kw), oracle_case(case, **kw), dtype)


@pytest.mark.parametrize('kind', ['bf16', 'fp32', 'int8'])
@pytest.mark.parametrize('heads,kvh', [(40, 2), (48, 1)])
def test_wide_groups_per_head_terms(kind, heads, kvh):
    """More than 16 query heads per KV head run as workgroups of up to 16 heads
    (40/2: 16 + 4 heads per KV head): every head's ALiBi slope, sink and T5 bias
    row must follow it into its workgroup."""
    g = torch.Generator().manual_seed(heads)
    base = torch.float32 if kind != 'bf16' else torch.bfloat16
    case = paged_decode_case([5, 700, 2600, 4100], heads, kvh, 128, base, seed=heads + 1)
    if kind == 'int8':
        qk, ks = oracle.quantize_q8(case['cache_k'], 32)
        qv, vs = oracle.quantize_q8(case['cache_v'], 32)
        case.update(cache_k=qk, cache_v=qv, k_scale=ks, v_scale=vs, query=case['query'].to(torch.bfloat16))
    alibi = -torch.rand(heads, generator=g) * 0.02
    sinks = torch.randn(heads, generator=g)
    rel = torch.randn(heads, 32, generator=g)
    for kw in ({'alibi': alibi, 'sinks': sinks}, {'relative_bias': rel, 'relative_max_distance': 128, 'window': 900}):
        dev_kw = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in kw.items()}
        check(run_case(case, **dev_kw), oracle_case(case, **kw), torch.int8 if kind == 'int8' else base)


@pytest.mark.parametrize('group', [32, 128])
def test_int8_alibi_sinks_relative_bias(group):
    """The bias, sink and window terms on the int8 path (two chunks per step)."""
    torch.manual_seed(5)
    case = paged_decode_case([3, 600, 2500, 5000], 8, 2, 128, torch.float32, seed=19)
    qk, ks = oracle.quantize_q8(case['cache_k'], group)
    qv, vs = oracle.quantize_q8(case['cache_v'], group)
    case.update(cache_k=qk, cache_v=qv, k_scale=ks, v_scale=vs, query=case['query'].to(torch.bfloat16))
    heads = 8
    alibi = torch.linspace(-0.01, -0.001, heads)
    sinks = torch.randn(heads)
    rel = torch.randn(heads, 32)
    for kw in ({'alibi': alibi, 'sinks': sinks, 'window': 300},
               {'relative_bias': rel, 'relative_max_distance': 128}):
        dev_kw = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in kw.items()}
        check(run_case(case, **dev_kw), oracle_case(case, **kw), torch.int8)


def test_sinks_single_split():
    case = paged_decode_case([3, 60, 100], 4, 2, 64, torch.float16, seed=4)
    sinks = torch.tensor([0.5, -1.0, 2.0, 0.0])
    check(run_case(case, sinks=sinks.to(DEV)), oracle_case(case, sinks=sinks), torch.float16)


def test_page_relocation_is_bitwise_invariant():
    """Moving pages to other physical slots (and rewriting the table) must not change a bit."""
    case = paged_decode_case([100, 2000, 4097], 32, 8, 128, torch.bfloat16, seed=12)
    out1 = run_case(case)
    cap = case['capacity']
    perm = torch.randperm(cap, generator=torch.Generator().manual_seed(1))
    moved = dict(case)
    moved['cache_k'] = torch.empty_like(case['cache_k'])
    moved['cache_v'] = torch.empty_like(case['cache_v'])
    moved['cache_k'][perm] = case['cache_k']
    moved['cache_v'][perm] = case['cache_v']
    t = case['page_table'].long()
    moved['page_table'] = torch.where(t >= 0, perm[t.clamp_min(0)], t).to(torch.int32)
    out2 = run_case(moved)
    assert torch.equal(out1, out2)


def test_scratch_bytes_partitions_rows():
    case = paged_decode_case([700, 50, 1800, 33, 900], 8, 2, 128, torch.float16, seed=21)
    part = run_case(case, scratch_bytes=8 * (4 * (128 + 1) * 4 + 128 * 2) * 2)
    check(part, oracle_case(case), torch.float16)


@pytest.mark.parametrize('batch', [65, 128, 200, 256, 257])
@pytest.mark.parametrize('window', [0, 300])
@pytest.mark.parametrize('kind', ['bf16', 'int8'])
def test_many_sequences_launch_order(batch, window, kind):
    """Batches across the in-kernel launch order's word boundaries (64
    sequences per wave) and past its 256-sequence limit, with contexts that
    end exactly on a split boundary, inside the first split and past it."""
    g = torch.Generator().manual_seed(batch + window)
    split_tokens = kernels._splits(3072, batch * 2, 64, torch.int8 if kind == 'int8' else torch.bfloat16)[1]
    fixed = [1, split_tokens, 2 * split_tokens, split_tokens + 1, 3072]
    contexts = fixed + torch.randint(1, 3073, (batch - len(fixed),), generator=g).tolist()
    case = paged_decode_case(contexts, 8, 2, 64, torch.float32 if kind == 'int8' else torch.bfloat16,
                             seed=batch, table_width=192)
    if kind == 'int8':
        qk, ks = oracle.quantize_q8(case['cache_k'], 64)
        qv, vs = oracle.quantize_q8(case['cache_v'], 64)
        case.update(cache_k=qk, cache_v=qv, k_scale=ks, v_scale=vs, query=case['query'].to(torch.bfloat16))
    kw = {'window': window} if window else {}
    check(run_case(case, **kw), oracle_case(case, **kw), torch.int8 if kind == 'int8' else torch.bfloat16)


def test_config_c2_bf16_rows():
    """Full 64-sequence bf16 decode, every row against the oracle."""
    contexts = uniform_contexts(64, 512, 8192, 2)
    case = paged_decode_case(contexts, 32, 8, 128, torch.bfloat16, seed=2, device=DEV, table_width=512)
    out = kernels.attention(case['query'], case['cache_k'], case['cache_v'], case['positions'], case['slots'],
                            page_table=case['page_table'])
    rows = list(range(64))
    cpu = {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in case.items()}
    expected = oracle_case(cpu, rows=rows)
    err = check(out, expected, torch.bfloat16, rows=rows)
    assert err <= 2e-3


def test_config_c5_long_context_outliers():
    """16 x 32768 tokens, D=256, 8 query heads per KV head, 1% K outliers x8."""
    ctx = [32768] * 16
    case = paged_decode_case(ctx, 16, 2, 256, torch.bfloat16, seed=5, device=DEV, capacity=16 * 2048,
                             outlier_frac=0.01)
    out = kernels.attention(case['query'], case['cache_k'], case['cache_v'], case['positions'], case['slots'],
                            page_table=case['page_table'])
    rows = list(range(16))
    cpu = {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in case.items()}
    expected = oracle_case(cpu, rows=rows)
    check(out, expected, torch.bfloat16, rows=rows)


def test_int8_wide_group():
    """int8 pages with 20 query heads per KV head (workgroups of <= 16 heads)."""
    case = paged_decode_case([9, 700, 2100], 40, 2, 128, torch.float32, seed=40)
    qk, ks = oracle.quantize_q8(case['cache_k'], 128)
    qv, vs = oracle.quantize_q8(case['cache_v'], 128)
    case.update(cache_k=qk, cache_v=qv, k_scale=ks, v_scale=vs, query=case['query'].to(torch.bfloat16))
    check(run_case(case), oracle_case(case), torch.int8)


def test_config_c3_int8_full_batch():
    """BASELINE config C3 at full size: 64 sequences, int8 pages with one fp16
    scale per (token, KV head) quantised on the GPU; every row against the oracle."""
    from damendaemon_amd import kv_quant
    from damendaemon_amd.workloads import config_c2, quantize_pages
    case = quantize_pages(config_c2(device=DEV), 128, kv_quant)
    out = kernels.attention(case['query'], case['cache_k'], case['cache_v'], case['positions'], case['slots'],
                            page_table=case['page_table'], k_scale=case['k_scale'], v_scale=case['v_scale'])
    rows = list(range(64))
    cpu = {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in case.items()}
    expected = oracle_case(cpu, rows=rows)
    check(out, expected, torch.int8, rows=rows)

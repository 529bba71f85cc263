"""Chunked-prefill and mixed-batch attention on the GPU against the CPU oracle.

Tolerance: max |gpu - oracle| <= 2e-3 + half an ulp of the reference value
in the output dtype.  The oracle is the reference's prefill arithmetic
(softmax(q.k * scale) . v, qwen2.py:754-770 / device.py:65-80) in float64;
the kernel accumulates in fp32, carries the probabilities into P.V at ~17
bits, and rounds the result once to the output dtype.
"""
import math
import random

import pytest
import torch

from _bounds import excess, half_ulp
from damendaemon_amd import packing, ragged
from damendaemon_amd.workloads import paged_decode_case
from oracle import paged_oracle as O

pytestmark = pytest.mark.gpu
DEV = 'cuda'
ATOL = 2e-3


def check(actual, expected, atol=ATOL):
    worst, err = excess(actual, expected, atol, actual.dtype)
    print(f'max abs err {err:.3e} (margin {-worst:.3e})')
    assert worst <= 0, f'max abs err {err:.3e} exceeds {atol} + half-ulp by {worst:.3e}'
    return err


def build(lengths, starts, heads, kvh, dim, dtype, seed, nan_fill=True, page=16):
    contexts = [s + n for s, n in zip(starts, lengths)]
    case = paged_decode_case(contexts, heads, kvh, dim, dtype, seed=seed, nan_fill=nan_fill, page=page)
    g = torch.Generator().manual_seed(seed + 1)
    q = torch.randn(sum(lengths), heads, dim, generator=g).to(dtype)
    slots = list(range(len(lengths)))
    return case, q, slots


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16])
@pytest.mark.parametrize('dim,heads,kvh', [(128, 32, 8), (64, 8, 2), (128, 14, 2), (256, 16, 2), (128, 8, 8)])
def test_prefill_segments(dtype, dim, heads, kvh):
    lengths = [1, 17, 64, 100, 33]
    starts = [0, 5, 0, 300, 1000]
    case, q, slots = build(lengths, starts, heads, kvh, dim, dtype, seed=dim + heads)
    packed = packing.pack_batch(lengths, starts, slots, case['page_table'].to(DEV))
    out = ragged.prefill_attention(q.to(DEV), case['cache_k'].to(DEV), case['cache_v'].to(DEV), packed,
                                   case['page_table'].to(DEV))
    exp = O.prefill_attention(q, case['cache_k'], case['cache_v'], lengths, starts, slots, case['page_table'])
    check(out, exp)


@pytest.mark.parametrize('window', [1, 40, 200])
def test_prefill_window(window):
    lengths = [50, 129]
    starts = [0, 400]
    case, q, slots = build(lengths, starts, 8, 2, 128, torch.bfloat16, seed=window)
    packed = packing.pack_batch(lengths, starts, slots, case['page_table'].to(DEV))
    out = ragged.prefill_attention(q.to(DEV), case['cache_k'].to(DEV), case['cache_v'].to(DEV), packed,
                                   case['page_table'].to(DEV), window=window)
    exp = O.prefill_attention(q, case['cache_k'], case['cache_v'], lengths, starts, slots, case['page_table'],
                              window=window)
    check(out, exp)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16])
@pytest.mark.parametrize('slope', [0.5, -0.5, 0.02])
def test_prefill_running_max_moves(dtype, slope):
    """Scores that rise (or fall) steeply along the keys: with slope 0.5 every
    64-key tile exceeds the running max by far more than the fp16 range of the
    probabilities, so each tile takes the kernel's re-offset path; slope 0.02
    moves the max a little on every tile."""
    lengths, starts = [64, 200], [0, 700]
    heads, kvh, dim = 8, 2, 128
    case, q, slots = build(lengths, starts, heads, kvh, dim, dtype, seed=77, nan_fill=False)
    u = torch.ones(dim) / dim ** 0.5
    g = torch.Generator().manual_seed(78)
    q = (4 * u + 0.05 * torch.randn(sum(lengths), heads, dim, generator=g)).to(dtype)
    ck, table = case['cache_k'], case['page_table']
    for slot, (n, st) in enumerate(zip(lengths, starts)):
        for j in range(st + n):
            page = int(table[slot, j // 16])
            ck[page, :, j % 16] = (slope * j * u + 0.05 * torch.randn(kvh, dim, generator=g)).to(dtype)
    packed = packing.pack_batch(lengths, starts, slots, table.to(DEV))
    out = ragged.prefill_attention(q.to(DEV), ck.to(DEV), case['cache_v'].to(DEV), packed, table.to(DEV))
    exp = O.prefill_attention(q, ck, case['cache_v'], lengths, starts, slots, table)
    check(out, exp)


@pytest.mark.parametrize('dim,dtype', [(128, torch.bfloat16), (256, torch.bfloat16), (96, torch.float16),
                                       (64, torch.float16), (160, torch.bfloat16), (144, torch.float16),
                                       (80, torch.bfloat16)])
def test_mixed_batch_end_to_end(dim, dtype):
    """Config C4 at reduced size: pack on the GPU, write the new K/V into the pages, attend
    (prefill chunks and decode rows on their two streams), at head sizes 64-256 including
    160 and 144 (the prefill kernel's 160 layout) and 80 (the prefill's 128 layout, the
    decode's 96 layout)."""
    rng = random.Random(4 + dim)
    heads, kvh = 32, 8
    starts = [rng.randint(0, 1024) for _ in range(3)] + [rng.randint(256, 2048) - 1 for _ in range(20)]
    lengths = [128] * 3 + [1] * 20
    contexts = [s + n for s, n in zip(starts, lengths)]
    case = paged_decode_case(contexts, heads, kvh, dim, dtype, seed=44, nan_fill=True)
    g = torch.Generator().manual_seed(45)
    T = sum(lengths)
    q = torch.randn(T, heads, dim, generator=g).to(dtype)
    k_new = torch.randn(T, kvh, dim, generator=g).to(dtype)
    v_new = torch.randn(T, kvh, dim, generator=g).to(dtype)
    slots = list(range(len(lengths)))
    table = case['page_table'].to(DEV)
    ck, cv = case['cache_k'].to(DEV), case['cache_v'].to(DEV)
    packed = packing.pack_batch(lengths, starts, slots, table)
    packing.store_kv_pages(k_new.to(DEV), v_new.to(DEV), packed.slot_map, ck, cv)
    out = ragged.ragged_attention(q.to(DEV), ck, cv, packed, table)
    # oracle: same page writes on the CPU, then float64 attention
    cpu_k, cpu_v = case['cache_k'].clone(), case['cache_v'].clone()
    for t, s in enumerate(O.pack_batch(lengths, starts, slots, case['page_table'])['slot_map']):
        cpu_k[s // 16, :, s % 16] = k_new[t]
        cpu_v[s // 16, :, s % 16] = v_new[t]
    assert torch.equal(ck.cpu().nan_to_num(3.), cpu_k.nan_to_num(3.))
    exp = O.prefill_attention(q, cpu_k, cpu_v, lengths, starts, slots, case['page_table'])
    case.update(cache_k=cpu_k, cache_v=cpu_v)
    check(out, exp)


def run_segments(lengths, starts, heads, kvh, dim, dtype, seed, window=0, scale=None, nan_fill=True, page=16):
    case, q, slots = build(lengths, starts, heads, kvh, dim, dtype, seed=seed, nan_fill=nan_fill, page=page)
    table = case['page_table'].to(DEV)
    packed = packing.pack_batch(lengths, starts, slots, table, page_size=page)
    out = ragged.prefill_attention(q.to(DEV), case['cache_k'].to(DEV), case['cache_v'].to(DEV), packed, table,
                                   window=window, scale=scale)
    exp = O.prefill_attention(q, case['cache_k'], case['cache_v'], lengths, starts, slots, case['page_table'],
                              window=window, scale=scale)
    return out, exp


@pytest.mark.parametrize('dim', [64, 96, 128])
@pytest.mark.parametrize('window', [0, 45])
def test_prefill_fp32_pages(dim, window):
    """fp32 compute dtype (qwen2.py:403-409): the fp32-arithmetic MFMA kernel
    (prefill_f32_kernel) at every head size here, fp32 bound."""
    out, exp = run_segments([1, 30, 70, 129], [0, 7, 300, 20], 8, 2, dim, torch.float32, seed=dim + window,
                            window=window)
    check(out, exp, atol=2e-5)


@pytest.mark.parametrize('dim', [64, 128])
@pytest.mark.parametrize('heads,kvh', [(4, 4), (14, 2), (32, 2), (128, 1), (130, 1)])
@pytest.mark.parametrize('page,window,scale', [(16, 0, None), (64, 0, None), (32, 77, -0.09)])
def test_prefill_fp32_groups_pages(dim, heads, kvh, page, window, scale):
    """fp32 pages on the matrix-core kernel across GQA widths (128 columns of
    (query row, head) per workgroup: 1 to 128 heads per KV head; 130 takes the
    vector-ALU kernel), page sizes, a window and a negative scale."""
    lengths = [1, 9, 130, 61] if heads <= 32 else [1, 9, 40]
    starts = [0, 33, 500, 31] if heads <= 32 else [0, 33, 200]
    out, exp = run_segments(lengths, starts, heads, kvh, dim, torch.float32, seed=heads + dim + page,
                            window=window, scale=scale, page=page)
    check(out, exp, atol=2e-5)


@pytest.mark.parametrize('dim', [16, 48, 112, 160, 176, 192, 240, 256])
@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16, torch.float16])
def test_prefill_fp32_arithmetic_head_sizes(dim, dtype):
    """Head sizes in steps of 16: fp32 pages on the fp32-arithmetic matrix-core kernel at
    every one; 16-bit pages on it at D 16, on the 16-bit kernels' 64 / 128 layouts at
    D 48 / 112 and on the 256 layout above 128."""
    out, exp = run_segments([1, 45, 100], [0, 70, 260], 12, 4, dim, dtype, seed=dim + 3, window=90)
    check(out, exp, atol=2e-5 if dtype == torch.float32 else 2e-3)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16])
@pytest.mark.parametrize('dim', [96, 80, 112, 48])
def test_prefill_other_head_sizes(dtype, dim):
    """Head sizes the 16-bit MFMA kernel takes inside its 64 / 128 layouts
    (the dims past the real head size are zeros no MFMA reads)."""
    out, exp = run_segments([3, 64, 100], [0, 200, 17], 12, 4, dim, dtype, seed=dim)
    check(out, exp)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16])
@pytest.mark.parametrize('dim', [144, 160, 176, 192, 208, 224, 240])
def test_prefill_wide_head_sizes(dtype, dim):
    """Head sizes between 128 and 256 on the 16-bit kernel's 160 and 256
    layouts (rows of the real length; the dims past it are zeros the MFMAs
    skip)."""
    out, exp = run_segments([3, 64, 100], [0, 200, 17], 12, 4, dim, dtype, seed=dim)
    check(out, exp)


@pytest.mark.parametrize('dim', [144, 160, 224, 256])
@pytest.mark.parametrize('page,window,heads,kvh', [(16, 0, 32, 8), (32, 70, 8, 1), (16, 0, 40, 2),
                                                   (16, 300, 130, 1)])
def test_prefill_wide_head_sizes_pages_windows(dim, page, window, heads, kvh):
    """The 160 and 256 layouts with larger pages, windows, wide groups, and
    130 query heads per KV head (at 224 and 256 more than the 128-column work
    item: the exact kernel)."""
    lengths = [1, 77, 200] if heads <= 40 else [1, 9, 40]
    starts = [5, 0, 1500] if heads <= 40 else [0, 17, 100]
    out, exp = run_segments(lengths, starts, heads, kvh, dim, torch.bfloat16, seed=dim + page + window + heads,
                            window=window, page=page)
    check(out, exp)


@pytest.mark.parametrize('dim', [96, 80, 64, 48])
@pytest.mark.parametrize('page,window,heads,kvh', [(16, 0, 32, 8), (32, 70, 8, 1), (64, 200, 4, 2), (16, 300, 130, 1)])
def test_prefill_other_head_sizes_pages_windows(dim, page, window, heads, kvh):
    """The 128 layout at 96 and 80 dims, the 64 layout (128-key tiles) at 64 and 48: larger
    pages, windows, and 130 query heads per KV head (one query row per work item)."""
    lengths = [1, 77, 200] if heads <= 32 else [1, 9, 40]
    starts = [5, 0, 1500] if heads <= 32 else [0, 17, 100]
    out, exp = run_segments(lengths, starts, heads, kvh, dim, torch.bfloat16, seed=dim + page + window,
                            window=window, page=page)
    check(out, exp)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_prefill_negative_scale(dtype):
    """SDPA accepts any scale; a negative one turns the softmax around."""
    out, exp = run_segments([40, 90], [0, 150], 8, 2, 128, dtype, seed=3, scale=-0.07)
    check(out, exp, atol=2e-3 if dtype != torch.float32 else 2e-5)


@pytest.mark.parametrize('heads,kvh', [(40, 2), (64, 2), (34, 1)])
def test_prefill_wide_groups(heads, kvh):
    """More than 16 query heads per KV head."""
    out, exp = run_segments([5, 77], [0, 260], heads, kvh, 128, torch.bfloat16, seed=heads)
    check(out, exp)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_prefill_history_past_table_cache(dtype):
    """A history longer than the page-table entries the MFMA kernels stage in
    LDS (8192 at D 256, 3584 at D 64 / 128; 131072 / 57344 tokens at page 16):
    the rest come from the table."""
    start = 8192 * 16 + 300
    lengths, starts = [50, 20], [start, 1000]
    out, exp = run_segments(lengths, starts, 4, 1, 64, dtype, seed=9, nan_fill=False)
    check(out, exp, atol=2e-3 if dtype != torch.float32 else 2e-5)
    # a window that starts past the cached entries
    out, exp = run_segments(lengths, starts, 4, 1, 64, dtype, seed=9, window=500, nan_fill=False)
    check(out, exp, atol=2e-3 if dtype != torch.float32 else 2e-5)


def test_prefill_rejects_bad_scale_and_out():
    lengths, starts = [4], [0]
    case, q, slots = build(lengths, starts, 4, 2, 64, torch.bfloat16, seed=1)
    table = case['page_table'].to(DEV)
    packed = packing.pack_batch(lengths, starts, slots, table)
    args = (q.to(DEV), case['cache_k'].to(DEV), case['cache_v'].to(DEV), packed, table)
    for bad in (float('inf'), float('nan'), float('-inf')):
        with pytest.raises(ValueError):
            ragged.prefill_attention(*args, scale=bad)
    wrong = torch.empty(4, 64, 4, dtype=torch.bfloat16, device=DEV).transpose(1, 2)
    with pytest.raises(ValueError):
        ragged.prefill_attention(*args, out=wrong)
    with pytest.raises(ValueError):
        ragged.prefill_attention(*args, out=torch.empty(4, 4, 64, dtype=torch.float16, device=DEV))


def test_config_c4_full_batch():
    """BASELINE config C4 at full size: 8 x 512-token chunks on U[0,4096]
    histories plus 120 decodes on U[256,8192], packed and written on the GPU.
    Every chunk and every decode row against the oracle."""
    from damendaemon_amd.workloads import config_c4
    case = config_c4(device=DEV)
    lengths, starts, slots = case['lengths'], case['starts'], case['seg_slots']
    table = case['page_table']
    packed = packing.pack_batch(lengths, starts, slots, table)
    packing.store_kv_pages(case['k_new'], case['v_new'], packed.slot_map, case['cache_k'], case['cache_v'])
    out = ragged.ragged_attention(case['q'], case['cache_k'], case['cache_v'], packed, table)
    torch.cuda.synchronize()
    ck, cv, tab, q = case['cache_k'].cpu(), case['cache_v'].cpu(), table.cpu(), case['q'].cpu()
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    for seg in range(len(lengths)):
        rows = slice(cu[seg], cu[seg + 1])
        exp = O.prefill_attention(q[rows], ck, cv, [lengths[seg]], [starts[seg]], [slots[seg]], tab)
        check(out[rows], exp)


def _relative_error(out, exp, exp_abs):
    """max |out - exp| less the bf16 output's half ulp, relative to each row's
    largest sum p|v| (``exp_abs``: the same attention over |V|).  A weighted
    sum with weights good to a relative e is good to e * sum p|v|; the
    output row itself can cancel far below that."""
    a = out.cpu().double()
    assert torch.isfinite(a).all(), 'non-finite output'
    row_mag = exp_abs.amax(dim=-1, keepdim=True).clamp_min(1e-300)
    return (((a - exp).abs() - half_ulp(exp, torch.bfloat16)) / row_mag).max().item()


def _scaled_v_case(lengths, starts, heads, kvh, dim, seed, magnitude):
    """bf16 pages whose V is N(0,1) times ``magnitude(shape)`` per
    (page, KV head, token) row."""
    case, q, slots = build(lengths, starts, heads, kvh, dim, torch.bfloat16, seed=seed)
    cv = case['cache_v'].double()
    mag = magnitude(cv.shape[:3] + (1,))
    case['cache_v'] = (cv * mag).to(torch.bfloat16)
    return case, q, slots


@pytest.mark.parametrize('dim,heads,kvh', [(128, 16, 4), (64, 8, 2), (128, 130, 1), (96, 16, 4), (256, 16, 2),
                                            (160, 16, 4)])
@pytest.mark.parametrize('spread', ['rows', 1e-6, 1e-5, 3e-3, 2e5, 1e6])
def test_prefill_bf16_value_range(dim, heads, kvh, spread):
    """bf16 V over the whole bf16 range that matters: per-row magnitudes
    log-uniform in 1e-6 .. 1e6 within one segment ('rows'), or a whole cache
    scaled by one factor (tiny values that fp16 holds only as subnormals, and
    values past fp16's 65504).  The reference upcasts to fp32
    (kernels.py:150,158,177; SDPA in fp32 accumulation), so no magnitude may
    cost accuracy: bound 2e-3 of each row's largest sum p|v| plus the bf16
    output's half ulp."""
    lengths = [1, 40, 129, 300] if heads <= 16 else [1, 9, 40]
    starts = [0, 3, 500, 70] if heads <= 16 else [0, 17, 100]
    seed = dim + heads + (7 if spread == 'rows' else int(abs(math.log10(spread)) * 10))
    g = torch.Generator().manual_seed(seed)
    if spread == 'rows':
        magnitude = lambda shape: torch.exp(torch.empty(shape, dtype=torch.float64).uniform_(
            math.log(1e-6), math.log(1e6), generator=g))
    else:
        magnitude = lambda shape: torch.full(shape, float(spread), dtype=torch.float64)
    case, q, slots = _scaled_v_case(lengths, starts, heads, kvh, dim, seed, magnitude)
    table = case['page_table'].to(DEV)
    packed = packing.pack_batch(lengths, starts, slots, table)
    out = ragged.prefill_attention(q.to(DEV), case['cache_k'].to(DEV), case['cache_v'].to(DEV), packed, table)
    exp = O.prefill_attention(q, case['cache_k'], case['cache_v'], lengths, starts, slots, case['page_table'])
    exp_abs = O.prefill_attention(q, case['cache_k'], case['cache_v'].abs(), lengths, starts, slots,
                                  case['page_table'])
    err = _relative_error(out, exp, exp_abs)
    print(f'max error {err:.3e} of the row magnitude')
    assert err <= 2e-3, f'max error {err:.3e} of the row magnitude'


def test_prefill_bf16_one_huge_key():
    """One key of V beyond fp16's range in an otherwise N(0,1) segment: every
    row that can see it and every row that cannot (same tiles) stays exact."""
    lengths, starts = [200], [100]
    case, q, slots = build(lengths, starts, 8, 2, 128, torch.bfloat16, seed=91, nan_fill=True)
    table = case['page_table']
    j = 150                      # a history key inside the chunk's first tiles
    case['cache_v'][int(table[0, j // 16]), 1, j % 16] *= 3e5
    packed = packing.pack_batch(lengths, starts, slots, table.to(DEV))
    out = ragged.prefill_attention(q.to(DEV), case['cache_k'].to(DEV), case['cache_v'].to(DEV), packed,
                                   table.to(DEV))
    exp = O.prefill_attention(q, case['cache_k'], case['cache_v'], lengths, starts, slots, table)
    exp_abs = O.prefill_attention(q, case['cache_k'], case['cache_v'].abs(), lengths, starts, slots, table)
    err = _relative_error(out, exp, exp_abs)
    assert err <= 2e-3, f'max error {err:.3e} of the row magnitude'


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize('dim', [64, 128, 256, 96, 160])
def test_prefill_scale_zero(dtype, dim):
    """scale 0: every allowed key gets the same weight (SDPA's result for a
    zero scale), windowed or not."""
    lengths, starts = [1, 33, 90], [0, 60, 7]
    for window in (0, 20):
        case, q, slots = build(lengths, starts, 8, 2, dim, dtype, seed=dim + window)
        table = case['page_table'].to(DEV)
        packed = packing.pack_batch(lengths, starts, slots, table)
        out = ragged.prefill_attention(q.to(DEV), case['cache_k'].to(DEV), case['cache_v'].to(DEV), packed, table,
                                       window=window, scale=0.0)
        exp = O.prefill_attention(q, case['cache_k'], case['cache_v'], lengths, starts, slots,
                                  case['page_table'], window=window, scale=0.0)
        check(out, exp, atol=2e-5 if dtype == torch.float32 else ATOL)


def test_prefill_bf16_rerun_flags_fire_only_where_needed():
    """The bf16 kernel flags exactly the work items whose V leaves fp16's
    range (here: one KV head of one segment) and none on N(0,1) data."""
    lengths, starts = [300, 70], [40, 900]
    heads, kvh, dim = 16, 4, 128
    case, q, slots = build(lengths, starts, heads, kvh, dim, torch.bfloat16, seed=5)
    table = case['page_table'].to(DEV)
    packed = packing.pack_batch(lengths, starts, slots, table)
    n = ragged.prefill_flag_count(2, 300, heads, kvh, dim, torch.bfloat16)
    rows = 256 // (heads // kvh)
    tiles = -(-300 // rows)
    assert n == 2 * kvh * tiles
    flags = torch.full((n,), 7, dtype=torch.int32, device=DEV)
    args = (q.to(DEV), case['cache_k'].to(DEV))
    ragged.prefill_attention(*args, case['cache_v'].to(DEV), packed, table, flags=flags)
    valid = [(g * tiles + t) for g in range(2 * kvh) for t in range(-(-lengths[g // kvh] // rows))]
    assert flags.cpu()[valid].eq(0).all()
    # segment 1, KV head 2: one history key past fp16's range
    cv = case['cache_v'].clone()
    cv[int(case['page_table'][1, 5]), 2, 3] = 1e6
    out = ragged.prefill_attention(*args, cv.to(DEV), packed, table, flags=flags)
    got = flags.cpu()
    hot = {(1 * kvh + 2) * tiles + t for t in range(-(-lengths[1] // rows))}
    assert all(got[i] == (1 if i in hot else 0) for i in valid), got
    exp = O.prefill_attention(q, case['cache_k'], cv, lengths, starts, slots, case['page_table'])
    exp_abs = O.prefill_attention(q, case['cache_k'], cv.abs(), lengths, starts, slots, case['page_table'])
    assert _relative_error(out, exp, exp_abs) <= 2e-3


def test_prefill_phases_equal_one_call():
    """dd_prefill_attention_phase 1 then 2 gives dd_prefill_attention's
    output bit for bit, also when the re-run has items to redo."""
    lengths, starts = [130, 40], [300, 0]
    case, q, slots = build(lengths, starts, 16, 4, 128, torch.bfloat16, seed=13)
    cv = case['cache_v'].clone()
    cv[int(case['page_table'][0, 3]), 1, 5] = 2e5     # one item of segment 0 needs the re-run
    table = case['page_table'].to(DEV)
    packed = packing.pack_batch(lengths, starts, slots, table)
    args = (q.to(DEV), case['cache_k'].to(DEV), cv.to(DEV), packed, table)
    whole = ragged.prepare_prefill(*args).run().clone()
    launch = ragged.prepare_prefill(*args)
    launch.out.fill_(float('nan'))
    launch.phase(1)
    launch.phase(2)
    assert torch.equal(launch.out, whole)
    assert torch.isfinite(whole.float()).all()

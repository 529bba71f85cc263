"""Chunked-prefill and mixed-batch attention on the GPU against the CPU oracle.

Tolerance.  The kernel accumulates in fp32 but, like the reference's own
prefill path (torch flash SDPA on bf16/fp16 tensors, qwen2.py:754-770),
feeds the probabilities to the P.V product in the input dtype and rounds the
output to it.  The bound is therefore: max |gpu - oracle| <= max(2e-3,
1.25 * max |torch SDPA - oracle|), with torch SDPA run on the same gathered
bf16/fp16 K/V on the GPU (the reference's own arithmetic); for fp16 that is
always 2e-3 in practice, for bf16 the probabilities carry 8 bits.
"""
import random

import pytest
import torch

from damendaemon_amd import packing, ragged
from damendaemon_amd.workloads import paged_decode_case
from oracle import paged_oracle as O

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def sdpa_error(q, cache_k, cache_v, lengths, starts, slots, table, expected, window=0):
    """max |torch SDPA (GPU, input dtype) - oracle| over the same segments."""
    from torch.nn.attention.bias import causal_lower_right
    from torch.nn import functional as F
    worst, t0 = 0.0, 0
    for n, s, slot in zip(lengths, starts, slots):
        k = O.gather_pages(cache_k, table, slot, s + n)[None].to(DEV)
        v = O.gather_pages(cache_v, table, slot, s + n)[None].to(DEV)
        qq = q[t0:t0 + n].transpose(0, 1)[None].to(DEV)
        if window:
            qp = torch.arange(s, s + n, device=DEV)[:, None]
            kp = torch.arange(s + n, device=DEV)[None, :]
            mask = (kp <= qp) & (kp > qp - window)
        else:
            mask = causal_lower_right(n, s + n)
        ref = F.scaled_dot_product_attention(qq, k, v, attn_mask=mask, enable_gqa=True)[0].transpose(0, 1)
        worst = max(worst, (ref.double().cpu() - expected[t0:t0 + n]).abs().max().item())
        t0 += n
    return worst


def check(actual, expected, bound=2e-3):
    a = actual.detach().float().cpu().double()
    assert torch.isfinite(a).all()
    err = (a - expected).abs().max().item()
    assert err <= bound, f'max abs err {err:.3e} > {bound:.3e}'
    return err


def bound_for(q, case, lengths, starts, slots, expected, window=0):
    ref_err = sdpa_error(q, case['cache_k'], case['cache_v'], lengths, starts, slots, case['page_table'], expected,
                         window)
    return max(2e-3, 1.25 * ref_err)


def build(lengths, starts, heads, kvh, dim, dtype, seed, nan_fill=True):
    contexts = [s + n for s, n in zip(starts, lengths)]
    case = paged_decode_case(contexts, heads, kvh, dim, dtype, seed=seed, nan_fill=nan_fill)
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
    check(out, exp, bound_for(q, case, lengths, starts, slots, exp))


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
    check(out, exp, bound_for(q, case, lengths, starts, slots, exp, window))


def test_mixed_batch_end_to_end():
    """Config C4 at reduced size: pack on the GPU, write the new K/V into the pages, attend."""
    rng = random.Random(4)
    heads, kvh, dim = 32, 8, 128
    starts = [rng.randint(0, 1024) for _ in range(3)] + [rng.randint(256, 2048) - 1 for _ in range(20)]
    lengths = [128] * 3 + [1] * 20
    contexts = [s + n for s, n in zip(starts, lengths)]
    case = paged_decode_case(contexts, heads, kvh, dim, torch.bfloat16, seed=44, nan_fill=True)
    g = torch.Generator().manual_seed(45)
    T = sum(lengths)
    q = torch.randn(T, heads, dim, generator=g).to(torch.bfloat16)
    k_new = torch.randn(T, kvh, dim, generator=g).to(torch.bfloat16)
    v_new = torch.randn(T, kvh, dim, generator=g).to(torch.bfloat16)
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
    check(out, exp, bound_for(q, case, lengths, starts, slots, exp))

"""Pin the CPU oracle against things other than itself (library routines,
closed forms, known answers, brute force), so a dropped term, wrong index or
transposed operand in the oracle fails here before any GPU comparison."""
import math

import pytest
import torch
from torch.nn import functional as F

from damendaemon_amd.workloads import paged_decode_case
from oracle import paged_oracle as O


def test_gather_matches_page_concatenation():
    """scripts/verify_paged_copies.py:15-24 builds the expected dense tensor with torch.cat."""
    g = torch.Generator().manual_seed(927)
    for length in (1, 15, 16, 17, 127, 513):
        pages = torch.randperm(40, generator=g)[:(length + 15) // 16]
        table = torch.full((4, 33), -1, dtype=torch.int32)
        table[3, :len(pages)] = pages.to(torch.int32)
        cache = torch.randn((2, 40, 3, 16, 96), generator=g)
        dense = O.copy_pages(cache, table, 3, length)
        expected = torch.cat([cache[:, p] for p in pages.tolist()], dim=2)[:, :, :length]
        assert torch.equal(dense, expected)
        restored = O.copy_pages(torch.full_like(cache, 17.), table, 3, length, snapshot=dense)
        wanted = torch.full_like(cache, 17.)
        for block, p in enumerate(pages.tolist()):
            n = min(16, length - 16 * block)
            wanted[:, p, :, :n] = expected[:, :, 16 * block:16 * block + n]
        assert torch.equal(restored, wanted)


def test_quantize_known_answers():
    x = torch.zeros(2, 64)
    x[0, :32] = torch.linspace(-3, 3, 32)
    x[1, 32:] = 0.5
    q, s = O.quantize_q8(x, 32)
    assert s.dtype == torch.float16 and s.shape == (2, 2)
    assert s[0, 1] == 0 and (q[0, 32:] == 0).all()            # zero group -> zero scale, zero data
    assert s[1, 0] == 0 and (q[1, :32] == 0).all()
    assert q[0, 0] == -127 and q[0, 31] == 127                 # +-absmax -> +-127
    assert (q[1, 32:] == 127).all()
    assert s[0, 0] == torch.tensor(3 / 127).half()
    # exact halves round away from zero: scale 1 -> x/1
    y = torch.tensor([[127.0, 0.5, -0.5, 1.5, -2.5, 2.4999] + [0.0] * 26])
    qy, sy = O.quantize_q8(y, 32)
    assert float(sy[0, 0]) == 1.0
    assert qy[0, :6].tolist() == [127, 1, -1, 2, -3, 2]


def test_quantize_error_bound_and_dequant():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(50, 128, generator=g) * 3
    for group in (32, 64, 128):
        q, s = O.quantize_q8(x, group)
        back = O.dequantize_q8(q, s)
        sc = s.float().repeat_interleave(group, -1)
        # half a quantisation step, plus the fp16 rounding of the scale itself
        bound = sc / 2 + x.abs() * 2 ** -10 + 1e-7
        assert ((back - x).abs() <= bound).all()
    d = torch.tensor([[1, -2, 127, -127]], dtype=torch.int8)
    assert O.dequantize_q8(d, torch.tensor([[0.5]], dtype=torch.float16)).tolist() == [[0.5, -1.0, 63.5, -63.5]]


def _dense(case, b):
    pos = int(case['positions'][b])
    slot = int(case['slots'][b])
    k = torch.cat([case['cache_k'][int(p)] for p in case['page_table'][slot] if p >= 0], dim=1)[:, :pos + 1]
    v = torch.cat([case['cache_v'][int(p)] for p in case['page_table'][slot] if p >= 0], dim=1)[:, :pos + 1]
    return k, v


def test_decode_matches_sdpa_library():
    case = paged_decode_case([1, 17, 130, 400], 8, 2, 64, torch.float32, seed=4)
    out = O.decode_attention(case['query'], case['cache_k'], case['cache_v'], case['positions'], case['slots'],
                             page_table=case['page_table'])
    for b in range(4):
        k, v = _dense(case, b)
        ref = F.scaled_dot_product_attention(case['query'][b:b + 1].double(), k[None].double(), v[None].double(),
                                             enable_gqa=True)
        assert torch.allclose(out[b:b + 1], ref, atol=1e-12)


def test_decode_alibi_window_match_sdpa_with_mask():
    case = paged_decode_case([50, 333], 4, 2, 64, torch.float32, seed=5)
    alibi = torch.tensor([-0.1, -0.05, 0.02, 0.0])
    out = O.decode_attention(case['query'], case['cache_k'], case['cache_v'], case['positions'], case['slots'],
                             page_table=case['page_table'], alibi=alibi, window=40, scale=0.3)
    for b in range(2):
        k, v = _dense(case, b)
        n = k.shape[1]
        t = torch.arange(n, dtype=torch.float64)
        bias = alibi.double()[:, None] * t[None, :]
        bias = torch.where(t[None, :] > n - 1 - 40, bias, torch.tensor(-math.inf, dtype=torch.float64))
        ref = F.scaled_dot_product_attention(case['query'][b:b + 1].double(), k[None].double(), v[None].double(),
                                             attn_mask=bias[None, :, None, :], enable_gqa=True, scale=0.3)
        assert torch.allclose(out[b:b + 1], ref, atol=1e-12)


def test_decode_special_cases():
    case = paged_decode_case([1, 64, 200], 4, 4, 32, torch.float32, seed=6)
    args = (case['query'], case['cache_k'], case['cache_v'], case['positions'], case['slots'])
    base = O.decode_attention(*args, page_table=case['page_table'])
    # one live key -> its value vector
    assert torch.allclose(base[0, :, 0], case['cache_v'][int(case['page_table'][0, 0]), :, 0].double())
    # a window covering the context changes nothing; a sink of -inf changes nothing; zero alibi changes nothing
    for kw in ({'window': 10 ** 6}, {'sinks': torch.full((4,), -math.inf)}, {'alibi': torch.zeros(4)}):
        assert torch.allclose(O.decode_attention(*args, page_table=case['page_table'], **kw), base, atol=1e-12)
    # constant V rows -> that constant
    cv = torch.ones_like(case['cache_v']) * 0.25
    out = O.decode_attention(case['query'], case['cache_k'], cv, case['positions'], case['slots'],
                             page_table=case['page_table'])
    assert torch.allclose(out, torch.full_like(out, 0.25))
    # a sink of s shrinks the output by sum(w)/(sum(w)+e^s): check on a single key, logit irrelevant
    s = torch.tensor([0.0, 1.0, -1.0, 2.0])
    out = O.decode_attention(*args, page_table=case['page_table'], sinks=s)
    k, v = _dense(case, 0)
    logit = (case['query'][0, :, 0] * k[:, 0]).sum(-1) * 32 ** -.5
    factor = 1 / (1 + torch.exp(s - logit))
    assert torch.allclose(out[0, :, 0], (v[:, 0] * factor[:, None]).double(), atol=1e-6)


def test_t5_bucket_matches_transformers():
    t5 = pytest.importorskip('transformers.models.t5.modeling_t5')
    for buckets, maxd in ((32, 128), (8, 20), (64, 300)):
        rel = -torch.arange(0, 2000)[None, :]          # memory - query = t - pos <= 0
        lib = t5.T5Attention._relative_position_bucket(rel, bidirectional=False, num_buckets=buckets,
                                                       max_distance=maxd)[0].tolist()
        ours = [O.t5_bucket(n, buckets, maxd) for n in range(2000)]
        assert ours == lib


def test_sdpa_baseline_agrees_with_oracle():
    case = paged_decode_case([5, 40, 300, 77], 8, 2, 64, torch.float32, seed=8)
    a = O.decode_attention(case['query'], case['cache_k'], case['cache_v'], case['positions'], case['slots'],
                           page_table=case['page_table'])
    b = O.decode_attention_sdpa(case['query'], case['cache_k'], case['cache_v'], case['positions'], case['slots'],
                                case['page_table'])
    assert torch.allclose(a.float(), b, atol=2e-5)


def test_pack_known_answer():
    table = torch.tensor([[7, 3, 9, -1], [2, 5, -1, -1], [0, 1, 4, 6]], dtype=torch.int32)
    out = O.pack_batch([3, 1, 2], [15, 0, 33], [0, 1, 2], table, page=16)
    assert out['cu_seqlens'] == [0, 3, 4, 6]
    assert out['ends'] == [2, 3, 5]
    assert out['positions'] == [15, 16, 17, 0, 33, 34]
    assert out['slot_ids'] == [0, 0, 0, 1, 2, 2]
    assert out['slot_map'] == [7 * 16 + 15, 3 * 16 + 0, 3 * 16 + 1, 2 * 16, 4 * 16 + 1, 4 * 16 + 2]
    assert out['context_lens'] == [18, 1, 35]
    assert out['cu_pages'] == [0, 2, 3, 6]
    assert out['gather_pages'] == [7, 3, 2, 0, 1, 4]


def test_rope_precise_matches_closed_form():
    """scripts/verify_paged_kernels.py:40-43 and verify_kernels.py:103-110 closed forms."""
    g = torch.Generator().manual_seed(3)
    for D, RD in ((64, 64), (96, 96), (128, 64)):
        x = torch.randn(5, D, generator=g)
        ang = torch.randn(5, RD // 2, generator=g)
        ang = torch.cat((ang, ang), -1)
        cos, sin = ang.cos(), ang.sin()
        got = O.rope_rows(x, cos, sin, precise=True)
        xr = x[:, :RD]
        a, b = xr.chunk(2, -1)
        want = torch.cat((xr * cos + torch.cat((-b, a), -1) * sin, x[:, RD:]), -1)
        assert torch.allclose(got, want, atol=1e-6)
        if RD == D:
            w = torch.randn(D, generator=g)
            got = O.rope_rows(x, cos, sin, weight=w, precise=True)
            xn = x * torch.rsqrt(x.square().mean(-1, keepdim=True) + 1e-6) * w
            a, b = xn.chunk(2, -1)
            assert torch.allclose(got, xn * cos + torch.cat((-b, a), -1) * sin, atol=1e-5)


def test_rope_rounding_points():
    # values whose products are exact in fp16: precise and rounded paths agree
    x = torch.tensor([[0.5, 1.0, -2.0, 0.25]])
    cos = torch.tensor([[1.0, 0.5, 0.5, 1.0]])
    sin = torch.tensor([[0.5, 0.25, 0.25, 0.5]])
    assert torch.equal(O.rope_rows(x, cos, sin), O.rope_rows(x, cos, sin, precise=True))
    # a product on an fp16 tie: 1 + 2^-11 rounds to 1 (even) before the add
    x = torch.tensor([[1.0 + 2 ** -11, 0.0]])
    cos = torch.tensor([[1.0, 1.0]])
    sin = torch.tensor([[0.0, 0.0]])
    assert O.rope_rows(x, cos, sin)[0, 0].item() == 1.0
    assert O.rope_rows(x, cos, sin, precise=True)[0, 0].item() == 1.0 + 2 ** -11


def test_prefill_oracle_matches_sdpa_lower_right():
    from torch.nn.attention.bias import causal_lower_right
    case = paged_decode_case([40, 100], 4, 2, 32, torch.float32, seed=11)
    lengths, starts, slots = [7, 30], [33, 70], [0, 1]
    g = torch.Generator().manual_seed(2)
    q = torch.randn(sum(lengths), 4, 32, generator=g)
    out = O.prefill_attention(q, case['cache_k'], case['cache_v'], lengths, starts, slots, case['page_table'])
    t0 = 0
    for n, s, slot in zip(lengths, starts, slots):
        k = O.gather_pages(case['cache_k'], case['page_table'], slot, s + n)[None].double()
        v = O.gather_pages(case['cache_v'], case['page_table'], slot, s + n)[None].double()
        qq = q[t0:t0 + n].transpose(0, 1)[None].double()
        ref = F.scaled_dot_product_attention(qq, k, v, attn_mask=causal_lower_right(n, s + n), enable_gqa=True)
        assert torch.allclose(out[t0:t0 + n], ref[0].transpose(0, 1), atol=1e-12)
        t0 += n


def test_prefill_sdpa_baseline_matches_oracle():
    """The vectorised fp32 gather + SDPA prefill (bench.py's CPU baseline of
    the mixed batch) against the float64 loop, GQA 4:1, histories spanning
    several pages, a single-row segment and a segment without history."""
    case = paged_decode_case([1, 47, 300, 33], 8, 2, 64, torch.float32, seed=13)
    lengths, starts, slots = [1, 40, 129, 33], [0, 7, 171, 0], [0, 1, 2, 3]
    g = torch.Generator().manual_seed(4)
    q = torch.randn(sum(lengths), 8, 64, generator=g)
    want = O.prefill_attention(q, case['cache_k'], case['cache_v'], lengths, starts, slots, case['page_table'])
    got = O.prefill_attention_sdpa(q, case['cache_k'], case['cache_v'], lengths, starts, slots, case['page_table'])
    assert got.dtype == torch.float32 and torch.allclose(got.double(), want, atol=2e-6)


@pytest.mark.parametrize('window', [1, 5, 33, 200])
def test_prefill_oracle_window_matches_sdpa_explicit_mask(window):
    """The windowed prefill of qwen2.py:765-770: keys with kpos <= qpos and
    kpos > qpos - window, built as an explicit SDPA mask (the construction of
    the reference's tests/test_prefill.py:22-30)."""
    case = paged_decode_case([60, 230], 4, 2, 32, torch.float32, seed=12)
    lengths, starts, slots = [20, 45], [40, 185], [0, 1]
    g = torch.Generator().manual_seed(3)
    q = torch.randn(sum(lengths), 4, 32, generator=g)
    out = O.prefill_attention(q, case['cache_k'], case['cache_v'], lengths, starts, slots, case['page_table'],
                              window=window)
    t0 = 0
    for n, s, slot in zip(lengths, starts, slots):
        k = O.gather_pages(case['cache_k'], case['page_table'], slot, s + n)[None].double()
        v = O.gather_pages(case['cache_v'], case['page_table'], slot, s + n)[None].double()
        qq = q[t0:t0 + n].transpose(0, 1)[None].double()
        qpos = torch.arange(s, s + n)[:, None]
        kpos = torch.arange(s + n)[None, :]
        mask = (kpos <= qpos) & (kpos > qpos - window)
        ref = F.scaled_dot_product_attention(qq, k, v, attn_mask=mask, enable_gqa=True)
        assert torch.allclose(out[t0:t0 + n], ref[0].transpose(0, 1), atol=1e-12)
        t0 += n
    # window 1: every row sees only its own key, so the output is that key's value
    if window == 1:
        v0 = O.gather_pages(case['cache_v'], case['page_table'], 0, 60)
        assert torch.allclose(out[0, :, :], v0[:, 40].double().repeat_interleave(2, 0), atol=1e-12)

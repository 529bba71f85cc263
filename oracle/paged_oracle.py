"""CPU oracle for the paged-attention hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or the timed
CPU baseline), never as the product path.  The product path is the HIP
library; it has no CPU fallback.

Each function restates the reference semantics it cites, in plain torch
(CPU) / Python, in float64 unless stated, written for clarity rather than
speed.  How each function is pinned (checked against something other than
itself) is listed in ``PINNING`` at the bottom and exercised by
``tests/test_oracle.py``.
"""
import math

import torch
from torch.nn import functional as F


# ---------------------------------------------------------------------------
# a8: page gather (damendaemon/paged_kernels.py:8-25)

def gather_pages(plane, table, slot, tokens):
    """Logical (KH, tokens, D) view of one sequence from a paged plane.

    ``plane`` is (capacity, KH, page, D).  Token t lives in physical page
    ``table[slot, t // page]`` at row ``t % page`` (paged_kernels.py:17-19).
    """
    page = plane.shape[2]
    out = []
    for t in range(tokens):
        phys = int(table[slot, t // page])
        out.append(plane[phys, :, t % page, :])
    if not out:
        return plane.new_zeros((plane.shape[1], 0, plane.shape[3]))
    return torch.stack(out, dim=1)


def copy_pages(cache, table, slot, tokens, snapshot=None):
    """Gather (2, KH, tokens, D) or restore it (paged_kernels.py:28-47)."""
    if snapshot is None:
        return torch.stack([gather_pages(cache[i], table, slot, tokens) for i in range(2)])
    page = cache.shape[3]
    out = cache.clone()
    for t in range(tokens):
        phys = int(table[slot, t // page])
        out[:, phys, :, t % page, :] = snapshot[:, :, t, :]
    return out


# ---------------------------------------------------------------------------
# a10: Q8_0 codec (damendaemon/kv_quant.py:23-76), generalised group

def group_for(dim):
    """Reference channel group: gcd(dim, 32) (kv_quant.py:23-31)."""
    return math.gcd(int(dim), 32)


def quantize_q8(values, group):
    """Symmetric int8 with one fp16 scale per ``group`` channels.

    scale = fp16(absmax / 127); inverse = 0 for a zero scale else
    1/float(scale); q = clamp(sign(x*inv) * floor(|x*inv| + 0.5), +-127)
    (kv_quant.py:55-64).  Arithmetic in fp32 as the reference does.
    """
    dim = values.shape[-1]
    g = values.float().reshape(*values.shape[:-1], dim // group, group)
    scale = (g.abs().amax(-1) / 127).to(torch.float16)
    inv = torch.where(scale == 0, torch.zeros_like(scale, dtype=torch.float32), scale.float().reciprocal())
    x = g * inv.unsqueeze(-1)
    q = (x.sign() * torch.floor(x.abs() + .5)).clamp(-127, 127)
    return q.reshape(values.shape).to(torch.int8), scale


def dequantize_q8(data, scales):
    """int8 * float(scale) per group (kv_quant.py:67-76), fp32 result."""
    dim = data.shape[-1]
    group = dim // scales.shape[-1]
    x = data.float().reshape(*data.shape[:-1], dim // group, group) * scales.float().unsqueeze(-1)
    return x.reshape(data.shape)


# ---------------------------------------------------------------------------
# a6/a7: decode attention (damendaemon/kernels.py:134-267)

def t5_bucket(distance, buckets, max_distance):
    """T5 relative bucket of kernels.py:162-167 for one non-negative distance."""
    exact = buckets // 2
    if distance < exact:
        return distance
    denom = math.log(max_distance / exact)
    large = exact + int(math.log(max(distance, exact) / exact) / denom * (buckets - exact))
    return min(large, buckets - 1)


def decode_attention(query, cache_k, cache_v, positions, slots=None, window=0, scale=None, alibi=None,
                     page_table=None, relative_bias=None, relative_max_distance=128, sinks=None,
                     k_scale=None, v_scale=None, rows=None):
    """Reference decode attention, float64, one query row per sequence.

    For row b: live keys are t in [lo, pos] with lo = pos-window+1 when a
    window is set (kernels.py:148-149), capped below the cache context;
    logits = q.k*scale + alibi[h]*t + rel[h, bucket(pos-t)]; softmax over
    the live keys plus, with sinks, one extra logit whose value vector is
    zero (kernels.py:198-206).  GQA head h reads KV head h // (H/KH).
    ``rows`` restricts the computation to some sequences (others are NaN).
    """
    B, H, _, D = query.shape
    KH = cache_k.shape[1]
    G = H // KH
    scale = D ** -.5 if scale is None else scale
    out = torch.full((B, H, 1, D), float('nan'), dtype=torch.float64)
    if page_table is not None:
        context = page_table.shape[1] * cache_k.shape[2]
    else:
        context = cache_k.shape[2]
    for b in (range(B) if rows is None else rows):
        pos = int(positions[b])
        slot = 0 if slots is None else int(slots[b])
        hi = min(pos + 1, context)
        lo = max(0, pos - window + 1) if window else 0
        if page_table is not None:
            k = gather_pages(cache_k, page_table, slot, hi)[:, lo:]
            v = gather_pages(cache_v, page_table, slot, hi)[:, lo:]
            if k_scale is not None:
                k = dequantize_q8(k, gather_pages(k_scale, page_table, slot, hi)[:, lo:])
                v = dequantize_q8(v, gather_pages(v_scale, page_table, slot, hi)[:, lo:])
        else:
            k = cache_k[slot, :, lo:hi]
            v = cache_v[slot, :, lo:hi]
            if k_scale is not None:
                k = dequantize_q8(k, k_scale[slot, :, lo:hi])
                v = dequantize_q8(v, v_scale[slot, :, lo:hi])
        k, v = k.double(), v.double()
        times = torch.arange(lo, hi, dtype=torch.float64)
        for h in range(H):
            q = query[b, h, 0].double()
            logits = (k[h // G] @ q) * scale
            if alibi is not None:
                logits = logits + float(alibi[h]) * times
            if relative_bias is not None:
                buckets = relative_bias.shape[1]
                idx = [t5_bucket(max(pos - t, 0), buckets, relative_max_distance) for t in range(lo, hi)]
                logits = logits + relative_bias[h, idx].double()
            m = logits.max()
            if sinks is not None:
                m = torch.maximum(m, torch.tensor(float(sinks[h]), dtype=torch.float64))
            w = torch.exp(logits - m)
            den = w.sum()
            if sinks is not None:
                den = den + torch.exp(float(sinks[h]) - m)
            out[b, h, 0] = (w @ v[h // G]) / den
    return out


def decode_attention_sdpa(query, cache_k, cache_v, positions, slots, page_table):
    """fp32 page gather + masked GQA SDPA (the reference's torch fallback,
    damendaemon/qwen2.py:788-797, applied after an a8 gather).

    Vectorised for timing: all sequences are gathered into one padded
    (B, KH, L, D) tensor and masked with ``t <= pos``.  Used as the CPU
    baseline of bench.py and as a cross-check of ``decode_attention``.
    """
    B, H, _, D = query.shape
    page = cache_k.shape[2]
    pos = positions.long()
    L = int(pos.max()) + 1
    npages = -(-L // page)
    rows = page_table[slots.long(), :npages].long()                  # (B, npages)
    k = cache_k[rows].permute(0, 2, 1, 3, 4).reshape(B, cache_k.shape[1], npages * page, D)[:, :, :L]
    v = cache_v[rows].permute(0, 2, 1, 3, 4).reshape(B, cache_k.shape[1], npages * page, D)[:, :, :L]
    mask = torch.arange(L)[None, None, None, :] <= pos[:, None, None, None]
    return F.scaled_dot_product_attention(query.float(), k.float(), v.float(), attn_mask=mask,
                                          enable_gqa=True)


def prefill_attention_sdpa(query, cache_k, cache_v, lengths, starts, slots, page_table):
    """fp32 chunked prefill the way the reference's executor runs it on the
    CPU: per segment, gather the slot's start+len tokens from the pages
    (damendaemon/paged.py:101-104, copy_pages) and call SDPA with the
    lower-right causal mask (qwen2.py:754-770, GQA by repeating the KV
    heads).  Used as the CPU baseline of bench.py's mixed-batch line and
    cross-checked against ``prefill_attention`` in tests/test_oracle.py.
    """
    T, H, D = query.shape
    KH, page = cache_k.shape[1], cache_k.shape[2]
    out = torch.empty((T, H, D), dtype=torch.float32)
    t0 = 0
    for n, s, slot in zip(lengths, starts, slots):
        npages = -(-(s + n) // page)
        rows = page_table[slot, :npages].long()     # the slot's pages, gathered at once
        k = cache_k[rows].transpose(0, 1).reshape(KH, npages * page, D)[:, :s + n].float()   # (KH, s+n, D)
        v = cache_v[rows].transpose(0, 1).reshape(KH, npages * page, D)[:, :s + n].float()
        q = query[t0:t0 + n].float().transpose(0, 1)                     # (H, n, D)
        mask = torch.arange(s + n)[None, :] <= (s + torch.arange(n))[:, None]   # row j sees keys <= s + j
        out[t0:t0 + n] = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=KH != H).transpose(0, 1)
        t0 += n
    return out


# ---------------------------------------------------------------------------
# a4: host packer (damendaemon/paged.py:149-159, 118-120; batch.py:133-140)

def pack_batch(lengths, starts, slots, table=None, page=16):
    """Pure-Python restatement of the reference's packing.

    positions = concat(range(start_i, start_i + len_i)) (paged.py:158);
    slot_ids = slot_i repeated len_i times (paged.py:159);
    ends = accumulate(lengths) - 1 (paged.py:118-120);
    cu_seqlens = [0] + accumulate(lengths);
    slot_map[t] = table[slot, pos // page] * page + pos % page, the physical
    row `_rope_batch` writes (kernels.py:279-281, 315, 319);
    gather lists = table[slot_i, :ceil((start_i+len_i)/page)] per segment.
    """
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    positions = [i for n, s in zip(lengths, starts) for i in range(s, s + n)]
    slot_ids = [slot for slot, n in zip(slots, lengths) for _ in range(n)]
    out = {'cu_seqlens': cu, 'ends': [e - 1 for e in cu[1:]], 'positions': positions, 'slot_ids': slot_ids,
           'context_lens': [s + n for s, n in zip(starts, lengths)]}
    if table is not None:
        out['slot_map'] = [int(table[slot, pos // page]) * page + pos % page for pos, slot in zip(positions, slot_ids)]
        cu_pages, gather = [0], []
        for s, n, slot in zip(starts, lengths, slots):
            count = -(-(s + n) // page)
            gather += [int(table[slot, j]) for j in range(count)]
            cu_pages.append(cu_pages[-1] + count)
        out['cu_pages'] = cu_pages
        out['gather_pages'] = gather
    return out


# ---------------------------------------------------------------------------
# a5: rotary embedding + page write (damendaemon/kernels.py:271-340)

def _f16(x):
    return x.to(torch.float16).to(torch.float32)


def rope_rows(x, cos_rows, sin_rows, weight=None, eps=1e-6, precise=False):
    """Rotate rows x (N, D) with per-row cos/sin (N, RD), fp32 arithmetic.

    Follows kernels.py:288-311: optional RMS norm (x * rsqrt(mean(x^2)+eps),
    then * weight), fp16 rounding after each multiply unless ``precise``;
    partner channel (j + RD/2) % RD negated for j < RD/2; channels >= RD
    keep cos 1, sin 0; a = x*cos, b = other*sin, each rounded to fp16
    unless ``precise``; result a + b.  Each product is its own fp32 op.
    """
    x = x.float()
    N, D = x.shape
    RD = cos_rows.shape[-1]
    idx = [(j + RD // 2) % RD for j in range(D)]
    other = x[:, idx]
    if weight is not None:
        inv = torch.rsqrt((x * x).sum(-1, keepdim=True) / D + eps)
        w = weight.float()
        x = x * inv
        other = other * inv
        if not precise:
            x, other = _f16(x), _f16(other)
        x = x * w
        other = other * w[idx]
        if not precise:
            x, other = _f16(x), _f16(other)
    sign = torch.ones(D)
    sign[:RD // 2] = -1
    other = other * sign
    cos = torch.ones(N, D)
    sin = torch.zeros(N, D)
    cos[:, :RD] = cos_rows.float()
    sin[:, :RD] = sin_rows.float()
    a = x * cos
    b = other * sin
    if not precise:
        a, b = _f16(a), _f16(b)
    return a + b


def rope_batch(qkv, cos, sin, positions, slots, cache_k, cache_v, heads, q_norm=None, k_norm=None, eps=1e-6,
               precise=False, page_table=None):
    """Returns (query (T,H,1,D), new cache_k, new cache_v, key (T,KH,D), value (T,KH,D)), CPU."""
    T = qkv.shape[0]
    _, KH, C, D = cache_k.shape
    x = qkv.float().reshape(T, heads + 2 * KH, D)
    pos = positions.long()
    cr, sr = cos[pos], sin[pos]
    q = torch.stack([rope_rows(x[:, h], cr, sr, q_norm, eps, precise) for h in range(heads)], 1)
    k = torch.stack([rope_rows(x[:, heads + h], cr, sr, k_norm, eps, precise) for h in range(KH)], 1)
    v = x[:, heads + KH:]
    ck, cv = cache_k.clone(), cache_v.clone()
    for t in range(T):
        p, s = int(pos[t]), int(slots[t])
        if page_table is not None:
            row, off = int(page_table[s, p // C]), p % C
        else:
            row, off = s, p
        ck[row, :, off] = k[t].to(ck.dtype)
        cv[row, :, off] = v[t].to(cv.dtype)
    return q.to(qkv.dtype).unsqueeze(2), ck, cv, k.to(cache_k.dtype), v.to(cache_k.dtype)


# ---------------------------------------------------------------------------
# a9: chunked prefill attention (damendaemon/paged.py:97-111, qwen2.py:754-770)

def prefill_attention(query, cache_k, cache_v, lengths, starts, slots, page_table, window=0, scale=None,
                      rows=None):
    """float64 attention of packed query rows (T, H, D) over paged history.

    Segment i's row j sits at position starts[i] + j and sees keys
    0 .. starts[i] + j of slot i (lower-right causal), and with a window
    only keys > position - window (qwen2.py:765-770).  ``rows`` limits the
    work to some segments (others stay NaN).
    """
    T, H, D = query.shape
    KH = cache_k.shape[1]
    G = H // KH
    scale = D ** -.5 if scale is None else scale
    out = torch.full((T, H, D), float('nan'), dtype=torch.float64)
    t0 = 0
    for i, (n, s, slot) in enumerate(zip(lengths, starts, slots)):
        if rows is None or i in rows:
            k = gather_pages(cache_k, page_table, slot, s + n).double()
            v = gather_pages(cache_v, page_table, slot, s + n).double()
            for j in range(n):
                p = s + j
                lo = max(0, p - window + 1) if window else 0
                for h in range(H):
                    logits = (k[h // G, lo:p + 1] @ query[t0 + j, h].double()) * scale
                    w = torch.softmax(logits, 0)
                    out[t0 + j, h] = w @ v[h // G, lo:p + 1]
        t0 += n
    return out


# ---------------------------------------------------------------------------
# How each function is pinned (exercised in tests/test_oracle.py).
PINNING = {
    'prefill_attention_sdpa': 'prefill_attention (float64 loop) on seeded ragged segments with GQA and '
                              'histories of several pages (tests/test_oracle.py)',
    'gather_pages': 'brute-force page walk vs torch.cat of pages '
                    '(scripts/verify_paged_copies.py:15-24 construction); permutation invariance',
    'copy_pages': 'gather/restore round trip; untouched tails stay bit-identical',
    'quantize_q8': 'known answers: +-absmax -> +-127, zero group -> scale 0 and data 0, '
                   'exact .5 rounds away from zero; |dequant - x| <= scale/2',
    'dequantize_q8': 'known answers on hand-built int8/scale pairs',
    'decode_attention': 'torch SDPA (library routine) on the gathered dense K/V, as '
                        'scripts/verify_paged_kernels.py:60-67 does; single-key -> v; '
                        'constant V -> V; window >= context == no window; '
                        'sink -inf == no sink; alibi 0 == no alibi',
    't5_bucket': 'transformers T5Attention._relative_position_bucket (library routine, '
                 'unidirectional) over 2000 distances and three (buckets, max_distance) geometries',
    'decode_attention_sdpa': 'agrees with decode_attention on random pages',
    'prefill_attention': 'torch SDPA with causal_lower_right on the gathered K/V (library routine); '
                         'windowed: SDPA with the explicit kpos <= qpos and kpos > qpos - window mask '
                         '(qwen2.py:765-770); window 1 returns each row its own value vector',
    'pack_batch': 'hand-written known answers (tests/test_oracle.py) and invariants: '
                  'positions step by one inside a segment, slot_map decodes to the page-table entry',
    'rope_rows': 'precise path vs the closed form x*cos + cat(-b, a)*sin of '
                 'scripts/verify_paged_kernels.py:40-43 (and verify_kernels.py QK-norm variant); '
                 'rounding points: a row whose products are exact in fp16 gives identical '
                 'precise / non-precise results, a row with an fp16 tie rounds to even',
}

"""GPU packer, page writes, copy_pages and rope_batch against the CPU oracle.

Packer, page writes and copies are integer / byte work: bit-exact.
rope_batch without QK-norm is elementwise fp32 with the reference's rounding
points and no FMA contraction: bit-exact too.  With QK-norm the sum of
squares order differs from any other implementation: tolerance 4e-3 (fp16,
as scripts/verify_kernels.py:109-111) and 2e-6 fp32.
"""
import random

import pytest
import torch

from damendaemon_amd import kernels, packing
from damendaemon_amd.paged_kernels import copy_pages
from oracle import paged_oracle as O

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def random_table(rng, rows, width, capacity):
    table = torch.full((rows, width), -1, dtype=torch.int32)
    perm = list(range(capacity))
    rng.shuffle(perm)
    k = 0
    for r in range(rows):
        n = rng.randint(0, width)
        table[r, :n] = torch.tensor(perm[k:k + n], dtype=torch.int32)
        k += n
    return table


@pytest.mark.parametrize('n', [1, 3, 37, 1024, 3001])
def test_pack_batch_bit_exact(n):
    rng = random.Random(n)
    width = 64
    table = torch.full((n, width), -1, dtype=torch.int32)
    perm = torch.randperm(n * width, generator=torch.Generator().manual_seed(n)).to(torch.int32)
    lengths, starts, slots = [], [], []
    for i in range(n):
        ln = rng.choice([1, 1, 2, 15, 16, 17, 100]) if n > 100 else rng.randint(1, 600)
        st = rng.randint(0, width * 16 - ln)
        lengths.append(ln)
        starts.append(st)
        slots.append(i)
        need = -(-(st + ln) // 16)
        table[i, :need] = perm[i * width:i * width + need]
    order = list(range(n))
    rng.shuffle(order)          # slots in arbitrary order
    lengths = [lengths[i] for i in order]
    starts = [starts[i] for i in order]
    slots = [slots[i] for i in order]
    got = packing.pack_batch(lengths, starts, slots, table.to(DEV))
    want = O.pack_batch(lengths, starts, slots, table)
    for key in ('cu_seqlens', 'ends', 'context_lens', 'positions', 'slot_ids', 'slot_map', 'cu_pages',
                'gather_pages'):
        assert getattr(got, key).cpu().tolist() == want[key], key


def test_pack_mixed_batch_shape():
    """Config C4 metadata: 8 chunks of 512 after contexts in [0,4096] + 120 decodes."""
    rng = random.Random(4)
    starts = [rng.randint(0, 4096) for _ in range(8)] + [rng.randint(256, 8192) - 1 for _ in range(120)]
    lengths = [512] * 8 + [1] * 120
    slots = list(range(128))
    width = (8192 + 512) // 16 + 1
    table = torch.arange(128 * width, dtype=torch.int32).reshape(128, width)
    got = packing.pack_batch(lengths, starts, slots, table.to(DEV))
    want = O.pack_batch(lengths, starts, slots, table)
    assert got.slot_map.cpu().tolist() == want['slot_map']
    assert got.positions.cpu().tolist() == want['positions']
    assert got.gather_pages.cpu().tolist() == want['gather_pages']


def test_pack_without_table_and_empty_segments():
    got = packing.pack_batch([0, 3, 0, 2], [5, 0, 7, 9], [2, 0, 1, 3])
    want = O.pack_batch([0, 3, 0, 2], [5, 0, 7, 9], [2, 0, 1, 3])
    for key in ('cu_seqlens', 'ends', 'context_lens', 'positions', 'slot_ids'):
        assert getattr(got, key).cpu().tolist() == want[key], key


@pytest.mark.parametrize('dtype', [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize('length', [1, 15, 16, 17, 127, 513])
def test_copy_pages_gather_restore_exact(dtype, length):
    """scripts/verify_paged_copies.py:7-28 recipe."""
    g = torch.Generator().manual_seed(927 + length)
    table = torch.full((4, 33), -1, dtype=torch.int32)
    pages = torch.randperm(40, generator=g)[:(length + 15) // 16]
    table[3, :len(pages)] = pages.to(torch.int32)
    original = torch.randn((2, 40, 3, 16, 96), generator=g).to(dtype)
    dense = copy_pages(original.to(DEV), table.to(DEV), 3, length)
    assert torch.equal(dense.cpu(), O.copy_pages(original, table, 3, length))
    restored = torch.full_like(original, 17).to(DEV)
    copy_pages(restored, table.to(DEV), 3, length, snapshot=dense)
    assert torch.equal(restored.cpu(), O.copy_pages(torch.full_like(original, 17), table, 3, length,
                                                    snapshot=dense.cpu()))


def test_copy_pages_validation():
    cache = torch.zeros((2, 4, 1, 16, 32), device=DEV)
    table = torch.zeros((2, 2), dtype=torch.int32, device=DEV)
    for slot, tokens in ((2, 1), (0, 0), (0, 33), (True, 1)):
        with pytest.raises(ValueError):
            copy_pages(cache, table, slot, tokens)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16, torch.float32])
def test_store_kv_pages_exact(dtype):
    g = torch.Generator().manual_seed(5)
    T, KH, D, cap = 50, 8, 128, 40
    key = torch.randn(T, KH, D, generator=g).to(dtype)
    value = torch.randn(T, KH, D, generator=g).to(dtype)
    slot_map = torch.randperm(cap * 16, generator=g)[:T]
    slot_map[3] = -1                                  # skipped
    ck = torch.zeros(cap, KH, 16, D, dtype=dtype)
    cv = torch.zeros_like(ck)
    dk, dv = ck.to(DEV), cv.to(DEV)
    packing.store_kv_pages(key.to(DEV), value.to(DEV), slot_map.to(DEV), dk, dv)
    for t in range(T):
        s = int(slot_map[t])
        if s >= 0:
            ck[s // 16, :, s % 16] = key[t]
            cv[s // 16, :, s % 16] = value[t]
    assert torch.equal(dk.cpu(), ck) and torch.equal(dv.cpu(), cv)


@pytest.mark.parametrize('group', [32, 128])
def test_store_kv_pages_q8_exact(group):
    g = torch.Generator().manual_seed(group)
    T, KH, D, cap = 33, 4, 128, 20
    key = torch.randn(T, KH, D, generator=g).to(torch.bfloat16)
    value = torch.randn(T, KH, D, generator=g).to(torch.bfloat16)
    slot_map = torch.randperm(cap * 16, generator=g)[:T]
    ck = torch.zeros(cap, KH, 16, D, dtype=torch.int8, device=DEV)
    cv = torch.zeros_like(ck)
    ks = torch.zeros(cap, KH, 16, D // group, dtype=torch.float16, device=DEV)
    vs = torch.zeros_like(ks)
    packing.store_kv_pages(key.to(DEV), value.to(DEV), slot_map.to(DEV), ck, cv, ks, vs)
    qk, sk = O.quantize_q8(key, group)
    qv, sv = O.quantize_q8(value, group)
    for t in range(T):
        s = int(slot_map[t])
        assert torch.equal(ck[s // 16, :, s % 16].cpu(), qk[t])
        assert torch.equal(cv[s // 16, :, s % 16].cpu(), qv[t])
        assert torch.equal(ks[s // 16, :, s % 16].cpu(), sk[t])
        assert torch.equal(vs[s // 16, :, s % 16].cpu(), sv[t])


@pytest.mark.parametrize('dtype', [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize('dim', [64, 96, 128])
@pytest.mark.parametrize('precise', [True, False])
def test_rope_batch_paged_exact(dtype, dim, precise):
    """scripts/verify_paged_kernels.py:30-58: paged writes into a NaN pool."""
    g = torch.Generator().manual_seed(dim)
    heads, kh, context, page, cap = 8, 2, 513, 16, 80
    slots = torch.tensor([3, 0, 2])
    pos = torch.tensor([15, 256, 512])
    table = torch.full((4, 33), -1, dtype=torch.int32)
    free = torch.randperm(cap, generator=g).tolist()
    for slot, p in zip(slots.tolist(), pos.tolist()):
        for first in range(0, p + 1, page):
            table[slot, first // page] = free.pop()
    ck = torch.full((cap, kh, page, dim), float('nan'), dtype=dtype)
    cv = torch.full_like(ck, float('nan'))
    packed = torch.randn((3, (heads + 2 * kh) * dim), generator=g).to(dtype)
    ang = torch.randn((context, dim // 2), generator=g)
    ang = torch.cat((ang, ang), -1)
    cos, sin = ang.cos(), ang.sin()
    dk, dv = ck.to(DEV), cv.to(DEV)
    q, k, v = kernels.rope_batch(packed.to(DEV), cos.to(DEV), sin.to(DEV), pos.to(DEV), slots.to(DEV), dk, dv,
                                 heads, precise=precise, page_table=table.to(DEV), materialize=True)
    eq, eck, ecv, ek, ev = O.rope_batch(packed, cos, sin, pos, slots, ck, cv, heads, precise=precise,
                                        page_table=table)
    assert torch.equal(q.cpu(), eq)
    assert torch.equal(k.cpu(), ek) and torch.equal(v.cpu(), ev)
    assert torch.equal(dk.cpu().nan_to_num(7.), eck.nan_to_num(7.))
    assert torch.equal(dv.cpu().nan_to_num(7.), ecv.nan_to_num(7.))


@pytest.mark.parametrize('cos_dtype', [torch.float32, torch.bfloat16])
@pytest.mark.parametrize('precise', [True, False])
def test_rope_batch_c4_batch_exact(cos_dtype, precise):
    """The C4 packed batch (4,216 tokens, H32/KH8/D128 bf16, page 16) through the
    per-token vector kernel, bit-exact against the oracle."""
    from damendaemon_amd.workloads import config_c4
    case = config_c4(device='cpu')
    packed = packing.pack_batch(case['lengths'], case['starts'], case['seg_slots'], case['page_table'].to(DEV))
    T, H, KH, D = packed.total_tokens, 32, 8, 128
    g = torch.Generator().manual_seed(11)
    qkv = torch.randn((T, (H + 2 * KH) * D), generator=g).to(torch.bfloat16)
    ang = torch.randn((8200, D // 2), generator=g) * 3
    ang = torch.cat((ang, ang), -1)
    cos, sin = ang.cos().to(cos_dtype), ang.sin().to(cos_dtype)
    ck, cv = case['cache_k'], case['cache_v']
    dk, dv = ck.to(DEV), cv.to(DEV)
    q = kernels.rope_batch(qkv.to(DEV), cos.to(DEV), sin.to(DEV), packed.positions, packed.slot_ids, dk, dv, H,
                           precise=precise, page_table=case['page_table'].to(DEV))
    eq, eck, ecv, _, _ = O.rope_batch(qkv, cos, sin, packed.positions.cpu(), packed.slot_ids.cpu(), ck, cv, H,
                                      precise=precise, page_table=case['page_table'])
    assert torch.equal(q.cpu(), eq)
    assert torch.equal(dk.cpu(), eck) and torch.equal(dv.cpu(), ecv)


@pytest.mark.parametrize('normalized', [False, True])
def test_rope_batch_d256_bf16_tables(normalized):
    """Head size 256, bf16 rows and bf16 cos/sin tables, slotted cache."""
    g = torch.Generator().manual_seed(256 + normalized)
    batch, heads, kvh, dim, context = 6, 8, 2, 256, 300
    pos = torch.tensor([0, 1, 17, 150, 298, 299])
    slots = torch.tensor([1, 0, 2, 3, 0, 1])
    qkv = torch.randn((batch, (heads + 2 * kvh) * dim), generator=g).to(torch.bfloat16)
    cos = torch.randn((context, dim), generator=g).to(torch.bfloat16)
    sin = torch.randn_like(cos)
    qw = torch.randn(dim, generator=g).to(torch.bfloat16) if normalized else None
    kw = torch.randn(dim, generator=g).to(torch.bfloat16) if normalized else None
    ck = torch.zeros((4, kvh, context, dim), dtype=torch.bfloat16)
    cv = torch.zeros_like(ck)
    dk, dv = ck.to(DEV), cv.to(DEV)
    dev = lambda t: None if t is None else t.to(DEV)
    q, k, v = kernels.rope_batch(qkv.to(DEV), cos.to(DEV), sin.to(DEV), pos.to(DEV), slots.to(DEV), dk, dv, heads,
                                 dev(qw), dev(kw), materialize=True)
    eq, eck, ecv, ek, ev = O.rope_batch(qkv, cos, sin, pos, slots, ck, cv, heads, qw, kw)
    if normalized:
        torch.testing.assert_close(q.cpu().float(), eq.float(), atol=4e-2, rtol=1e-2)
        torch.testing.assert_close(dk.cpu().float(), eck.float(), atol=4e-2, rtol=1e-2)
    else:
        assert torch.equal(q.cpu(), eq) and torch.equal(dk.cpu(), eck) and torch.equal(k.cpu(), ek)
    assert torch.equal(dv.cpu(), ecv) and torch.equal(v.cpu(), ev)


def test_rope_batch_unaligned_rows():
    """Rows that do not start on a 16-byte boundary take the per-(token, head) kernel."""
    g = torch.Generator().manual_seed(77)
    T, heads, kvh, dim, context = 7, 4, 2, 128, 64
    width = (heads + 2 * kvh) * dim
    flat = torch.randn(T * width + 1, generator=g).to(torch.bfloat16)
    pos = torch.tensor([0, 3, 17, 40, 63, 5, 9])
    slots = torch.tensor([0, 1, 0, 1, 0, 1, 1])
    cos = torch.randn((context, dim), generator=g)
    sin = torch.randn_like(cos)
    ck = torch.zeros((2, kvh, context, dim), dtype=torch.bfloat16)
    cv = torch.zeros_like(ck)
    dflat = flat.to(DEV)
    qkv_dev = dflat[1:].view(T, width)            # 2-byte offset
    assert qkv_dev.data_ptr() % 16 != 0
    dk, dv = ck.to(DEV), cv.to(DEV)
    q = kernels.rope_batch(qkv_dev, cos.to(DEV), sin.to(DEV), pos.to(DEV), slots.to(DEV), dk, dv, heads)
    eq, eck, ecv, _, _ = O.rope_batch(flat[1:].view(T, width), cos, sin, pos, slots, ck, cv, heads)
    assert torch.equal(q.cpu(), eq) and torch.equal(dk.cpu(), eck) and torch.equal(dv.cpu(), ecv)


@pytest.mark.parametrize('dim', [64, 96, 128])
@pytest.mark.parametrize('normalized', [False, True])
def test_rope_batch_slotted_qk_norm(dim, normalized):
    """scripts/verify_kernels.py:93-117: slotted fp16 cache, optional QK-norm."""
    g = torch.Generator().manual_seed(dim + normalized)
    batch, heads, kvh, context = 4, 16, 8, 1024
    pos = torch.tensor([0, 255, 256, 1023])
    slots = torch.tensor([3, 1, 2, 0])
    qkv = torch.randn((batch, (heads + 2 * kvh) * dim), generator=g).half()
    cos = torch.randn((context, dim), generator=g).half()
    sin = torch.randn_like(cos)
    qw = torch.randn(dim, generator=g).half() if normalized else None
    kw = torch.randn(dim, generator=g).half() if normalized else None
    ck = torch.zeros((4, kvh, context, dim), dtype=torch.float16)
    cv = torch.zeros_like(ck)
    dk, dv = ck.to(DEV), cv.to(DEV)
    dev = lambda t: None if t is None else t.to(DEV)
    q = kernels.rope_batch(qkv.to(DEV), cos.to(DEV), sin.to(DEV), pos.to(DEV), slots.to(DEV), dk, dv, heads,
                           dev(qw), dev(kw))
    eq, eck, ecv, _, _ = O.rope_batch(qkv, cos, sin, pos, slots, ck, cv, heads, qw, kw)
    if normalized:
        torch.testing.assert_close(q.cpu(), eq, atol=4e-3, rtol=2e-3)
        torch.testing.assert_close(dk.cpu(), eck, atol=4e-3, rtol=2e-3)
    else:
        assert torch.equal(q.cpu(), eq) and torch.equal(dk.cpu(), eck)
    assert torch.equal(dv.cpu(), ecv)


def test_rope_partial_rotary_fp32():
    g = torch.Generator().manual_seed(9)
    T, heads, kvh, dim, rd, context = 5, 4, 2, 96, 32, 64
    qkv = torch.randn((T, (heads + 2 * kvh) * dim), generator=g)
    cos = torch.randn((context, rd), generator=g)
    sin = torch.randn_like(cos)
    pos = torch.tensor([0, 3, 17, 40, 63])
    slots = torch.tensor([0, 1, 0, 1, 0])
    ck = torch.zeros((2, kvh, context, dim))
    cv = torch.zeros_like(ck)
    dk, dv = ck.to(DEV), cv.to(DEV)
    q = kernels.rope_batch(qkv.to(DEV), cos.to(DEV), sin.to(DEV), pos.to(DEV), slots.to(DEV), dk, dv, heads)
    eq, eck, ecv, _, _ = O.rope_batch(qkv, cos, sin, pos, slots, ck, cv, heads)
    assert torch.equal(q.cpu(), eq) and torch.equal(dk.cpu(), eck) and torch.equal(dv.cpu(), ecv)

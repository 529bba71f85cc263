"""Host-side prefill schedule (dd_prefill_plan): runs on the CPU."""
import ctypes
import random

import numpy as np
import pytest

from damendaemon_amd import _native, ragged



def _geometry(dim):
    cols, kt = ctypes.c_int(), ctypes.c_int()
    assert _native.library().dd_prefill_geometry(dim, ctypes.byref(cols), ctypes.byref(kt)) == 0
    return cols.value, kt.value


DIMS = (48, 64, 80, 96, 112, 128, 160, 224, 256)    # head sizes with a 16-bit MFMA kernel
ROWS = {d: _geometry(d)[0] for d in DIMS}   # (query row, head) columns per workgroup
KT = {d: _geometry(d)[1] for d in DIMS}     # keys per tile


def _items(lengths, starts, heads, kv_heads, dim, window):
    rows = ROWS[dim] // (heads // kv_heads)
    max_tiles = -(-max(lengths) // rows) if lengths else 0
    cost = {}
    for seg, (n, s) in enumerate(zip(lengths, starts)):
        for kh in range(kv_heads):
            for qt in range(-(-n // rows)):
                r0 = qt * rows
                k_hi = s + r0 + min(rows, n - r0)
                k_lo = max(0, s + r0 - window + 1) if window > 0 else 0
                cost[(seg * kv_heads + kh) * max_tiles + qt] = (k_hi - 1) // KT[dim] - k_lo // KT[dim] + 1
    return cost, max_tiles


@pytest.mark.parametrize('seed', range(6))
def test_plan_covers_every_tile_once_grouped_per_xcd_longest_first(seed):
    rng = random.Random(seed)
    dim = rng.choice(DIMS)
    kv_heads = rng.choice([1, 2, 8])
    heads = kv_heads * rng.choice([1, 4, 8])
    n = rng.randint(1, 12)
    lengths = [rng.choice([1, 7, 64, 300, 512, 1000]) for _ in range(n)]
    starts = [rng.randint(0, 5000) for _ in range(n)]
    window = rng.choice([0, 0, 700])
    entries = ragged.prefill_plan(lengths, starts, heads, kv_heads, dim, window)
    plan = entries[:, 0]
    cost, max_tiles = _items(lengths, starts, heads, kv_heads, dim, window)
    assert entries.dtype == np.int32 and entries.shape[1] == 8 and len(plan) % 8 == 0
    # each entry carries its segment's packed offset, length, start and slot
    tok0 = np.concatenate([[0], np.cumsum(lengths)])
    for e in entries[plan >= 0]:
        seg = int(e[0]) // max_tiles // kv_heads
        assert list(e[1:6]) == [tok0[seg], lengths[seg], starts[seg], seg, 1] and not e[6:].any()
    real = plan[plan >= 0].tolist()
    assert sorted(real) == sorted(cost)             # every item exactly once
    xcd_of_group = {}
    for x in range(8):
        lst = [int(i) for i in plan[x::8]]
        seen_pad = False
        prev = None
        for item in lst:
            if item < 0:
                seen_pad = True
                continue
            assert not seen_pad                      # padding only at the end
            grp = item // max_tiles
            assert xcd_of_group.setdefault(grp, x) == x
            assert prev is None or cost[item] <= prev
            prev = cost[item]


def test_plan_balances_xcds():
    lengths = [512] * 8
    starts = [3198, 2211, 2253, 3990, 2141, 2468, 3884, 968]
    plan = ragged.prefill_plan(lengths, starts, 32, 8, 128, 0)[:, 0]
    cost, _ = _items(lengths, starts, 32, 8, 128, 0)
    loads = [sum(cost[i] for i in plan[x::8] if i >= 0) for x in range(8)]
    assert max(loads) <= 1.2 * min(loads)


def test_plan_rejects_bad_arguments():
    with pytest.raises(Exception):
        ragged.prefill_plan([4], [0], 6, 4, 128)     # heads not a multiple of kv_heads
    with pytest.raises(Exception):
        ragged.prefill_plan([4], [0], 8, 2, 152)     # no 16-bit MFMA kernel for head dim 152
    with pytest.raises(Exception):
        ragged.prefill_plan([4], [0], 130, 1, 224)   # more heads per KV head than an item's 128 columns
    assert len(ragged.prefill_plan([], [], 8, 2, 128)) == 0
    cols, kt = ctypes.c_int(), ctypes.c_int()
    assert _native.library().dd_prefill_geometry(152, ctypes.byref(cols), ctypes.byref(kt)) != 0
    assert _native.library().dd_prefill_geometry(16, ctypes.byref(cols), ctypes.byref(kt)) != 0
    # the 160 layout takes 144 and 160, the 256 layout the multiples of 16 above
    for dim in (144, 160):
        assert _native.library().dd_prefill_geometry(dim, ctypes.byref(cols), ctypes.byref(kt)) == 0
        assert (cols.value, kt.value) == (256, 64)
    for dim in (176, 240, 256):
        assert _native.library().dd_prefill_geometry(dim, ctypes.byref(cols), ctypes.byref(kt)) == 0
        assert (cols.value, kt.value) == (128, 32)


@pytest.mark.parametrize('seed', range(4))
def test_persistent_plan_rounds(seed):
    """With a workgroup count, each workgroup gets a list of items (round r
    of workgroup b at entry r * G + b): every item once, each list on its
    workgroup's XCD (b % 8, the XCD of the item's group in the one-item
    plan), and within an XCD the loads balanced as longest-first greedy
    assignment guarantees (max - min <= the largest item)."""
    rng = random.Random(seed)
    dim = rng.choice([64, 96, 128])
    kv_heads = rng.choice([2, 8])
    heads = kv_heads * rng.choice([1, 4])
    n = rng.randint(4, 12)
    lengths = [rng.choice([64, 300, 512, 1000]) for _ in range(n)]
    starts = [rng.randint(0, 5000) for _ in range(n)]
    flat = ragged.prefill_plan(lengths, starts, heads, kv_heads, dim, 0)
    xcd_of_group = {}
    cost, max_tiles = _items(lengths, starts, heads, kv_heads, dim, 0)
    for idx, item in enumerate(flat[:, 0]):
        if item >= 0:
            xcd_of_group[int(item) // max_tiles] = idx % 8
    plan = ragged.prefill_plan(lengths, starts, heads, kv_heads, dim, 0, workgroups=64)
    rounds = int(plan[0, 5])
    wgs = len(plan) // rounds     # fewer when every item gets a workgroup of its own
    assert (plan[:, 5] == rounds).all() and wgs * rounds == len(plan) and wgs <= 64 and wgs % 8 == 0
    items = plan[:, 0].reshape(rounds, wgs)
    real = items[items >= 0].tolist()
    assert sorted(real) == sorted(cost)
    load = [0] * wgs
    for b in range(wgs):
        for r in range(rounds):
            item = int(items[r, b])
            if item < 0:
                assert (items[r:, b] < 0).all()     # padding only at the end
                break
            assert xcd_of_group[item // max_tiles] == b % 8
            load[b] += cost[item]
    biggest = max(cost.values())
    for x in range(8):
        ls = load[x::8]
        assert max(ls) - min(ls) <= biggest + 2 * rounds + 2   # the schedule also charges 2 per item

"""PagePool contract: the exact expectations of the reference's tests/test_pages.py:5-50,
plus brute-force checks of the LIFO allocation order (pages.py:16,46)."""
import random

import pytest

from damendaemon_amd.pages import PageCapacityError, PagePool


def test_fragmentation_reuse_and_isolation():
    pool = PagePool(128, 4, 128)
    pool.resize_many([(0, 33), (1, 17), (2, 16)])
    original = list(pool.pages[0])
    pool.release(1)
    pool.resize_many([(3, 48)])
    assert pool.pages[0] == original
    owned = [p for pages in pool.pages for p in pages]
    assert len(owned) == len(set(owned))
    assert set(owned) | set(pool.free) == set(range(8))
    assert pool.used_tokens == 112
    assert pool.pages[3] != sorted(pool.pages[3])


def test_failed_multislot_admission_is_atomic():
    pool = PagePool(64, 2, 128)
    pool.resize_many([(0, 32)])
    before = ([p.copy() for p in pool.pages], pool.free.copy(), pool.revision)
    with pytest.raises(PageCapacityError):
        pool.resize_many([(0, 16), (1, 64)], replace=True)
    assert before == (pool.pages, pool.free, pool.revision)
    pool.resize_many([(0, 16), (1, 48)], replace=True)
    assert pool.used_tokens == 64


def test_decode_growth_and_idempotent_release():
    pool = PagePool(64, 2, 33)
    pool.resize_many([(0, 16)])
    page = pool.pages[0][0]
    pool.resize_many([(0, 17)])
    assert pool.pages[0][0] == page
    pool.resize_many([(0, 33)])
    assert len(pool.pages[0]) == 3
    pool.release(0)
    pool.release(0)
    assert pool.used_tokens == 0
    assert len(pool.free) == 4


@pytest.mark.parametrize('requests', [[(0, 1), (0, 2)], [(2, 1)], [(0, 65)], [(True, 1)], [(0, -1)]])
def test_invalid_requests_do_not_mutate(requests):
    pool = PagePool(64, 2, 64)
    with pytest.raises(ValueError):
        pool.resize_many(requests)
    assert pool.used_tokens == 0


@pytest.mark.parametrize('tokens', [0, 31, 16, True])
def test_invalid_pool_geometry(tokens):
    with pytest.raises(ValueError):
        PagePool(tokens, 2, 64)


def test_fresh_pool_hands_out_ascending_pages_and_lifo_reuse():
    pool = PagePool(160, 3, 160)
    pool.resize_many([(0, 40)])
    assert pool.pages[0] == [0, 1, 2]
    pool.resize_many([(1, 20)])
    assert pool.pages[1] == [3, 4]
    pool.release(0)                       # free tail: ..., 9..5, 0, 1, 2
    pool.resize_many([(2, 48)])
    assert pool.pages[2] == [2, 1, 0]
    assert pool.revision == 4


def _model_resize(pages, free, requests, replace):
    """Independent brute-force restatement used to cross-check random traffic."""
    target = {}
    for slot, tokens in requests:
        count = -(-tokens // 16)
        target[slot] = count if replace else max(count, len(pages[slot]))
    if sum(c - len(pages[s]) for s, c in target.items()) > len(free):
        return False
    for s, c in target.items():
        if c < len(pages[s]):
            free.extend(pages[s][c:])
            pages[s] = pages[s][:c]
    for s, c in target.items():
        while len(pages[s]) < c:
            pages[s].append(free.pop())
    return True


def test_random_traffic_matches_brute_force_model():
    rng = random.Random(5)
    pool = PagePool(16 * 40, 6, 16 * 30)
    pages = [[] for _ in range(6)]
    free = list(range(39, -1, -1))
    for _ in range(2000):
        slots = rng.sample(range(6), rng.randint(1, 3))
        reqs = [(s, rng.randint(0, 16 * 30)) for s in slots]
        replace = rng.random() < 0.5
        ok = _model_resize(pages, free, reqs, replace)
        if ok:
            pool.resize_many(reqs, replace=replace)
        else:
            with pytest.raises(PageCapacityError):
                pool.resize_many(reqs, replace=replace)
        assert pool.pages == pages and pool.free == free
        owned = [p for ps in pool.pages for p in ps]
        assert sorted(owned + pool.free) == list(range(40))


def test_page_table_matches_pages():
    pool = PagePool(128, 3, 64)
    pool.resize_many([(0, 33), (2, 1)])
    table = pool.page_table()
    assert table.shape == (3, 4)
    assert table[0].tolist() == pool.pages[0] + [-1]
    assert table[1].tolist() == [-1] * 4
    assert table[2].tolist() == pool.pages[2] + [-1] * 3

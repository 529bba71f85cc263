"""Host-side drop-ins: prompt grouping (damendaemon/prefill.py) and the
decode scratch budget (damendaemon/attention_budget.py).

Expectations transcribed from the reference's tests
(tests/test_prefill.py:8-20, tests/test_attention_budget.py:5-27), plus a
brute-force model of the grouping contract.
"""
import random

import pytest

from damendaemon_amd.attention_budget import query_rows
from damendaemon_amd.prefill import groups


def test_groups_bound_work_and_keep_order():
    prompts = [[1] * 7, [2] * 3, [3] * 8, [4] * 9, [5]]
    slots = [3, 0, 4, 1, 2]
    batches = list(groups(prompts, slots, 10))
    assert all(sum(map(len, batch)) <= 10 for batch, _ in batches)
    assert [p for batch, _ in batches for p in batch] == prompts
    assert [s for _, assigned in batches for s in assigned] == slots
    assert len(batches) == 3


def test_small_prompts_stay_batched():
    prompts = [[1], [2], [3]]
    assert list(groups(prompts, [2, 0, 1], 20)) == [(prompts, [2, 0, 1])]


def test_groups_brute_force():
    """A group is closed exactly before the prompt that would overflow it;
    an oversized prompt forms its own group."""
    rng = random.Random(0)
    for _ in range(300):
        n = rng.randint(0, 12)
        prompts = [[0] * rng.randint(1, 15) for _ in range(n)]
        slots = list(range(n))
        budget = rng.randint(1, 30)
        got = list(groups(prompts, slots, budget))
        assert [s for _, a in got for s in a] == slots
        for batch, _ in got:
            assert len(batch) == 1 or sum(map(len, batch)) <= budget
        for (batch, _), (nxt, _) in zip(got, got[1:]):
            assert sum(map(len, batch)) + len(nxt[0]) > budget   # the next prompt did not fit


def test_query_rows_fit_and_known_answers():
    budget = 32 * 1024 ** 2
    for splits in (1, 2, 4, 16, 32, 512):
        rows = query_rows(64, 64, splits, budget)
        assert rows * 64 * (splits * 65 + 64) * 4 <= budget < (rows + 1) * 64 * (splits * 65 + 64) * 4
    assert query_rows(64, 64, 16, budget) == 118
    assert query_rows(64, 64, 32, budget) == 61
    for itemsize in (2, 4, 8):
        rows = query_rows(64, 64, 16, budget, itemsize)
        per_row = 64 * (16 * 65 * 4 + 64 * itemsize)
        assert rows * per_row <= budget < (rows + 1) * per_row


@pytest.mark.parametrize('budget', [None, 0, -1, True, 1.5, 64 * 16 * 65 * 4 - 1])
def test_query_rows_rejects_bad_budgets(budget):
    with pytest.raises(ValueError):
        query_rows(64, 64, 16, budget)


def test_last_writer_picks_the_final_duplicate():
    import torch
    from damendaemon_amd.kv_quant import _last_writer
    keys = torch.tensor([[5, 3, 5], [7, 3, 5]])
    assert _last_writer(keys).tolist() == [5, 4, 5, 3, 4, 5]
    g = torch.Generator().manual_seed(1)
    keys = torch.randint(0, 20, (300,), generator=g)
    want = [max(j for j in range(300) if keys[j] == keys[i]) for i in range(300)]
    assert _last_writer(keys).tolist() == want

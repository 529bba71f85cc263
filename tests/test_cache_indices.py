"""cache_indices plans: the brute-force expectations of the reference's
tests/test_cache_indices.py:10-68 (GPU), and validation before allocation (CPU)."""
from unittest.mock import patch

import pytest
import torch

from damendaemon_amd.cache_indices import prefill_indices, ring_decode_indices


@pytest.mark.gpu
def test_prefill_matches_causal_logical_history_at_boundaries():
    for length in (1, 3, 4, 5, 8, 13):
        for window in (1, 4, 16):
            for ratio in (0, 4, 8):
                actual = prefill_indices(length, window=window, ratio=ratio, batch=2).cpu()
                for position in range(length):
                    expected = list(range(max(0, position - window + 1), position + 1))
                    expected += [length + i for i in range((position + 1) // ratio)] if ratio else []
                    for batch in range(2):
                        assert [x for x in actual[batch, position].tolist() if x >= 0] == expected


@pytest.mark.gpu
def test_chunked_query_plans_keep_full_sequence_compression_offset():
    full = prefill_indices(19, window=4, ratio=4).cpu()
    for start, stop in ((0, 3), (3, 8), (8, 19)):
        chunk = prefill_indices(19, window=4, ratio=4, query_start=start, query_stop=stop).cpu()
        for offset, position in enumerate(range(start, stop)):
            assert ([x for x in chunk[0, offset].tolist() if x >= 0]
                    == [x for x in full[0, position].tolist() if x >= 0])


@pytest.mark.gpu
def test_ring_wrap_reordered_slots_and_compressed_visibility():
    positions = [17, 0, 3, 4, 7, 8, 2]
    actual = ring_decode_indices(positions, window=4, ratio=4).cpu()
    assert actual.shape == (7, 1, 4 + 18 // 4)
    for row, position in enumerate(positions):
        expected = [x % 4 for x in range(max(0, position - 3), position + 1)]
        expected += [4 + i for i in range((position + 1) // 4)]
        assert [x for x in actual[row, 0].tolist() if x >= 0] == expected


@pytest.mark.gpu
def test_padding_positions_are_minus_one_in_place():
    plan = prefill_indices(6, window=4, ratio=2).cpu()[0]
    assert plan[0].tolist() == [0, -1, -1, -1, -1, -1, -1]
    assert plan[5].tolist() == [2, 3, 4, 5, 6, 7, 8]


def test_invalid_geometry_and_budget_rejected_before_allocation():
    with patch('damendaemon_amd.cache_indices.torch.empty', side_effect=AssertionError('allocation started')), \
            patch('damendaemon_amd.cache_indices.torch.tensor', side_effect=AssertionError('allocation started')):
        for options in ({'window': 0}, {'window': True}, {'window': 4, 'ratio': -1},
                        {'window': 4, 'query_start': 5, 'query_stop': 4}, {'window': 4, 'batch': 0}):
            with pytest.raises(ValueError):
                prefill_indices(16, **options)
        with pytest.raises(ValueError):
            prefill_indices(32768, window=128, ratio=4)
        for positions in ([], [[1, 2]], [True], [-1]):
            with pytest.raises(ValueError):
                ring_decode_indices(positions, window=4)
        with pytest.raises(ValueError):
            ring_decode_indices([2 ** 30], window=4, ratio=4)

"""Host logic of the deferred commit, on the CPU: the request-keyed row map
that ``continue_pending`` and ``DeferredGroupedCommit.continue_with`` build for
the next batch, and the lengths ``settle`` folds (every pending row that no
next row applies; the verify applies pending row r through next row b only
when rows[b] == r and the next state index of b is r's final page,
csrc/verify_kernel.cuh, the deferred verify's pending test).
"""

import random

import pytest
import torch

from gdn_recoverssm_ascend.kernels import _request_row_map, _unapplied_lengths


def test_row_map_keys_rows_by_request():
    rows, left = _request_row_map(4, [10, 11, 12, 13], [12, 99, 10], torch.device("cpu"))
    assert rows.dtype == torch.int32 and rows.tolist() == [2, -1, 0]
    assert left == [1, 3]


def test_row_map_of_an_empty_batch_and_extra_ids():
    rows, left = _request_row_map(3, ["a", "b", "c", "unused"], [], torch.device("cpu"))
    assert rows.tolist() == [-1] and left == [0, 1, 2]
    # ids past num_rows name no pending row: a request with such an id is new
    rows, left = _request_row_map(3, ["a", "b", "c", "d"], ["d", "a"], torch.device("cpu"))
    assert rows.tolist() == [-1, 0] and left == [1, 2]


@pytest.mark.parametrize("prev,nxt,msg", [
    ([1, 2, 1], [1], "appears twice in the pending step"),
    ([1, 2, 3], [3, 3], "appears twice in the next batch"),
    ([1, 2], [1], "do not cover the pending rows"),
])
def test_row_map_refuses_ambiguous_ids(prev, nxt, msg):
    with pytest.raises(ValueError, match=msg):
        _request_row_map(3, prev, nxt, torch.device("cpu"))


def test_unapplied_lengths_known_case():
    lengths = torch.tensor([3, 2, 1, 4, 7], dtype=torch.int32)  # the last entry is past num_rows
    finals = torch.tensor([10, 11, 12, 13, 14], dtype=torch.int32)
    rows = torch.tensor([2, 0, -1, 3], dtype=torch.int32)
    nxt = torch.tensor([12, 99, 5, 13], dtype=torch.int32)
    # next row 0 continues pending row 2 on its final page: applied;
    # next row 1 continues pending row 0 on another page: not applied;
    # next row 2 is a new request; next row 3 applies pending row 3;
    # pending row 1 left the batch.
    out = _unapplied_lengths(lengths, finals, 4, rows, nxt)
    assert out.tolist() == [3, 2, 0, 0, 7]
    assert lengths.tolist() == [3, 2, 1, 4, 7], "the plan's lengths are not modified"


def test_unapplied_lengths_edges():
    lengths = torch.tensor([1, 2, 3], dtype=torch.int32)
    finals = torch.tensor([5, 6, 7], dtype=torch.int32)
    # an empty next batch applies nothing
    assert _unapplied_lengths(lengths, finals, 3, torch.tensor([-1], dtype=torch.int32),
                              torch.zeros(0, dtype=torch.int32)).tolist() == [1, 2, 3]
    # a row map longer than the batch: only the batch's rows count;
    # row indices outside the pending step name no pending row
    rows = torch.tensor([5, 1, 0], dtype=torch.int32)
    nxt = torch.tensor([7, 6], dtype=torch.int64)
    assert _unapplied_lengths(lengths, finals, 3, rows, nxt).tolist() == [1, 0, 3]


@pytest.mark.parametrize("seed", range(6))
def test_unapplied_lengths_random_batches(seed):
    """Random batch changes built from request ids: a pending row keeps its
    length exactly when no next row continues it on its final page."""
    rng = random.Random(seed)
    n = rng.randint(1, 24)
    prev = rng.sample(range(1000), n)
    lengths = torch.tensor([rng.randint(0, 4) for _ in range(n)], dtype=torch.int32)
    finals = torch.tensor([rng.randint(1, 50) for _ in range(n)], dtype=torch.int32)
    stay = [r for r in prev if rng.random() < 0.7]
    nxt_ids = stay + rng.sample(range(1000, 2000), rng.randint(0, 5))
    rng.shuffle(nxt_ids)
    rows, left = _request_row_map(n, prev, nxt_ids, torch.device("cpu"))
    si = []
    for req in nxt_ids:
        r = prev.index(req) if req in prev else -1
        moved = r >= 0 and rng.random() < 0.25
        si.append(rng.randint(51, 60) if r < 0 or moved else int(finals[r]))
    si = torch.tensor(si, dtype=torch.int32)
    out = _unapplied_lengths(lengths, finals, n, rows, si)
    assert left == sorted(r for r, req in enumerate(prev) if req not in nxt_ids)
    for r in range(n):
        applied = any(int(rows[b]) == r and int(si[b]) == int(finals[r]) for b in range(len(nxt_ids)))
        assert int(out[r]) == (0 if applied else int(lengths[r])), (seed, r)
        if r in left:
            assert int(out[r]) == int(lengths[r]), "a departed request's commit is left to the fold"

"""Host logic of the deferred commit, on the CPU: the request-keyed row map
that ``continue_pending`` and ``DeferredGroupedCommit.continue_with`` build for
the next batch (the lengths a settle folds from it are computed on the device,
tests/test_gpu_deferred.py).
"""

import random

import pytest
import torch

from gdn_recoverssm_ascend.kernels import _request_row_map


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


@pytest.mark.parametrize("seed", range(6))
def test_row_map_random_batches(seed):
    """Random batch changes built from request ids: next row b maps to the
    pending row of its request (-1 for a new one), and the departed rows are
    exactly the pending rows whose request is not in the next batch."""
    rng = random.Random(seed)
    n = rng.randint(1, 24)
    prev = rng.sample(range(1000), n)
    stay = [r for r in prev if rng.random() < 0.7]
    nxt = stay + rng.sample(range(1000, 2000), rng.randint(0, 5))
    rng.shuffle(nxt)
    rows, left = _request_row_map(n, prev + [5000], nxt, torch.device("cpu"))
    want = [prev.index(req) if req in prev else -1 for req in nxt] or [-1]
    assert rows.tolist() == want
    assert left == sorted(r for r, req in enumerate(prev) if req not in nxt)


def test_settle_spec_refuses_bad_arguments_on_the_host():
    """The settle's launch is checked before it is built: 1-3 plan groups,
    pending rows within the plan, an int32 row map covering the next batch,
    1-D int32 / int64 next state indices on the plan's device."""
    from gdn_recoverssm_ascend.kernels import _settle_spec

    i32 = torch.int32
    lengths, finals = torch.zeros(8, dtype=i32), torch.ones(8, dtype=i32)
    out, rl, cnt = torch.zeros(8, dtype=i32), torch.zeros(8, dtype=i32), torch.zeros(1, dtype=i32)
    rows, nxt = torch.arange(4, dtype=i32), torch.ones(4, dtype=i32)

    def spec(**kw):
        a = dict(lengths=lengths, finals=finals, capacity=8, num_rows=4, rows=rows, nexts=[nxt], out=out,
                 row_list=rl, row_count=cnt)
        a.update(kw)
        return _settle_spec(a["lengths"], a["finals"], a["capacity"], a["num_rows"], a["rows"], a["nexts"], a["out"],
                            a["row_list"], a["row_count"])

    assert spec().name == "settle"
    for kw, msg in [
        (dict(nexts=[]), "plan groups"),
        (dict(nexts=[nxt] * 4), "plan groups"),
        (dict(num_rows=9), "pending rows"),
        (dict(rows=rows.long()), "row map"),
        (dict(rows=rows[:3]), "does not cover"),
        (dict(nexts=[nxt.view(2, 2)]), "1-D int32 or int64"),
        (dict(nexts=[nxt.float()]), "1-D int32 or int64"),
    ]:
        with pytest.raises(ValueError, match=msg):
            spec(**kw)

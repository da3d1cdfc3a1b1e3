"""Pins the CPU oracle's commit plan, conv compaction and publication.

Checks: the reference's own known-answer vectors (tests/golden/reference_known_answers.json)
and a brute-force token walk of block ownership, which reaches the final /
boundary columns by simulating positions one token at a time instead of the
closed-form arithmetic the plan uses.
"""

import itertools
import json
import os

import pytest
import torch

import gdn_oracle as O

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))


def _row(C, Bk, n, W, *, grouped=False, Q=8, table=None, source=99, num_blocks=1000):
    table = table if table is not None else [100 + c for c in range(W)]
    return O.oracle_plan_row(
        source=source, accepted=n, bos=0, eos=Q, spec_query_len=Q, num_blocks=num_blocks,
        align=True, table_row=table, num_computed=C, block_size=Bk, grouped=grouped,
    )


@pytest.mark.parametrize("grouped", [False, True])
def test_plan_boundary_cases_from_reference(grouped):
    for C, Bk, n, W, fcol, bcol, blen in GOLD["plan_boundary_cases"]["cases"]:
        pr = _row(C, Bk, n, W, grouped=grouped)
        assert pr.col == fcol, (C, Bk, n, W)
        if n > 0:
            assert pr.final == 100 + fcol
            assert pr.boundary == (O.NULL_BLOCK_ID if bcol is None else 100 + bcol)
            assert pr.boundary_len == blen
        else:
            assert pr.valid == 0 and pr.commit_len == 0 and pr.final == O.NULL_BLOCK_ID


def test_plan_destination_is_allocated_and_running_column():
    g = GOLD["plan_allocated_columns"]
    for C, A in g["cases"]:
        pr = _row(C, g["block_size"], A, g["table_width"])
        needed = -(-(C + A) // g["block_size"])
        assert pr.col <= max(needed - 1, 0)
    r = GOLD["plan_running_column"]
    for C, A, want in r["cases"]:
        assert _row(C, r["block_size"], A, 8).col == want


def _token_walk(C, Bk, n, W):
    """Block ownership by walking tokens: token p (0-based) lives in column p // Bk.

    The committed state after n tokens belongs to the column of the last
    committed token (or column 0 when nothing precedes it); the first block
    boundary reached strictly after C within the window owns a snapshot of the
    state at that boundary.
    """
    last = C + n - 1
    final_col = min(max(last, 0) // Bk, W - 1)
    boundary_col, blen = None, 0
    for step in range(1, n + 1):
        pos = C + step  # tokens consumed so far
        if pos % Bk == 0:
            boundary_col, blen = pos // Bk - 1, step
            break
    if boundary_col is not None and boundary_col >= W:
        boundary_col, blen = None, 0
    return final_col, boundary_col, blen


@pytest.mark.parametrize("grouped", [False, True])
def test_plan_matches_token_walk_bruteforce(grouped):
    for Bk, W, Q in ((4, 3, 4), (8, 5, 8), (64, 2, 4), (5, 4, 3)):
        for C, n in itertools.product(range(0, 3 * Bk + 2), range(0, Q + 1)):
            pr = _row(C, Bk, n, W, grouped=grouped, Q=Q)
            fcol, bcol, blen = _token_walk(C, Bk, n, W)
            assert pr.col == fcol, (Bk, W, C, n)
            if n == 0:
                assert (pr.valid, pr.final, pr.boundary, pr.boundary_len) == (0, 0, 0, 0)
                continue
            assert pr.valid == 1
            assert pr.commit_len == n
            assert pr.final == 100 + fcol
            assert pr.boundary == (0 if bcol is None else 100 + bcol), (Bk, W, C, n)
            assert pr.boundary_len == blen, (Bk, W, C, n)
            assert pr.source == (99 if grouped else 99)


def test_plan_validity_edges():
    base = dict(accepted=2, spec_query_len=4, num_blocks=10, align=False, grouped=True)
    ok = O.oracle_plan_row(source=3, bos=0, eos=4, **base)
    assert (ok.valid, ok.commit_len, ok.final, ok.source) == (1, 2, 3, 3)
    for src in (0, -1, 10, 11):  # null, padding, out of pool
        assert O.oracle_plan_row(source=src, bos=0, eos=4, **base).valid == 0
    assert O.oracle_plan_row(source=3, bos=-1, eos=3, **base).valid == 0  # negative start
    assert O.oracle_plan_row(source=3, bos=5, eos=4, **base).valid == 0  # reversed
    assert O.oracle_plan_row(source=3, bos=0, eos=5, **base).valid == 0  # longer than the window
    short = O.oracle_plan_row(source=3, bos=0, eos=1, **base)
    assert short.commit_len == 1  # clamped to the query length
    neg = O.oracle_plan_row(source=3, bos=0, eos=4, **{**base, "accepted": -3})
    assert neg.valid == 0 and neg.commit_len == 0
    # negative num_computed invalidates an align row
    al = O.oracle_plan_row(source=3, bos=0, eos=4, accepted=2, spec_query_len=4, num_blocks=10,
                           align=True, table_row=[3, 4], num_computed=-1, block_size=4, grouped=True)
    assert al.valid == 0 and al.boundary == 0 and al.boundary_len == 0


def _gp_groups(gp, n_groups, *, sources_override=None, blocks=None, align=True):
    groups = []
    for gi in range(n_groups):
        src = list(gp["sources"])
        if sources_override and gi in sources_override:
            src = list(sources_override[gi])
        groups.append(dict(
            state_indices=torch.tensor(src),
            query_start_loc=torch.tensor(gp["query_start_loc"]),
            request_indices=torch.tensor(gp["request_indices"]),
            block_table=torch.tensor(gp["block_table"]) + gi * gp["group_page_offset"] if align else None,
            num_computed=torch.tensor(gp["num_computed"]) if align else None,
            block_size=gp["block_size"] if align else None,
            num_blocks=(blocks[gi] if blocks else gp["num_blocks"]),
        ))
    return groups


def _persist(gp):
    n = gp["persistent_size"]
    return (torch.full((n,), gp["persistent_cols_init"], dtype=torch.int32),
            torch.full((n,), gp["persistent_accepted_init"], dtype=torch.int32))


def test_grouped_plan_reference_vectors():
    gp = GOLD["grouped_plan"]
    cols, acc = _persist(gp)
    res = O.oracle_plan_grouped(
        torch.tensor(gp["sampled"]), _gp_groups(gp, 3), spec_query_len=gp["spec_query_len"],
        capacity=gp["capacity"], rows=gp["rows"], align=True, idx_mapping=torch.tensor(gp["idx_mapping"]),
        persistent_cols=cols, persistent_accepted=acc,
    )
    cap = gp["capacity"]
    for gi in range(3):
        s = gi * cap
        assert res["final"][s:s + 2].tolist() == [x + 20 * gi for x in gp["expected_final_group0"]]
        assert int(res["boundary"][s]) == gp["expected_boundary_row0_group0"] + 20 * gi
        assert int(res["boundary_len"][s]) == gp["expected_boundary_len_row0"]
        assert res["length"][s:s + 2].tolist() == gp["expected_length"]
    assert res["persistent_cols"].tolist() == gp["expected_cols"]
    assert res["persistent_accepted"].tolist() == gp["expected_accepted"]


def test_grouped_plan_invalid_group_blocks_publication():
    gp = GOLD["grouped_plan"]
    inv = GOLD["grouped_invalid_group"]
    cols, acc = _persist(gp)
    res = O.oracle_plan_grouped(
        torch.tensor(gp["sampled"]), _gp_groups(gp, 2, sources_override={1: inv["group1_sources"]}),
        spec_query_len=4, capacity=gp["capacity"], rows=2, align=True,
        idx_mapping=torch.tensor(gp["idx_mapping"]), persistent_cols=cols, persistent_accepted=acc,
    )
    assert int(res["length"][gp["capacity"]]) == inv["expected_group1_row0_length"]
    assert int(res["persistent_cols"][1]) == inv["expected_cols_1"]
    assert int(res["persistent_accepted"][1]) == inv["expected_accepted_1"]
    assert int(res["persistent_cols"][5]) == inv["expected_cols_5"]
    assert int(res["persistent_accepted"][5]) == inv["expected_accepted_5"]


def test_grouped_plan_none_mode_and_zero_acceptance():
    gp = GOLD["grouped_plan"]
    cols, acc = _persist(gp)
    res = O.oracle_plan_grouped(
        torch.tensor(gp["sampled"]), _gp_groups(gp, 1, align=False), spec_query_len=4,
        capacity=gp["capacity"], rows=2, align=False, idx_mapping=torch.tensor(gp["idx_mapping"]),
        persistent_cols=cols, persistent_accepted=acc,
    )
    assert res["final"][:2].tolist() == gp["none_mode_expected_final"]
    assert res["length"][:2].tolist() == gp["none_mode_expected_length"]
    assert res["persistent_accepted"].tolist() == [7] * 6
    res = O.oracle_plan_grouped(
        torch.zeros(3, dtype=torch.int32), _gp_groups(gp, 1), spec_query_len=4, capacity=gp["capacity"],
        rows=2, align=True, idx_mapping=torch.full((3,), -1), persistent_cols=cols, persistent_accepted=acc,
    )
    assert res["length"][:2].tolist() == [0, 0]
    assert res["persistent_cols"].tolist() == [-9] * 6
    assert res["persistent_accepted"].tolist() == [7] * 6


def test_grouped_plan_small_pool_boundary_is_canonicalised():
    gp = GOLD["grouped_plan"]
    sp = GOLD["grouped_small_pool"]
    groups = _gp_groups(gp, 2, blocks=[sp["small_blocks"], sp["large_blocks"]])
    r, c, val = sp["patched_table_entry"]
    groups[0]["block_table"][r, c] = val
    res = O.oracle_plan_grouped(torch.tensor(gp["sampled"]), groups, spec_query_len=4, capacity=gp["capacity"],
                                rows=2, align=True, idx_mapping=torch.tensor(gp["idx_mapping"]),
                                persistent_cols=_persist(gp)[0], persistent_accepted=_persist(gp)[1])
    assert int(res["final"][0]) == sp["expected_final_group0_row0"]
    assert int(res["boundary"][0]) == sp["expected_boundary_group0_row0"]
    assert int(res["boundary_len"][0]) == sp["expected_boundary_len_group0_row0"]
    assert int(res["boundary"][gp["capacity"]]) == sp["expected_boundary_group1_row0"]


def test_single_plan_keeps_raw_invalid_boundary_but_zero_length():
    # The single-context kernel does not canonicalise the boundary index
    # (kernels.py:1053-1065): an out-of-pool page keeps its id with length 0.
    pr = _row(7, 4, 3, 4, table=[1, 50, 3, 4], num_blocks=10, source=2)
    assert pr.final == 3 and pr.boundary == 50 and pr.boundary_len == 0
    prg = _row(7, 4, 3, 4, table=[1, 50, 3, 4], num_blocks=10, grouped=True, source=2)
    assert prg.boundary == 0 and prg.boundary_len == 0


def test_publish_across_buckets_requires_all_valid_and_agreeing_columns():
    valid_a = torch.tensor([1, 1, 0, 0], dtype=torch.int32)
    col_a = torch.tensor([2, 0, 0, 0], dtype=torch.int32)
    valid_b = torch.tensor([1, 0, 0, 0], dtype=torch.int32)
    col_b = torch.tensor([2, 0, 0, 0], dtype=torch.int32)
    cols = torch.full((4,), -9, dtype=torch.int32)
    acc = torch.full((4,), 7, dtype=torch.int32)
    c, a = O.oracle_publish([(valid_a, col_a, 4, 1), (valid_b, col_b, 4, 1)], torch.tensor([2, 0]),
                            torch.tensor([3, -1, 1]), cols, acc, rows=2)
    assert c.tolist() == [-9, 2, -9, -9] and a.tolist() == [7, 1, 7, 7]


def test_publish_maps_committed_rows_to_slots():
    """Only committed rows are published, each at its idx_mapping slot; a row
    whose request maps to -1 and every other slot keep their values. Row 1 is
    a valid plan row here, so the -1 mapping alone must skip it."""
    sm = GOLD["publication_slot_mapping"]
    rows = len(sm["idx_mapping"])
    valid = torch.ones(rows, dtype=torch.int32)
    col = torch.full((rows,), 5, dtype=torch.int32)
    for r, c in zip(sm["committed_rows"], sm["committed_cols"]):
        col[r] = c
    init = torch.full((sm["slots"],), sm["initial"], dtype=torch.int32)
    c, a = O.oracle_publish([(valid, col, rows, 1)], torch.arange(rows), torch.tensor(sm["idx_mapping"]),
                            init, init.clone(), rows=rows)
    assert c.tolist() == sm["expected_cols"] and a.tolist() == sm["expected_accepted"]


def test_conv_compaction_index_identity():
    hist, Q = 3, 4
    window = hist + Q - 1
    conv = torch.arange(4 * 2 * window, dtype=torch.float32).reshape(4, 2, window)
    out = O.oracle_conv_compact(
        [conv], source=torch.tensor([1]), lengths=torch.tensor([2]), final=torch.tensor([2]),
        boundary=torch.tensor([3]), boundary_len=torch.tensor([1]), history=hist,
        num_blocks=4, rows=1, align=True,
    )[0]
    assert torch.equal(out[2, :, :hist], conv[1, :, 1:4])
    assert torch.equal(out[2, :, hist:], conv[2, :, hist:])  # tail untouched
    assert torch.equal(out[3, :, :hist], conv[1, :, 0:3])
    # final aliasing the source reads the original source
    out = O.oracle_conv_compact(
        [conv], source=torch.tensor([1]), lengths=torch.tensor([4]), final=torch.tensor([1]),
        boundary=torch.tensor([0]), boundary_len=torch.tensor([0]), history=hist,
        num_blocks=4, rows=1, align=True,
    )[0]
    assert torch.equal(out[1, :, :hist], conv[1, :, 3:6])
    # n == 0 is a no-op
    out = O.oracle_conv_compact(
        [conv], source=torch.tensor([1]), lengths=torch.tensor([0]), final=torch.tensor([1]),
        boundary=torch.tensor([0]), boundary_len=torch.tensor([0]), history=hist,
        num_blocks=4, rows=1, align=False,
    )[0]
    assert torch.equal(out, conv)

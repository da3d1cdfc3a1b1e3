"""Which thread of which workgroup loads and stores each 16-byte chunk of a
(page, head) state tile, restated on the CPU from the index arithmetic of the
kernels that write state pages in place:

* the fold (csrc/fold.hip, ``fold_body``): one 256-thread workgroup per
  (layer, row, value head); thread ``tid`` owns chunk ``tid % KCH`` of rows
  ``tid // KCH + pass * RP``; passes go in batches of ``64 / E`` loads, each
  batch's stores after its loads;
* the deferred verify (csrc/verify_kernel.cuh, ``DEFER``): one wave per
  (row, value head, 64-row half tile); block ``rb``'s stores (final page and
  boundary snapshot) come after its loads, and the loads of block ``rb + 2``
  after those stores.

A row's source, final and boundary pages may be one page (the plan makes
``boundary == source`` whenever the window crosses a block boundary from the
block the row started in; the alias case of the reference's
tests/test_math_oracle.py:206-235). Folding in place is then correct only if
every chunk of the tile is loaded and stored by exactly one thread, and that
thread stores it only after loading it: a chunk loaded by one thread after
another thread stored it would be folded twice. The checks below establish
both properties for every tile shape the kernels accept, and show that a
decomposition splitting a tile's passes between two workgroups whose batches
still span the whole tile breaks them (the failure such a split would have
in the alias case).
"""

import itertools

import pytest

FOLD_THREADS = 256


def _fold_events(K, V, E, vs, split=None):
    """(workgroup, thread, batch, kind, chunk) for every in-tile access of one
    fold tile, in each thread's program order. ``split`` models two
    workgroups per tile, workgroup h taking passes from h * passes / 2 and
    loading whole batches of ITERS passes from there (the mutant)."""
    kch, kch_log = 1, 0
    while kch * E < K:
        kch, kch_log = kch * 2, kch_log + 1
    RP = FOLD_THREADS // kch
    ITERS = 64 // E
    passes = -(-V // RP)
    events = []
    groups = [(0, 0, passes)] if split is None else [(h, h * passes // 2, (h + 1) * passes // 2) for h in range(2)]
    for wg, lo, hi in groups:
        for tid in range(FOLD_THREADS):
            kc, r0 = tid & (kch - 1), tid >> kch_log
            if kc * E >= K:
                continue
            last = hi if split is None else lo + ITERS * (-(-(hi - lo) // ITERS))
            for batch, first in enumerate(range(lo, last, ITERS)):
                rows = [r0 + (first + i) * RP for i in range(ITERS)]
                # The tile's buffer resource spans V rows of vs elements.
                chunks = [(r, kc) for r in rows if r * vs + kc * E < V * vs]
                for ch in chunks:
                    events.append((wg, tid, batch, "load", ch))
                for ch in chunks:
                    events.append((wg, tid, batch, "store", ch))
    return events


def _check_single_owner(events, K, V, E):
    """Every chunk of the tile loaded once and stored once, by the same
    (workgroup, thread), its store after its load in that thread's order."""
    want = {(r, c) for r in range(V) for c in range(-(-K // E))}
    owner_load, owner_store = {}, {}
    order = {}
    for i, (wg, tid, batch, kind, ch) in enumerate(events):
        table = owner_load if kind == "load" else owner_store
        if ch in table:
            return f"chunk {ch} {kind}ed twice"
        table[ch] = (wg, tid)
        order[(kind, ch)] = i
    if set(owner_load) != want or set(owner_store) != want:
        return "the accesses do not cover the tile"
    for ch in want:
        if owner_load[ch] != owner_store[ch]:
            return f"chunk {ch} stored by another thread than the one that loaded it"
        if order[("store", ch)] < order[("load", ch)]:
            return f"chunk {ch} stored before its load"
    return None


SHAPES = [
    # (K, V, E, row stride): FP32 (E=4) and 16-bit (E=8) state, the benchmark's
    # 128 x 128, head dims off the tile, several batches of passes, padded rows.
    (128, 128, 4, 128), (128, 128, 8, 128), (256, 1024, 4, 256), (96, 128, 4, 96), (192, 64, 8, 192),
    (16, 32, 4, 16), (256, 256, 8, 256), (128, 200, 4, 132), (64, 1024, 8, 64), (32, 8, 4, 32),
]


@pytest.mark.parametrize("K,V,E,vs", SHAPES)
def test_fold_tile_has_one_owner_per_chunk(K, V, E, vs):
    assert _check_single_owner(_fold_events(K, V, E, vs), K, V, E) is None


@pytest.mark.parametrize("K,V,E,vs", [(128, 128, 4, 128), (128, 128, 8, 128)])
def test_split_with_whole_batches_breaks_the_single_owner_rule(K, V, E, vs):
    """Two workgroups per tile whose batches run past their half of the
    passes load and store the same chunks: with source == boundary, the
    second can read a chunk after the first stored its snapshot there."""
    problem = _check_single_owner(_fold_events(K, V, E, vs, split=True), K, V, E)
    assert problem is not None and "twice" in problem


def _alias_fold(h0, decay, c, k, n, blen, two_pass):
    """The scalar alias case: source == boundary page. A correct fold reads
    the source once; a second reader after the snapshot store folds the
    snapshot again."""
    h = h0
    pages = {"src": h0}
    snap = None
    for t in range(n):
        h = c * k + h * decay
        if t + 1 == blen:
            snap = h
            pages["src"] = snap  # boundary page is the source page
    final = h
    if two_pass:
        h2 = pages["src"]  # a second workgroup loading after the snapshot store
        for t in range(n):
            h2 = c * k + h2 * decay
        final = h2
    return final, snap


def test_alias_case_known_answer_and_the_double_fold():
    """tests/test_math_oracle.py:206-235 of the reference: h0 = 10, decay 0.5,
    c = k = 1, n = 3, boundary after 2 tokens: final 3, boundary 4; reading
    the source again after the snapshot store gives 2.25."""
    final, snap = _alias_fold(10.0, 0.5, 1.0, 1.0, 3, 2, two_pass=False)
    assert (final, snap) == (3.0, 4.0)
    bad, _ = _alias_fold(10.0, 0.5, 1.0, 1.0, 3, 2, two_pass=True)
    assert bad == 2.25


def _defer_events(K, V, E, vs, J, rounds):
    """The deferred verify's non-temporal body for one tile: wave vt covers
    rows [64 vt, 64 vt + 64); block rb's 16 rows are loaded as row runs
    (load j: rows (j % JR) * RPL + lane // SC, chunks (j // JR) * SC + lane % SC)
    and stored back with the same offsets after its fold; blocks rb and
    rb + 1 are in flight together, rb + 2 is loaded after rb's stores."""
    cpr = 4 * J
    SC, JR = cpr // rounds, J // rounds
    RPL = 64 // SC
    events = []
    nvt = -(-V // 64)
    for vt in range(nvt):
        row0 = vt * 64
        tile_rows = min(64, V - row0)

        def block(rb):
            out = []
            for j in range(J):
                for lane in range(64):
                    r = rb * 16 + (j % JR) * RPL + lane // SC
                    c = (j // JR) * SC + lane % SC
                    if c * E < K and r < tile_rows:
                        out.append((lane, (row0 + r, c)))
            return out

        order = [("load", 0), ("load", 1)]
        for rb in range(4):
            order.append(("store", rb))
            if rb + 2 < 4:
                order.append(("load", rb + 2))
        for kind, rb in order:
            for lane, ch in block(rb):
                events.append((vt, lane, 0, kind, ch))
    return events


@pytest.mark.parametrize("K,V,E,J", [(128, 128, 4, 8), (128, 128, 8, 4), (256, 256, 4, 16), (64, 96, 4, 4),
                                     (16, 8, 4, 1), (32, 128, 4, 2)])
@pytest.mark.parametrize("rounds", [1, 2, 4])
def test_deferred_verify_tile_has_one_owner_per_chunk(K, V, E, J, rounds):
    """For any number of staging rounds that divides the block's loads."""
    if J % rounds or 64 % (4 * J // rounds):
        pytest.skip("not a staging of this J")
    assert 4 * E * J >= K
    assert _check_single_owner(_defer_events(K, V, E, K, J, rounds), K, V, E) is None


def test_plan_outputs_never_feed_the_fused_launch():
    """In the fused plan + fold launch the writer workgroups store the plan
    arrays while the folding workgroups plan from the step's metadata; the
    two sets must not share memory (the host refuses overlapping ranges).
    The folding workgroups' reads, per csrc/plan_row.cuh and csrc/fold.hip."""
    fold_reads = {"state_indices", "query_start_loc", "request_indices", "sampled", "num_computed", "block_table",
                  "layer_tables", "layer_groups", "records", "decay"}
    writer_writes = {"source_plan", "lens_plan", "final_plan", "boundary_plan", "boundary_lens_plan", "valid_plan",
                     "col_plan", "persistent_cols", "persistent_accepted"}
    assert not fold_reads & writer_writes
    for a, b in itertools.combinations(sorted(writer_writes), 2):
        assert a != b

"""The deferred commit through the grouped coordinator
(``GroupedCommitCoordinator.commit_deferred``, the commit the reference's
commit proxy drives, layer_patch.py:108-149 -> grouped_commit.py:896-1016,
with the fold left to the next verify as docs/GDN-RecoverSSM-实现方案.md:515-527
proposes), checked against the CPU oracle.

Four align-mode cache groups in two buckets (three groups, then one) commit one
step with the folds deferred. Checked bit for bit against the oracle: every
group's plan, the conv compaction and the persistent publication across the two
buckets (``oracle_publish`` through ``oracle_plan_grouped``); no page changes
before a fold. The next batch is keyed by request: one request whose commit
crosses a block boundary leaves, another continued request is given a page
other than its pending final page, a new request takes a row, and the rows come
in another order. ``settle`` folds the commits the next verifies will not
apply (those two), then every layer's deferred verify, run with no token,
applies the rest through the re-keyed row map. The pages then equal the
oracle's fold of the whole step (FP32 within max-abs 1e-5 relative to the
pages' max-abs), and pages outside it are bit-identical.
"""

import pytest
import torch

import gdn_oracle as O
from gdn_recoverssm_ascend.grouped_commit import GroupedCommitCoordinator
from gdn_recoverssm_ascend.kernels import GDNRecoverSSMCommitContext, ReplayRecordBuffers, gdn_recoverssm_verify_deferred
from test_gpu_commit import HIST, _check_states, _entry, _group, _index_by_request, _oracle_grouped, _planes, _to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(gpu_device):
    return gpu_device


def _groups(B, n_groups, seed):
    """Align-mode groups on one set of logical rows and positions (each with
    its own pages and records), one or two layers each."""
    groups = [_group(B, 2, 4, 64, 64, 4, 1 + g % 2, align=True, seed=seed + g) for g in range(n_groups)]
    for G in groups[1:]:
        G["qsl"] = groups[0]["qsl"].clone()
        G["C"] = groups[0]["C"].clone()
    for G in groups:
        C = G["C"].long()
        src_col = torch.clamp(C - 1, min=0) // G["Bk"]
        table = torch.zeros_like(G["table"])
        for r in range(B):
            for j in range(3):
                table[r, int(src_col[r]) + j] = 1 + 3 * r + j
        G["table"], G["src"] = table, table[torch.arange(B), src_col].clone()
    return groups


@pytest.mark.parametrize("seed", [700, 710])
def test_coordinator_deferred_commit_against_oracle(dev, seed):
    B, n_groups = 6, 4
    gen = torch.Generator().manual_seed(seed)
    request_rows = torch.randperm(B, generator=gen).tolist()
    groups = _groups(B, n_groups, seed)
    # Accepted counts are read by request; row b's is the count group 0's
    # positions were drawn for, so that half the rows cross a block boundary.
    sampled = torch.zeros(B, dtype=torch.int32)
    for b, r in enumerate(request_rows):
        sampled[r] = max(1, int(groups[0]["acc"][b]))
    metas, devs, spare = [], [], []
    for G in groups:
        _index_by_request(G, request_rows)
        ckpts, convs, recs = _to_dev(G, dev)
        ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=4, max_num_reqs=B)
        devs.append((ckpts, convs))
        metas.append(_entry(G, ctx, dev, request_rows).metadata)
        # the next verify writes another record set than the pending one
        spare.append([ReplayRecordBuffers.allocate(B, 4, 2, 4, 64, 64, device=dev) for _ in G["ckpts"]])
    mapping = torch.randperm(B + 2, generator=gen)[:B].to(torch.int32)
    cols = torch.full((B + 2,), -9, dtype=torch.int32)
    accp = torch.full((B + 2,), 7, dtype=torch.int32)
    cols_d, accp_d = cols.to(dev), accp.to(dev)
    before = [[c.clone() for c in ck] for ck, _ in devs]
    print(f"deferred coordinator: seed={seed} requests={request_rows} sampled={sampled.tolist()}", flush=True)

    coord = GroupedCommitCoordinator()
    d = coord.commit_deferred(metas, sampled.to(dev), mapping.to(dev), cols_d, accp_d)
    torch.cuda.synchronize()
    assert len(coord._buckets) == 2 and coord.last_launch_count == 2 * 2 + 1  # plan + conv per bucket, publish
    want = _oracle_grouped(groups, sampled, mapping, cols, accp, request_rows, True, B)
    assert cols_d.cpu().tolist() == want["persistent_cols"].tolist(), "publication differs"
    assert accp_d.cpu().tolist() == want["persistent_accepted"].tolist(), "publication differs"
    assert int((accp_d.cpu() == 1).sum()) > 0, "nothing was published"
    for gi, G in enumerate(groups):
        seg = slice(gi * B, gi * B + B)
        plan = d._plan(gi)
        for name, got in zip(("source", "length", "final", "boundary", "boundary_len"), plan):
            assert got[:B].cpu().tolist() == want[name][seg].tolist(), f"group {gi}: plan {name} differs"
        for li, (got, b) in enumerate(zip(devs[gi][0], before[gi])):
            assert torch.equal(got, b), f"group {gi} layer {li}: a page changed before any fold"
        wconv = O.oracle_conv_compact(G["convs"], source=want["source"][seg], lengths=want["length"][seg],
                                      final=want["final"][seg], boundary=want["boundary"][seg],
                                      boundary_len=want["boundary_len"][seg], history=HIST, num_blocks=G["NB"],
                                      rows=B, align=True)
        for li, (got, w) in enumerate(zip(devs[gi][1], wconv)):
            assert torch.equal(got.cpu(), w), f"group {gi} layer {li}: conv states differ"

    # The next batch, keyed by request id (here: the request row).
    lens, bnd, blen = want["length"][:B], want["boundary"][:B], want["boundary_len"][:B]
    crossing = [b for b in range(B) if int(lens[b]) > 0 and 0 < int(bnd[b]) and int(blen[b]) > 0]
    assert crossing, "no committed row crosses a block boundary"
    leaving = crossing[0]
    stay = [b for b in range(B) if b != leaving]
    moved = [b for b in stay if int(lens[b]) > 0]
    assert moved, "no continued row committed"
    moved = moved[0]  # continued, but the next batch names another page for it
    prev_ids = [request_rows[b] for b in range(B)]
    next_rows = list(reversed(stay)) + [None]  # pending rows in another order, then a new request
    next_ids = [prev_ids[r] if r is not None else 99 for r in next_rows]
    left = d.continue_with(prev_ids, next_ids)
    assert left == [leaving]
    next_metas = []
    for gi, G in enumerate(groups):
        seg = slice(gi * B, gi * B + B)
        fin = want["final"][seg]
        si = torch.tensor([int(fin[r]) if r is not None and int(lens[r]) > 0 else
                           (int(G["src"][r]) if r is not None else G["NB"] - 1) for r in next_rows], dtype=torch.int32)
        si[next_rows.index(moved)] = G["NB"] - 2  # a page no row uses
        nm = _entry(dict(G, src=si, B=len(next_rows)), metas[gi].recoverssm_context, dev, list(range(len(next_rows))))
        next_metas.append(nm.metadata)
    d.settle(next_metas)
    # Every layer's deferred verify, with no token, applies the commits it continues.
    T0 = torch.zeros(len(next_rows) + 1, dtype=torch.int32, device=dev)
    for gi, G in enumerate(groups):
        pend = d.pending(gi)
        si = next_metas[gi].recoverssm_commit.state_indices
        for li in range(len(G["ckpts"])):
            e = torch.empty(1, 0, 2, 64, device=dev, dtype=torch.bfloat16)
            ev = torch.empty(1, 0, 4, 64, device=dev, dtype=torch.bfloat16)
            gb = torch.empty(0, 4, device=dev)
            gdn_recoverssm_verify_deferred(gb, gb, e, e, ev, checkpoint_state=devs[gi][0][li],
                                           replay_cache=spare[gi][li], pending=pend[li], query_start_loc=T0,
                                           state_indices=si, spec_query_len=4)
    torch.cuda.synchronize()
    for gi, G in enumerate(groups):
        seg = slice(gi * B, gi * B + B)
        corrs, keys, decays = _planes(G)
        wstate = O.oracle_fold(G["ckpts"], corrs, keys, decays, source=want["source"][seg],
                               lengths=want["length"][seg], final=want["final"][seg], boundary=want["boundary"][seg],
                               boundary_len=want["boundary_len"][seg], rows=B, num_blocks=G["NB"], record_rows=B)
        targeted = set(want["final"][seg].tolist()) | set(want["boundary"][seg].tolist())
        _check_states(devs[gi][0], wstate, torch.float32, targeted)


def test_deferred_commit_rejects_groups_on_other_rows(dev):
    """One row map serves every group of a deferred step: groups on
    different logical rows (allowed in "none" mode, where they commit in
    buckets of their own) are refused before anything is launched."""
    B = 4
    groups = [_group(B, 2, 4, 64, 64, 4, 1, align=False, seed=720 + g) for g in range(2)]
    metas = []
    for gi, G in enumerate(groups):
        rows = [0, 1, 2, 3] if gi == 0 else [1, 0, 3, 2]
        ckpts, convs, recs = _to_dev(G, dev)
        ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=4, max_num_reqs=B)
        metas.append(_entry(G, ctx, dev, rows).metadata)
    one = torch.zeros(B + 1, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError, match="GDN RecoverSSM: the deferred grouped commit needs every group on one"):
        GroupedCommitCoordinator().commit_deferred(metas, one[:B], one[:B], one, one.clone())


def test_grouped_flushes_fold_each_row_once(dev):
    """``DeferredGroupedCommit.flush`` marks what it folds in every bucket's
    plan: a flush of one committed row, a flush of that row and another, then
    a flush of everything fold each pending commit once, so every group's
    pages equal the oracle's fold of the whole step."""
    B, n_groups, seed = 6, 4, 730
    gen = torch.Generator().manual_seed(seed)
    request_rows = torch.randperm(B, generator=gen).tolist()
    groups = _groups(B, n_groups, seed)
    sampled = torch.zeros(B, dtype=torch.int32)
    for b, r in enumerate(request_rows):
        sampled[r] = max(1, int(groups[0]["acc"][b]))
    metas, devs = [], []
    for G in groups:
        _index_by_request(G, request_rows)
        ckpts, convs, recs = _to_dev(G, dev)
        ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=4, max_num_reqs=B)
        devs.append((ckpts, convs))
        metas.append(_entry(G, ctx, dev, request_rows).metadata)
    mapping = torch.randperm(B + 2, generator=gen)[:B].to(torch.int32)
    cols = torch.full((B + 2,), -9, dtype=torch.int32)
    accp = torch.full((B + 2,), 7, dtype=torch.int32)
    d = GroupedCommitCoordinator().commit_deferred(metas, sampled.to(dev), mapping.to(dev), cols.to(dev),
                                                   accp.to(dev))
    torch.cuda.synchronize()
    want = _oracle_grouped(groups, sampled, mapping, cols, accp, request_rows, True, B)
    committed = [b for b in range(B) if int(want["length"][b]) > 0]
    assert len(committed) >= 2
    print(f"grouped flushes: rows {committed[:2]}", flush=True)
    d.flush(rows=[committed[0]])
    d.flush(rows=committed[:2])
    d.flush()
    torch.cuda.synchronize()
    for gi, G in enumerate(groups):
        seg = slice(gi * B, gi * B + B)
        assert int(d._plan(gi)[1][:B].abs().sum()) == 0, f"group {gi}: every pending row is marked folded"
        corrs, keys, decays = _planes(G)
        wstate = O.oracle_fold(G["ckpts"], corrs, keys, decays, source=want["source"][seg],
                               lengths=want["length"][seg], final=want["final"][seg], boundary=want["boundary"][seg],
                               boundary_len=want["boundary_len"][seg], rows=B, num_blocks=G["NB"], record_rows=B)
        targeted = set(want["final"][seg].tolist()) | set(want["boundary"][seg].tolist())
        _check_states(devs[gi][0], wstate, torch.float32, targeted)

"""GPU parity of the commit path (plan, conv compaction, fold, publication).

Bar: plan arrays, conv histories and persistent publication bit-exact; FP32
committed state within max-abs 1e-5 of the oracle relative to the pages'
max-abs; pages the commit does not target bit-identical.
"""

from types import SimpleNamespace

import pytest
import torch

import gdn_oracle as O
from gdn_recoverssm_ascend.grouped_commit import CommitEntry, GroupedCommitBucket, GroupedCommitCoordinator
from gdn_recoverssm_ascend.kernels import GDNRecoverSSMCommitContext, ReplayRecordBuffers
import sweep_cases as SC
from gpu_helpers import assert_state_close

pytestmark = pytest.mark.gpu

CONV_DIM = 40
HIST = 3


@pytest.fixture(scope="module")
def dev(gpu_device):
    return gpu_device


def _l2(x):
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + 1e-6)


def _group(B, H, HV, K, V, Q, L, *, align, seed, Bk=8, key_dtype=torch.bfloat16, state_dtype=torch.float32,
           packed=False, accepted=None, page_offset=0, qlens=None):
    """One cache group: L layers of pages, records and per-step metadata (CPU)."""
    gen = torch.Generator().manual_seed(seed)
    acc = torch.randint(0, Q + 1, (B,), generator=gen, dtype=torch.int32) if accepted is None else accepted.clone()
    qlens = torch.full((B,), Q) if qlens is None else torch.tensor(qlens)
    qsl = torch.zeros(B + 1, dtype=torch.int32)
    qsl[1:] = torch.cumsum(qlens, 0)
    if align:
        C = torch.randint(0, 5 * Bk, (B,), generator=gen)
        for r in range(0, B, 2):  # half the rows cross a boundary inside the window
            n = int(acc[r])
            if n >= 1:
                ahead = int(torch.randint(1, n + 1, (1,), generator=gen))
                C[r] = max(int(C[r]) // Bk, 1) * Bk - ahead
        W = 5 + 3
        table = torch.zeros(B, W, dtype=torch.int32)
        src_col = torch.clamp(C - 1, min=0) // Bk
        for r in range(B):
            for j in range(3):
                table[r, int(src_col[r]) + j] = 1 + page_offset + 3 * r + j
        NB = 1 + page_offset + 3 * B + 2
        src = table[torch.arange(B), src_col].clone()
        num_computed = C.to(torch.int32)
    else:
        NB = 1 + page_offset + B + 3
        src = (torch.randperm(B + 3, generator=gen)[:B] + 1 + page_offset).to(torch.int32)
        table = num_computed = None
    ckpts, convs, recs = [], [], []
    for _ in range(L):
        ckpts.append((torch.randn(NB, HV, V, K, generator=gen) * 0.1).to(state_dtype))
        convs.append(torch.randn(NB, CONV_DIM, HIST + Q - 1, generator=gen).to(torch.bfloat16))
        corr = torch.randn(B, HV, Q, V, generator=gen)
        key = _l2(torch.randn(B, H, Q, K, generator=gen)).to(key_dtype)
        decay = torch.rand(B, HV, Q, generator=gen) * 0.5 + 0.5
        if packed:
            keyv = key.float().repeat_interleave(HV // H, dim=1)
            recs.append(torch.cat([corr, keyv, decay[..., None]], dim=-1))
        else:
            recs.append((corr, key, decay))
    return dict(B=B, H=H, HV=HV, K=K, V=V, Q=Q, L=L, NB=NB, acc=acc, qsl=qsl, src=src, table=table,
                C=num_computed, Bk=Bk if align else None, ckpts=ckpts, convs=convs, recs=recs, packed=packed)


def _to_dev(G, dev):
    ckpts = [c.to(dev) for c in G["ckpts"]]
    convs = [c.to(dev) for c in G["convs"]]
    if G["packed"]:
        recs = [r.to(dev) for r in G["recs"]]
    else:
        recs = [ReplayRecordBuffers(*(t.to(dev) for t in r)) for r in G["recs"]]
    return ckpts, convs, recs


def _planes(G):
    if G["packed"]:
        V, K = G["V"], G["K"]
        return ([r[..., :V] for r in G["recs"]], [r[..., V:V + K] for r in G["recs"]], [r[..., V + K] for r in G["recs"]])
    return tuple([r[i] for r in G["recs"]] for i in range(3))


def _check_states(got_list, want_list, state_dtype, targeted_pages):
    for li, (got, want) in enumerate(zip(got_list, want_list)):
        got = got.cpu()
        untouched = [p for p in range(got.shape[0]) if p not in targeted_pages]
        assert torch.equal(got[untouched], want[untouched]), f"layer {li}: untouched pages changed"
        if state_dtype == torch.float32:
            assert_state_close(got, want, f"layer {li} state")
        else:
            err = O.max_abs_rel(got, want)
            assert err <= 8e-3, f"layer {li}: {err}"


@pytest.mark.parametrize("align", [False, True])
@pytest.mark.parametrize("packed", [False, True])
def test_single_context_commit(dev, align, packed):
    G = _group(12, 2, 4, 128, 128, 4, 2, align=align, seed=3 + align + 2 * packed, packed=packed)
    ckpts, convs, recs = _to_dev(G, dev)
    ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=4, max_num_reqs=16)
    ctx.commit(
        G["acc"].to(dev), G["src"].to(dev), G["qsl"].to(dev),
        block_table=None if not align else G["table"].to(dev),
        num_computed_tokens=None if not align else G["C"].to(dev),
        mamba_block_size=G["Bk"],
    )
    torch.cuda.synchronize()
    plan = O.oracle_plan_single(G["acc"], G["src"], G["qsl"], spec_query_len=4, num_blocks=G["NB"],
                                block_table=G["table"], num_computed=G["C"], block_size=G["Bk"])
    B = G["B"]
    assert ctx.commit_lens[:B].cpu().tolist() == plan["commit_lens"].tolist()
    assert ctx.final_state_indices[:B].cpu().tolist() == plan["final"].tolist()
    assert ctx.boundary_state_indices[:B].cpu().tolist() == plan["boundary"].tolist()
    assert ctx.boundary_recovery_lens[:B].cpu().tolist() == plan["boundary_len"].tolist()
    assert ctx.align_valid[:B].cpu().tolist() == plan["align_valid"].tolist()
    assert ctx.align_col[:B].cpu().tolist() == plan["align_col"].tolist()
    corrs, keys, decays = _planes(G)
    want = O.oracle_fold(G["ckpts"], corrs, keys, decays, source=G["src"], lengths=plan["commit_lens"],
                         final=plan["final"], boundary=plan["boundary"], boundary_len=plan["boundary_len"],
                         rows=B, num_blocks=G["NB"], record_rows=B)
    targeted = set(plan["final"].tolist()) | set(plan["boundary"].tolist())
    _check_states(ckpts, want, torch.float32, targeted)
    want_conv = O.oracle_conv_compact(G["convs"], source=G["src"], lengths=plan["commit_lens"], final=plan["final"],
                                      boundary=plan["boundary"], boundary_len=plan["boundary_len"], history=HIST,
                                      num_blocks=G["NB"], rows=B, align=align)
    for got, w in zip(convs, want_conv):
        assert torch.equal(got.cpu(), w)
    if align:
        assert int(plan["boundary_len"].gt(0).sum()) > 0, "the case must exercise boundary snapshots"


@pytest.mark.parametrize("n", [0, 1, 2, 3, 4])
def test_commit_every_accepted_length(dev, n):
    B = 6
    G = _group(B, 2, 4, 128, 128, 4, 1, align=True, seed=20 + n, accepted=torch.full((B,), n, dtype=torch.int32))
    ckpts, convs, recs = _to_dev(G, dev)
    before = [c.clone() for c in ckpts]
    ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=4, max_num_reqs=B)
    ctx.commit(G["acc"].to(dev), G["src"].to(dev), G["qsl"].to(dev), block_table=G["table"].to(dev),
               num_computed_tokens=G["C"].to(dev), mamba_block_size=G["Bk"], commit_conv=False)
    torch.cuda.synchronize()
    if n == 0:
        assert all(torch.equal(a, b) for a, b in zip(ckpts, before)), "n = 0 must leave every page bit-identical"
        return
    plan = O.oracle_plan_single(G["acc"], G["src"], G["qsl"], spec_query_len=4, num_blocks=G["NB"],
                                block_table=G["table"], num_computed=G["C"], block_size=G["Bk"])
    corrs, keys, decays = _planes(G)
    want = O.oracle_fold(G["ckpts"], corrs, keys, decays, source=G["src"], lengths=plan["commit_lens"],
                         final=plan["final"], boundary=plan["boundary"], boundary_len=plan["boundary_len"],
                         rows=B, num_blocks=G["NB"], record_rows=B)
    _check_states(ckpts, want, torch.float32, set(plan["final"].tolist()) | set(plan["boundary"].tolist()))


@pytest.mark.parametrize("state_dtype,key_dtype", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32),
                                                   (torch.float16, torch.float16)])
def test_commit_dtypes(dev, state_dtype, key_dtype):
    G = _group(8, 2, 4, 128, 128, 4, 1, align=True, seed=41, key_dtype=key_dtype, state_dtype=state_dtype)
    ckpts, convs, recs = _to_dev(G, dev)
    ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=4, max_num_reqs=8)
    ctx.commit(G["acc"].to(dev), G["src"].to(dev), G["qsl"].to(dev), block_table=G["table"].to(dev),
               num_computed_tokens=G["C"].to(dev), mamba_block_size=G["Bk"])
    torch.cuda.synchronize()
    plan = O.oracle_plan_single(G["acc"], G["src"], G["qsl"], spec_query_len=4, num_blocks=G["NB"],
                                block_table=G["table"], num_computed=G["C"], block_size=G["Bk"])
    corrs, keys, decays = _planes(G)
    want = O.oracle_fold(G["ckpts"], corrs, keys, decays, source=G["src"], lengths=plan["commit_lens"],
                         final=plan["final"], boundary=plan["boundary"], boundary_len=plan["boundary_len"],
                         rows=8, num_blocks=G["NB"], record_rows=8)
    _check_states(ckpts, want, state_dtype, set(plan["final"].tolist()) | set(plan["boundary"].tolist()))


def _index_by_request(G, request_rows):
    """The grouped plan reads the block table and positions by request index
    (grouped_commit.py:147-187): lay them out so that plan row b's request owns
    plan row b's pages. Rows never share a page, as in serving; the kernels,
    like the reference's, do not order one row's stores against another row's
    loads."""
    if G["table"] is None:
        return G
    t, c = G["table"].clone(), G["C"].clone()
    for b, r in enumerate(request_rows):
        t[r] = G["table"][b]
        c[r] = G["C"][b]
    G["table"], G["C"] = t, c
    return G


def _entry(G, ctx, dev, request_rows):
    table = torch.zeros(G["B"], G["Q"], dtype=torch.int32, device=dev)
    table[:, 0] = G["src"].to(dev)
    payload = SimpleNamespace(
        state_indices=table[:, 0],
        query_start_loc=G["qsl"].to(dev),
        request_indices=torch.tensor(request_rows, dtype=torch.int64, device=dev),
        block_table=None if G["table"] is None else G["table"].to(dev),
        num_computed_tokens=None if G["C"] is None else G["C"].to(dev),
        block_size=G["Bk"],
        request_rows=tuple(request_rows),
        query_lens=tuple(int(G["qsl"][i + 1] - G["qsl"][i]) for i in range(G["B"])),
    )
    meta = SimpleNamespace(recoverssm_commit=payload, recoverssm_builder=SimpleNamespace(), recoverssm_context=ctx)
    return CommitEntry(meta, payload, ctx)


def _oracle_grouped(groups, sampled, mapping, cols, acc, request_rows, align, capacity, publish=True):
    og = []
    for G in groups:
        og.append(dict(state_indices=G["src"], query_start_loc=G["qsl"], request_indices=torch.tensor(request_rows),
                       block_table=G["table"], num_computed=G["C"], block_size=G["Bk"], num_blocks=G["NB"]))
    return O.oracle_plan_grouped(sampled, og, spec_query_len=groups[0]["Q"], capacity=capacity, rows=groups[0]["B"],
                                 align=align, idx_mapping=mapping, persistent_cols=cols, persistent_accepted=acc,
                                 publish_align=publish)


@pytest.mark.parametrize("align", [True, False])
def test_grouped_bucket_two_groups_reordered_rows(dev, align):
    B = 6
    request_rows = [2, 0, 5, 1, 4, 3]
    sampled = torch.tensor([4, 0, 3, 1, 2, 4], dtype=torch.int32)
    groups = [_index_by_request(_group(B, 2, 4, 128, 128, 4, 2, align=align, seed=60 + g, page_offset=10 * g),
                                request_rows) for g in range(2)]
    # the accepted count is indexed by request; share it between groups
    contexts, entries, devs = [], [], []
    for G in groups:
        ckpts, convs, recs = _to_dev(G, dev)
        ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=4, max_num_reqs=B)
        contexts.append(ctx)
        devs.append((ckpts, convs))
        entries.append(_entry(G, ctx, dev, request_rows))
    bucket = GroupedCommitBucket(tuple(contexts))
    mapping = torch.tensor([3, 1, -1, 0, 5, 2], dtype=torch.int32)
    cols = torch.full((7,), -9, dtype=torch.int32)
    accp = torch.full((7,), 7, dtype=torch.int32)
    cols_d, accp_d = cols.to(dev), accp.to(dev)
    specs = bucket.make_specs(entries, sampled.to(dev), mapping.to(dev), cols_d, accp_d)
    assert [s.name for s in specs] == ["plan_fold", "conv"]
    for s in specs:
        s.launch()
    torch.cuda.synchronize()
    want = _oracle_grouped(groups, sampled, mapping, cols, accp, request_rows, align, bucket.capacity)
    cap = bucket.capacity
    for name, arr in (("source", bucket.source), ("length", bucket.length), ("final", bucket.final),
                      ("boundary", bucket.boundary), ("boundary_len", bucket.boundary_len), ("valid", bucket.valid),
                      ("col", bucket.col)):
        got = arr.cpu()
        for gi in range(2):
            seg = slice(gi * cap, gi * cap + B)
            assert got[seg].tolist() == want[name][seg].tolist(), (name, gi)
    if align:
        assert cols_d.cpu().tolist() == want["persistent_cols"].tolist()
        assert accp_d.cpu().tolist() == want["persistent_accepted"].tolist()
    else:
        assert accp_d.cpu().tolist() == [7] * 7
    for gi, G in enumerate(groups):
        seg = slice(gi * cap, gi * cap + cap)
        corrs, keys, decays = _planes(G)
        wstate = O.oracle_fold(G["ckpts"], corrs, keys, decays, source=want["source"][seg], lengths=want["length"][seg],
                               final=want["final"][seg], boundary=want["boundary"][seg],
                               boundary_len=want["boundary_len"][seg], rows=B, num_blocks=G["NB"], record_rows=B)
        targeted = set(want["final"][seg].tolist()) | set(want["boundary"][seg].tolist())
        _check_states(devs[gi][0], wstate, torch.float32, targeted)
        wconv = O.oracle_conv_compact(G["convs"], source=want["source"][seg], lengths=want["length"][seg],
                                      final=want["final"][seg], boundary=want["boundary"][seg],
                                      boundary_len=want["boundary_len"][seg], history=HIST, num_blocks=G["NB"],
                                      rows=B, align=align)
        for got, w in zip(devs[gi][1], wconv):
            assert torch.equal(got.cpu(), w)


def test_coordinator_seven_groups_three_buckets_and_publication(dev):
    B = 4
    request_rows = [1, 3, 0, 2]
    sampled = torch.tensor([2, 4, 0, 3], dtype=torch.int32)
    groups = [_group(B, 2, 4, 64, 64, 4, 1, align=True, seed=80 + g) for g in range(7)]
    # All groups share the same logical rows, positions and block size.
    for G in groups[1:]:
        G["C"] = groups[0]["C"].clone()
        G["qsl"] = groups[0]["qsl"].clone()
    metas, devs, contexts = [], [], []
    for G in groups:
        # re-derive the table/source from the shared positions
        C = G["C"].long()
        src_col = torch.clamp(C - 1, min=0) // G["Bk"]
        table = torch.zeros_like(G["table"])
        for r in range(B):
            for j in range(3):
                table[r, int(src_col[r]) + j] = 1 + 3 * r + j
        G["table"], G["src"] = table, table[torch.arange(B), src_col].clone()
        _index_by_request(G, request_rows)
        ckpts, convs, recs = _to_dev(G, dev)
        ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=4, max_num_reqs=B)
        contexts.append(ctx)
        devs.append((ckpts, convs))
        metas.append(_entry(G, ctx, dev, request_rows).metadata)
    mapping = torch.tensor([2, -1, 0, 3], dtype=torch.int32)
    cols = torch.full((5,), -9, dtype=torch.int32)
    accp = torch.full((5,), 7, dtype=torch.int32)
    cols_d, accp_d = cols.to(dev), accp.to(dev)
    coord = GroupedCommitCoordinator()
    coord.commit(metas, sampled.to(dev), mapping.to(dev), cols_d, accp_d)
    torch.cuda.synchronize()
    # three buckets of (plan + fold, conv) and one publication across buckets
    assert coord.last_group_count == 7 and coord.last_launch_count == 7
    assert [len(b.contexts) for b in coord._buckets.values()] == [3, 3, 1]
    want = _oracle_grouped(groups, sampled, mapping, cols, accp, request_rows, True, B)
    assert cols_d.cpu().tolist() == want["persistent_cols"].tolist()
    assert accp_d.cpu().tolist() == want["persistent_accepted"].tolist()
    for gi, G in enumerate(groups):
        seg = slice(gi * B, gi * B + B)
        corrs, keys, decays = _planes(G)
        wstate = O.oracle_fold(G["ckpts"], corrs, keys, decays, source=want["source"][seg], lengths=want["length"][seg],
                               final=want["final"][seg], boundary=want["boundary"][seg],
                               boundary_len=want["boundary_len"][seg], rows=B, num_blocks=G["NB"], record_rows=B)
        targeted = set(want["final"][seg].tolist()) | set(want["boundary"][seg].tolist())
        _check_states(devs[gi][0], wstate, torch.float32, targeted)


@pytest.mark.parametrize("align", [False, True])
def test_fused_plan_fold_equals_plan_then_fold(dev, align):
    """The fused entry (every fold workgroup plans its own row) against the
    plan kernel followed by the fold reading the stored plan: plan arrays,
    pages and conv states bit-identical, including padded and short rows."""
    B = 12
    G = _group(B, 2, 4, 128, 128, 4, 2, align=align, seed=91 + align, qlens=[4] * 9 + [2, 0, 4])
    G["src"][7] = -1  # a padded row
    runs = []
    for fused in (True, False):
        ckpts, convs, recs = _to_dev(G, dev)
        ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=4, max_num_reqs=16)
        src = G["src"].to(dev)
        kw = dict(block_table=None if not align else G["table"].to(dev),
                  num_computed_tokens=None if not align else G["C"].to(dev), mamba_block_size=G["Bk"])
        if not fused:
            kw["_fold_source"] = src  # the reference's three launches: plan, conv, fold
        ctx.commit(G["acc"].to(dev), src, G["qsl"].to(dev), **kw)
        torch.cuda.synchronize()
        names = [sp.name for sp in ctx._last_specs]
        assert names == (["plan_fold", "conv"] if fused else ["plan", "conv", "fold"])
        runs.append(([c.cpu() for c in ckpts], [c.cpu() for c in convs],
                     [t[:B].cpu() for t in (ctx.plan_source, ctx.commit_lens, ctx.final_state_indices,
                                            ctx.boundary_state_indices, ctx.boundary_recovery_lens, ctx.align_valid,
                                            ctx.align_col)]))
    (pa, ca, qa), (pb, cb, qb) = runs
    for x, y in zip(qa, qb):
        assert torch.equal(x, y)
    for x, y in zip(pa + ca, pb + cb):
        assert torch.equal(x, y)
    assert int(qa[1].gt(0).sum()) > 0
    if align:
        assert int(qa[4].gt(0).sum()) > 0, "the case must exercise boundary snapshots"


@pytest.mark.parametrize("align", [False, True])
def test_grouped_fused_equals_three_launches(dev, align):
    B = 6
    request_rows = [2, 0, 5, 1, 4, 3]
    sampled = torch.tensor([4, 0, 3, 1, 2, 4], dtype=torch.int32)
    results = []
    for fuse in (True, False):
        groups = [_index_by_request(_group(B, 2, 4, 128, 128, 4, 2, align=align, seed=160 + g, page_offset=10 * g),
                                    request_rows) for g in range(2)]
        contexts, entries, devs = [], [], []
        for G in groups:
            ckpts, convs, recs = _to_dev(G, dev)
            ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=4, max_num_reqs=B)
            contexts.append(ctx)
            devs.append((ckpts, convs))
            entries.append(_entry(G, ctx, dev, request_rows))
        bucket = GroupedCommitBucket(tuple(contexts))
        cols_d = torch.full((7,), -9, dtype=torch.int32, device=dev)
        accp_d = torch.full((7,), 7, dtype=torch.int32, device=dev)
        mapping = torch.tensor([3, 1, -1, 0, 5, 2], dtype=torch.int32, device=dev)
        specs = bucket.make_specs(entries, sampled.to(dev), mapping, cols_d, accp_d, fuse_plan_fold=fuse)
        assert len(specs) == (2 if fuse else 3)
        for sp in specs:
            sp.launch()
        torch.cuda.synchronize()
        results.append([t.cpu() for t in (bucket.source, bucket.length, bucket.final, bucket.boundary,
                                          bucket.boundary_len, bucket.valid, bucket.col, cols_d, accp_d)]
                       + [t.cpu() for d in devs for part in d for t in part])
    for x, y in zip(*results):
        assert torch.equal(x, y)


@pytest.mark.parametrize("case", ["f32", "odd_dim", "token_major", "many_tiles"])
def test_conv_layouts_fused_and_three_launches(dev, case):
    """Conv compaction after the fused plan + fold and after the three
    separate launches, against the oracle: FP32 conv states (24-byte windows,
    moved element by element), an odd channel count, token-major pages
    (element by element) and pages spanning several workgroups with a partial
    last one."""
    B, Q = 10, 4
    G = _group(B, 2, 4, 128, 128, Q, 2, align=True, seed=300 + len(case))
    dim = {"odd_dim": 41, "many_tiles": 3000}.get(case, CONV_DIM)
    dtype = torch.float32 if case == "f32" else torch.bfloat16
    gen = torch.Generator().manual_seed(17)
    convs = [torch.randn(G["NB"], dim, HIST + Q - 1, generator=gen).to(dtype) for _ in range(2)]
    plan = O.oracle_plan_single(G["acc"], G["src"], G["qsl"], spec_query_len=Q, num_blocks=G["NB"],
                                block_table=G["table"], num_computed=G["C"], block_size=G["Bk"])
    want = O.oracle_conv_compact(convs, source=G["src"], lengths=plan["commit_lens"], final=plan["final"],
                                 boundary=plan["boundary"], boundary_len=plan["boundary_len"], history=HIST,
                                 num_blocks=G["NB"], rows=B, align=True)
    assert int(plan["boundary_len"].gt(0).sum()) > 0 and int(plan["commit_lens"].gt(0).sum()) > 0
    token_major = case == "token_major"
    for fused in (True, False):
        ckpts, _, recs = _to_dev(G, dev)
        # token-major pages are [blocks, window, dim] in memory
        dconvs = [(c.transpose(1, 2).contiguous() if token_major else c).to(dev) for c in convs]
        ctx = GDNRecoverSSMCommitContext.from_tensors(dconvs, ckpts, recs, spec_query_len=Q, max_num_reqs=B,
                                                      conv_dim_first=not token_major)
        src = G["src"].to(dev)
        kw = dict(block_table=G["table"].to(dev), num_computed_tokens=G["C"].to(dev), mamba_block_size=G["Bk"])
        if not fused:
            kw["_fold_source"] = src  # plan, conv, fold as three launches
        ctx.commit(G["acc"].to(dev), src, G["qsl"].to(dev), **kw)
        torch.cuda.synchronize()
        assert [sp.name for sp in ctx._last_specs] == (["plan_fold", "conv"] if fused else ["plan", "conv", "fold"])
        for li, (got, w) in enumerate(zip(dconvs, want)):
            got = got.cpu()
            if token_major:
                got = got.transpose(1, 2)
            assert torch.equal(got, w), f"{case} fused={fused} layer {li}: conv states differ"


@pytest.mark.parametrize("case", range(SC.COMMIT_CASES))
def test_random_configurations(dev, case):
    """Seeded draws of every commit option together: head dims, GQA ratio,
    window, layers, none / align mode and block size, state and key dtypes,
    packed records, short and empty windows, a padded row."""
    c = SC.commit_case(case)
    print(f"commit sweep case {case}: {c}", flush=True)
    B, Q, align = c["B"], c["Q"], c["align"]
    G = _group(B, c["H"], c["HV"], c["K"], c["V"], Q, c["L"], align=align, seed=c["seed"], Bk=c["Bk"],
               key_dtype=c["key_dtype"], state_dtype=c["state_dtype"], packed=c["packed"], qlens=c["qlens"])
    if c["padded"]:
        G["src"][B // 2] = -1
    ckpts, convs, recs = _to_dev(G, dev)
    ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=Q, max_num_reqs=B + 3)
    ctx.commit(G["acc"].to(dev), G["src"].to(dev), G["qsl"].to(dev),
               block_table=G["table"].to(dev) if align else None,
               num_computed_tokens=G["C"].to(dev) if align else None, mamba_block_size=G["Bk"])
    torch.cuda.synchronize()
    plan = O.oracle_plan_single(G["acc"], G["src"], G["qsl"], spec_query_len=Q, num_blocks=G["NB"],
                                block_table=G["table"], num_computed=G["C"], block_size=G["Bk"])
    for key, t in (("commit_lens", ctx.commit_lens), ("final", ctx.final_state_indices),
                   ("boundary", ctx.boundary_state_indices), ("boundary_len", ctx.boundary_recovery_lens),
                   ("align_valid", ctx.align_valid), ("align_col", ctx.align_col)):
        assert t[:B].cpu().tolist() == plan[key].tolist(), f"plan {key} differs"
    corrs, keys, decays = _planes(G)
    want = O.oracle_fold(G["ckpts"], corrs, keys, decays, source=G["src"], lengths=plan["commit_lens"],
                         final=plan["final"], boundary=plan["boundary"], boundary_len=plan["boundary_len"],
                         rows=B, num_blocks=G["NB"], record_rows=B)
    targeted = set(plan["final"].tolist()) | set(plan["boundary"].tolist())
    _check_states(ckpts, want, c["state_dtype"], targeted)
    want_conv = O.oracle_conv_compact(G["convs"], source=G["src"], lengths=plan["commit_lens"], final=plan["final"],
                                      boundary=plan["boundary"], boundary_len=plan["boundary_len"],
                                      history=HIST, num_blocks=G["NB"], rows=B, align=align)
    for li, (got, w) in enumerate(zip(convs, want_conv)):
        assert torch.equal(got.cpu(), w), f"layer {li}: conv states differ"


@pytest.mark.parametrize("n_groups,align,B,seed,hetero", [
    (1, True, 5, 1, False), (2, False, 6, 2, False), (4, True, 3, 3, False), (5, False, 7, 4, False),
    (7, True, 6, 5, False), (6, True, 4, 6, False), (4, True, 5, 7, True), (3, False, 4, 8, True),
])
def test_coordinator_groups_against_oracle(dev, n_groups, align, B, seed, hetero):
    """The coordinator over 1-7 cache groups (buckets of up to three), none
    and align mode, shuffled request rows, and (hetero) groups of two record
    layouts that land in separate buckets (FP32 keys in every other group):
    plan, folded pages, conv states and the align publication, which must wait
    for every bucket, against the oracle group by group; a second commit of
    the same groups reuses the buckets (grouped_commit.py:955-1002)."""
    gen = torch.Generator().manual_seed(seed)
    request_rows = torch.randperm(B, generator=gen).tolist()
    sampled = torch.randint(0, 5, (B,), generator=gen, dtype=torch.int32)
    key_dtypes = [torch.float32 if hetero and g % 2 else torch.bfloat16 for g in range(n_groups)]
    groups = [_group(B, 2, 4, 64, 64, 4, 1 + g % 2, align=align, seed=400 + 10 * seed + g, page_offset=3 * g,
                     key_dtype=key_dtypes[g]) for g in range(n_groups)]
    for G in groups[1:]:
        G["qsl"] = groups[0]["qsl"].clone()
        if align:
            G["C"] = groups[0]["C"].clone()
    metas, devs = [], []
    for G in groups:
        if align:
            C = G["C"].long()
            src_col = torch.clamp(C - 1, min=0) // G["Bk"]
            table = torch.zeros_like(G["table"])
            for r in range(B):
                for j in range(3):
                    table[r, int(src_col[r]) + j] = 1 + 3 * r + j
            G["table"], G["src"] = table, table[torch.arange(B), src_col].clone()
        _index_by_request(G, request_rows)
        ckpts, convs, recs = _to_dev(G, dev)
        ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=4, max_num_reqs=B)
        devs.append((ckpts, convs))
        metas.append(_entry(G, ctx, dev, request_rows).metadata)
    mapping = torch.randperm(B + 2, generator=gen)[:B].to(torch.int32)
    mapping[0] = -1
    cols = torch.full((B + 2,), -9, dtype=torch.int32)
    accp = torch.full((B + 2,), 7, dtype=torch.int32)
    cols_d, accp_d = cols.to(dev), accp.to(dev)
    print(f"coordinator: {n_groups} groups align={align} B={B} requests={request_rows}", flush=True)
    coord = GroupedCommitCoordinator()
    coord.commit(metas, sampled.to(dev), mapping.to(dev), cols_d, accp_d)
    torch.cuda.synchronize()
    n_fp32 = sum(dt == torch.float32 for dt in key_dtypes)
    buckets = -(-(n_groups - n_fp32) // 3) + -(-n_fp32 // 3)
    assert coord.last_group_count == n_groups and len(coord._buckets) == buckets
    assert coord.last_launch_count == 2 * buckets + (1 if align and buckets > 1 else 0)
    want = _oracle_grouped(groups, sampled, mapping, cols, accp, request_rows, align, B)
    if align:
        assert cols_d.cpu().tolist() == want["persistent_cols"].tolist()
        assert accp_d.cpu().tolist() == want["persistent_accepted"].tolist()
    for gi, G in enumerate(groups):
        seg = slice(gi * B, gi * B + B)
        corrs, keys, decays = _planes(G)
        wstate = O.oracle_fold(G["ckpts"], corrs, keys, decays, source=want["source"][seg], lengths=want["length"][seg],
                               final=want["final"][seg], boundary=want["boundary"][seg],
                               boundary_len=want["boundary_len"][seg], rows=B, num_blocks=G["NB"], record_rows=B)
        targeted = set(want["final"][seg].tolist()) | set(want["boundary"][seg].tolist())
        _check_states(devs[gi][0], wstate, torch.float32, targeted)
        wconv = O.oracle_conv_compact(G["convs"], source=want["source"][seg], lengths=want["length"][seg],
                                      final=want["final"][seg], boundary=want["boundary"][seg],
                                      boundary_len=want["boundary_len"][seg], history=HIST, num_blocks=G["NB"],
                                      rows=B, align=align)
        for li, (got, w) in enumerate(zip(devs[gi][1], wconv)):
            assert torch.equal(got.cpu(), w), f"group {gi} layer {li}: conv states differ"
    assert int(want["length"].gt(0).sum()) > 0
    # the same groups again: same buckets, no new epoch
    first = dict(coord._buckets)
    coord.commit(metas, torch.zeros(B, dtype=torch.int32, device=dev), mapping.to(dev), cols_d, accp_d)
    torch.cuda.synchronize()
    assert coord._buckets.keys() == first.keys()
    assert all(coord._buckets[k] is first[k] for k in first)


@pytest.mark.parametrize("case", range(SC.COORDINATOR_CASES))
def test_random_coordinator_commits(dev, case):
    """Seeded draws of a grouped commit through the coordinator: 1-7 cache
    groups on one set of shuffled request rows, each with its own layer count
    and record layout (groups of different layouts commit in separate
    buckets), none or align mode, head dims, window and state dtype: plans,
    folded pages, conv states and the align publication across every bucket
    against the oracle, group by group."""
    c = SC.coordinator_case(case)
    print(f"coordinator sweep case {case}: {c}", flush=True)
    B, Q, align, n_groups = c["B"], c["Q"], c["align"], c["n_groups"]
    gen = torch.Generator().manual_seed(c["seed"])
    request_rows = torch.randperm(B, generator=gen).tolist()
    sampled = torch.randint(0, Q + 1, (B,), generator=gen, dtype=torch.int32)
    sampled[0] = max(int(sampled[0]), 1)
    groups = []
    for g in range(n_groups):
        layout = c["layouts"][g]
        groups.append(_group(B, c["H"], c["HV"], c["K"], c["V"], Q, c["layers"][g], align=align,
                             seed=c["seed"] + 7 * g, page_offset=3 * g, state_dtype=c["state"],
                             key_dtype=torch.float32 if layout == "f32" else torch.bfloat16,
                             packed=layout == "packed"))
    for G in groups[1:]:
        G["qsl"] = groups[0]["qsl"].clone()
        if align:
            G["C"] = groups[0]["C"].clone()
    metas, devs = [], []
    for G in groups:
        if align:
            src_col = torch.clamp(G["C"].long() - 1, min=0) // G["Bk"]
            table = torch.zeros_like(G["table"])
            for r in range(B):
                for j in range(3):
                    table[r, int(src_col[r]) + j] = 1 + 3 * r + j
            G["table"], G["src"] = table, table[torch.arange(B), src_col].clone()
        _index_by_request(G, request_rows)
        ckpts, convs, recs = _to_dev(G, dev)
        ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=Q, max_num_reqs=B)
        devs.append((ckpts, convs))
        metas.append(_entry(G, ctx, dev, request_rows).metadata)
    mapping = torch.randperm(B + 2, generator=gen)[:B].to(torch.int32)
    cols = torch.full((B + 2,), -9, dtype=torch.int32)
    accp = torch.full((B + 2,), 7, dtype=torch.int32)
    cols_d, accp_d = cols.to(dev), accp.to(dev)
    coord = GroupedCommitCoordinator()
    coord.commit(metas, sampled.to(dev), mapping.to(dev), cols_d, accp_d)
    torch.cuda.synchronize()
    assert coord.last_group_count == n_groups
    want = _oracle_grouped(groups, sampled, mapping, cols, accp, request_rows, align, B)
    if align:
        assert cols_d.cpu().tolist() == want["persistent_cols"].tolist(), "publication differs"
        assert accp_d.cpu().tolist() == want["persistent_accepted"].tolist(), "publication differs"
    for gi, G in enumerate(groups):
        seg = slice(gi * B, gi * B + B)
        corrs, keys, decays = _planes(G)
        wstate = O.oracle_fold(G["ckpts"], corrs, keys, decays, source=want["source"][seg], lengths=want["length"][seg],
                               final=want["final"][seg], boundary=want["boundary"][seg],
                               boundary_len=want["boundary_len"][seg], rows=B, num_blocks=G["NB"], record_rows=B)
        targeted = set(want["final"][seg].tolist()) | set(want["boundary"][seg].tolist())
        _check_states(devs[gi][0], wstate, c["state"], targeted)
        wconv = O.oracle_conv_compact(G["convs"], source=want["source"][seg], lengths=want["length"][seg],
                                      final=want["final"][seg], boundary=want["boundary"][seg],
                                      boundary_len=want["boundary_len"][seg], history=HIST, num_blocks=G["NB"],
                                      rows=B, align=align)
        for li, (got, w) in enumerate(zip(devs[gi][1], wconv)):
            assert torch.equal(got.cpu(), w), f"group {gi} layer {li}: conv states differ"


@pytest.mark.parametrize("align", [False, True])
def test_commit_int64_metadata(dev, align):
    """int64 accepted counts, state indices (a column view of a wider table),
    query offsets, request mapping, block table and computed-token counts:
    the same plan, pages and conv states as the oracle."""
    B = 9
    G = _group(B, 2, 4, 128, 128, 4, 1, align=align, seed=55 + align, qlens=[4] * 7 + [3, 0])
    ckpts, convs, recs = _to_dev(G, dev)
    ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=4, max_num_reqs=B)
    table64 = torch.zeros(B, 5, dtype=torch.int64, device=dev)
    table64[:, 0] = G["src"].to(dev).long()
    i64 = lambda t: None if t is None else t.long().to(dev)  # noqa: E731
    ctx.commit(i64(G["acc"]), table64[:, 0], i64(G["qsl"]), request_indices=torch.arange(B, device=dev),
               block_table=i64(G["table"]), num_computed_tokens=i64(G["C"]), mamba_block_size=G["Bk"])
    torch.cuda.synchronize()
    plan = O.oracle_plan_single(G["acc"], G["src"], G["qsl"], spec_query_len=4, num_blocks=G["NB"],
                                block_table=G["table"], num_computed=G["C"], block_size=G["Bk"])
    for key, t in (("commit_lens", ctx.commit_lens), ("final", ctx.final_state_indices),
                   ("boundary", ctx.boundary_state_indices), ("boundary_len", ctx.boundary_recovery_lens)):
        assert t[:B].cpu().tolist() == plan[key].tolist(), f"plan {key} differs"
    corrs, keys, decays = _planes(G)
    want = O.oracle_fold(G["ckpts"], corrs, keys, decays, source=G["src"], lengths=plan["commit_lens"],
                         final=plan["final"], boundary=plan["boundary"], boundary_len=plan["boundary_len"],
                         rows=B, num_blocks=G["NB"], record_rows=B)
    _check_states(ckpts, want, torch.float32, set(plan["final"].tolist()) | set(plan["boundary"].tolist()))
    want_conv = O.oracle_conv_compact(G["convs"], source=G["src"], lengths=plan["commit_lens"], final=plan["final"],
                                      boundary=plan["boundary"], boundary_len=plan["boundary_len"], history=HIST,
                                      num_blocks=G["NB"], rows=B, align=align)
    assert torch.equal(convs[0].cpu(), want_conv[0])
    assert int(plan["commit_lens"].gt(0).sum()) > 0


# A configuration drawn by the random sweep (case 405 of a 50-fold sweep) that
# found 16-bit boundary snapshots with a wrong first dword in some lanes: the
# value the next instruction read reached memory when a 128-bit store's data
# registers were reused right after it (csrc/gdn_common.cuh,
# store_b128_settled). Kept as a fixed case, run several times because the
# failure depended on timing.
_SNAPSHOT_CASE = dict(B=9, H=3, HV=12, K=40, V=100, Q=8, L=3, align=True, seed=905, Bk=8, key_dtype=torch.float32,
                      packed=True, qlens=[7, 5, 6, 0, 5, 8, 8, 2, 6])


@pytest.mark.parametrize("state_dtype", [torch.float16, torch.bfloat16])
def test_16bit_boundary_snapshot_stores(dev, state_dtype):
    c = dict(_SNAPSHOT_CASE, state_dtype=state_dtype)
    B, Q = c["B"], c["Q"]
    G = _group(B, c["H"], c["HV"], c["K"], c["V"], Q, c["L"], align=True, seed=c["seed"], Bk=c["Bk"],
               key_dtype=c["key_dtype"], state_dtype=state_dtype, packed=c["packed"], qlens=c["qlens"])
    plan = O.oracle_plan_single(G["acc"], G["src"], G["qsl"], spec_query_len=Q, num_blocks=G["NB"],
                                block_table=G["table"], num_computed=G["C"], block_size=G["Bk"])
    # rows whose boundary snapshot goes back to their source page
    alias = [r for r in range(B) if int(plan["commit_lens"][r]) > 0 and int(plan["boundary"][r]) == int(G["src"][r])
             and int(plan["boundary"][r]) != int(plan["final"][r])]
    assert len(alias) >= 3
    corrs, keys, decays = _planes(G)
    want = O.oracle_fold(G["ckpts"], corrs, keys, decays, source=G["src"], lengths=plan["commit_lens"],
                         final=plan["final"], boundary=plan["boundary"], boundary_len=plan["boundary_len"],
                         rows=B, num_blocks=G["NB"], record_rows=B)
    targeted = set(plan["final"].tolist()) | set(plan["boundary"].tolist())
    for rep in range(5):
        print(f"16-bit snapshot case: {state_dtype} repetition {rep}", flush=True)
        ckpts, convs, recs = _to_dev(G, dev)
        ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=Q, max_num_reqs=B + 3)
        ctx.commit(G["acc"].to(dev), G["src"].to(dev), G["qsl"].to(dev), block_table=G["table"].to(dev),
                   num_computed_tokens=G["C"].to(dev), mamba_block_size=G["Bk"])
        torch.cuda.synchronize()
        _check_states(ckpts, want, state_dtype, targeted)

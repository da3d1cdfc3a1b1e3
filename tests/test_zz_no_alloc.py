"""The no-allocation commit, ``gdn_recoverssm_commit_noalloc``, called through
the C ABI, against the commit with caller-owned plan arrays
(``gdn_recoverssm_plan_fold`` then ``gdn_recoverssm_conv_compact``, the launches
``GDNRecoverSSMCommitContext.commit`` and ``GroupedCommitBucket`` make) on
copies of the same pages.

Pages, conv states and the align publication must come out bit-identical (the
two run the same kernels), on two calls in a row, the second with fewer rows:
the library's plan buffer keeps the first call's contents, which the second
must not read. Each single-context call is also checked against the CPU oracle
directly (``oracle_plan_single``, ``oracle_fold``, ``oracle_conv_compact``):
FP32 pages within max-abs 1e-5 relative to the pages' max-abs, pages outside
the commit and conv histories bit-exact.
"""

import ctypes

import pytest
import torch

import gdn_oracle as O
import sweep_cases as SC
from gdn_recoverssm_ascend import _native as N
from gdn_recoverssm_ascend.grouped_commit import GroupedCommitBucket
from gdn_recoverssm_ascend.kernels import GDNRecoverSSMCommitContext
from test_gpu_commit import HIST, _check_states, _entry, _group, _index_by_request, _planes, _to_dev

pytestmark = pytest.mark.gpu

_PLAN_ARRAYS = ("source_plan", "lens_plan", "final_plan", "boundary_plan", "boundary_lens_plan", "valid_plan",
                "col_plan")


@pytest.fixture(scope="module")
def dev(gpu_device):
    return gpu_device


def _commit_noalloc(specs, device):
    """Call the no-allocation entry with the arguments of a plan + fold spec
    and a conv spec (built, not launched): the plan block without its arrays,
    the fold's tables and configuration, the conv tables."""
    fused, conv = specs
    assert (fused.name, conv.name) == ("plan_fold", "conv")
    launch = N.PlanLaunch.from_buffer_copy(fused.keepalive[2])
    for name in _PLAN_ARRAYS:
        setattr(launch, name, None)
    a = conv.args
    tables = N.ConvLaunch(conv_addrs=a[0], conv_block_strides=a[1], conv_dim_strides=a[2], conv_token_strides=a[3],
                          conv_dim=a[16], history=a[17], window=a[18], element_bytes=a[20])
    lib = N.load()
    status = lib.gdn_recoverssm_commit_noalloc(ctypes.byref(launch), *fused.args[1:], ctypes.byref(tables),
                                               N.stream_handle(device))
    N.check(status, "commit_noalloc")


def _copies(G, dev):
    return _to_dev(G, dev), _to_dev(G, dev)


def _assert_same(ref, got, before, what):
    (rc, rv), (gc, gv) = ref, got
    for li, (a, b) in enumerate(zip(rc, gc)):
        assert torch.equal(a, b), f"{what}: layer {li} pages differ"
    for li, (a, b) in enumerate(zip(rv, gv)):
        assert torch.equal(a, b), f"{what}: layer {li} conv states differ"
    assert any(not torch.equal(a, b) for a, b in zip(rc, before)), f"{what}: the commit changed no page"


@pytest.mark.parametrize("align", [True, False])
def test_single_context_two_calls(dev, align):
    """Single-context commits of 24 rows, then 10 rows, two layers each."""
    for call, (B, seed) in enumerate(((24, 301), (10, 302))):
        G = _group(B, 2, 4, 128, 128, 4, 2, align=align, seed=seed + 10 * align)
        (rc, rv, rr), (gc, gv, gr) = _copies(G, dev)
        before = [c.clone() for c in rc]
        meta = dict(block_table=G["table"].to(dev) if align else None,
                    num_computed_tokens=G["C"].to(dev) if align else None, mamba_block_size=G["Bk"])
        acc, src, qsl = G["acc"].to(dev), G["src"].to(dev), G["qsl"].to(dev)
        ref_ctx = GDNRecoverSSMCommitContext.from_tensors(rv, rc, rr, spec_query_len=4, max_num_reqs=32)
        ref_ctx.commit(acc, src, qsl, **meta)
        ctx = GDNRecoverSSMCommitContext.from_tensors(gv, gc, gr, spec_query_len=4, max_num_reqs=32)
        _commit_noalloc(ctx.make_commit_specs(acc, src, qsl, **meta), dev)
        torch.cuda.synchronize()
        what = f"call {call} (B={B}, align={align})"
        _assert_same((rc, rv), (gc, gv), before, what)
        _assert_oracle(G, gc, gv, align, what)


def _assert_oracle(G, pages, convs, align, what):
    """The no-allocation commit's pages and conv states against the oracle."""
    B = G["B"]
    plan = O.oracle_plan_single(G["acc"], G["src"], G["qsl"], spec_query_len=4, num_blocks=G["NB"],
                                block_table=G["table"], num_computed=G["C"], block_size=G["Bk"])
    corrs, keys, decays = _planes(G)
    want = O.oracle_fold(G["ckpts"], corrs, keys, decays, source=G["src"], lengths=plan["commit_lens"],
                         final=plan["final"], boundary=plan["boundary"], boundary_len=plan["boundary_len"],
                         rows=B, num_blocks=G["NB"], record_rows=B)
    _check_states(pages, want, torch.float32, set(plan["final"].tolist()) | set(plan["boundary"].tolist()))
    want_conv = O.oracle_conv_compact(G["convs"], source=G["src"], lengths=plan["commit_lens"], final=plan["final"],
                                      boundary=plan["boundary"], boundary_len=plan["boundary_len"], history=HIST,
                                      num_blocks=G["NB"], rows=B, align=align)
    for li, (got, w) in enumerate(zip(convs, want_conv)):
        assert torch.equal(got.cpu(), w), f"{what}: layer {li} conv states differ from the oracle"
    assert int(plan["commit_lens"].gt(0).sum()) > 0, f"{what}: nothing committed"


def test_captured_commit_replays(dev):
    """The no-allocation commit captured into a HIP graph (torch.cuda.graph)
    after one eager call, then replayed three times on fresh copies of the
    same pages, with eager copies and synchronisations between replays: every
    replay's pages and conv states bit-identical to the eager call's."""
    B = 16
    G = _group(B, 2, 4, 128, 128, 4, 2, align=True, seed=333)
    pages, convs, recs = _to_dev(G, dev)
    fresh = [c.clone() for c in pages], [c.clone() for c in convs]
    meta = dict(block_table=G["table"].to(dev), num_computed_tokens=G["C"].to(dev), mamba_block_size=G["Bk"])
    acc, src, qsl = G["acc"].to(dev), G["src"].to(dev), G["qsl"].to(dev)
    ctx = GDNRecoverSSMCommitContext.from_tensors(convs, pages, recs, spec_query_len=4, max_num_reqs=B)
    specs = ctx.make_commit_specs(acc, src, qsl, **meta)

    def reset():
        for dst, s0 in zip(pages + convs, fresh[0] + fresh[1]):
            dst.copy_(s0)

    _commit_noalloc(specs, dev)  # eager: the reference result (and the buffer's address lookup)
    torch.cuda.synchronize()
    want = [c.clone() for c in pages], [c.clone() for c in convs]
    _assert_oracle(G, want[0], want[1], True, "eager call")
    reset()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _commit_noalloc(specs, dev)
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(pages, fresh[0])), "capturing must not run the commit"
    for replay in range(3):
        reset()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for li, (a, b) in enumerate(zip(pages, want[0])):
            assert torch.equal(a, b), f"replay {replay}: layer {li} pages differ from the eager call"
        for li, (a, b) in enumerate(zip(convs, want[1])):
            assert torch.equal(a, b), f"replay {replay}: layer {li} conv states differ from the eager call"


def _bucket_commit(groups, dev, request_rows, sampled, mapping, noalloc):
    """One two-group bucket commit with publication; returns the pages, conv
    states and persistent outputs."""
    contexts, entries, state = [], [], []
    for G in groups:
        ckpts, convs, recs = _to_dev(G, dev)
        ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=4, max_num_reqs=8)
        contexts.append(ctx)
        state.append((ckpts, convs))
        entries.append(_entry(G, ctx, dev, request_rows))
    bucket = GroupedCommitBucket(tuple(contexts))
    cols = torch.full((9,), -9, dtype=torch.int32, device=dev)
    accp = torch.full((9,), 7, dtype=torch.int32, device=dev)
    specs = bucket.make_specs(entries, sampled.to(dev), mapping.to(dev), cols, accp)
    if noalloc:
        _commit_noalloc(specs, dev)
    else:
        for spec in specs:
            spec.launch()
    torch.cuda.synchronize()
    return state, cols, accp


@pytest.mark.parametrize("align", [True, False])
def test_grouped_bucket_two_calls(dev, align):
    """A two-group bucket (requests reordered, align publication) of 6 rows,
    then one of 4 rows."""
    cases = (([2, 0, 5, 1, 4, 3], [4, 0, 3, 1, 2, 4], [3, 1, -1, 0, 5, 2], 71),
             ([2, 0, 3, 1], [1, 4, 2, 3], [1, -1, 0, 2], 83))
    for call, (request_rows, accepted, mapping, seed) in enumerate(cases):
        B = len(request_rows)
        # One seed for both groups: the same positions, so that every valid
        # row's groups agree on its column and the row is published.
        groups = [_index_by_request(_group(B, 2, 4, 128, 128, 4, 2, align=align, seed=seed, page_offset=10 * g),
                                    request_rows) for g in range(2)]
        sampled = torch.tensor(accepted, dtype=torch.int32)
        mapping = torch.tensor(mapping, dtype=torch.int32)
        before = [[c.to(dev) for c in G["ckpts"]] for G in groups]
        ref = _bucket_commit(groups, dev, request_rows, sampled, mapping, noalloc=False)
        got = _bucket_commit(groups, dev, request_rows, sampled, mapping, noalloc=True)
        what = f"call {call} (B={B}, align={align})"
        for gi in range(2):
            _assert_same(ref[0][gi], got[0][gi], before[gi], f"{what} group {gi}")
        assert torch.equal(ref[1], got[1]) and torch.equal(ref[2], got[2]), f"{what}: publication differs"
        if align:
            assert int((got[2] == 1).sum()) > 0, f"{what}: nothing was published"


@pytest.mark.parametrize("case", range(SC.COMMIT_CASES // 2))
def test_random_configurations_two_calls(dev, case):
    """Two seeded random commit draws in a row (head dims, GQA ratio, window,
    layers, none / align mode and block size, state and key dtypes, packed
    records, short and empty windows, a padded row): each call of the
    no-allocation commit bit-identical to the commit with caller-owned plan
    arrays, the second reading none of what the first left in the buffer."""
    for call, draw in enumerate((2 * case, 2 * case + 1)):
        c = SC.commit_case(draw)
        print(f"no-allocation sweep case {case} call {call}: {c}", flush=True)
        B, Q, align = c["B"], c["Q"], c["align"]
        G = _group(B, c["H"], c["HV"], c["K"], c["V"], Q, c["L"], align=align, seed=c["seed"], Bk=c["Bk"],
                   key_dtype=c["key_dtype"], state_dtype=c["state_dtype"], packed=c["packed"], qlens=c["qlens"])
        if c["padded"]:
            G["src"][B // 2] = -1
        (rc, rv, rr), (gc, gv, gr) = _copies(G, dev)
        meta = dict(block_table=G["table"].to(dev) if align else None,
                    num_computed_tokens=G["C"].to(dev) if align else None, mamba_block_size=G["Bk"])
        acc, src, qsl = G["acc"].to(dev), G["src"].to(dev), G["qsl"].to(dev)
        ref_ctx = GDNRecoverSSMCommitContext.from_tensors(rv, rc, rr, spec_query_len=Q, max_num_reqs=B + 3)
        ref_ctx.commit(acc, src, qsl, **meta)
        ctx = GDNRecoverSSMCommitContext.from_tensors(gv, gc, gr, spec_query_len=Q, max_num_reqs=B + 3)
        _commit_noalloc(ctx.make_commit_specs(acc, src, qsl, **meta), dev)
        torch.cuda.synchronize()
        for li, (a, b) in enumerate(zip(rc, gc)):
            assert torch.equal(a, b), f"draw {draw}: layer {li} pages differ"
        for li, (a, b) in enumerate(zip(rv, gv)):
            assert torch.equal(a, b), f"draw {draw}: layer {li} conv states differ"

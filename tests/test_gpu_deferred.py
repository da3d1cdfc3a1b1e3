"""The deferred commit: the fold of step k applied inside step k+1's verify
(``gdn_recoverssm_verify_deferred``), checked two ways.

* Against the CPU oracle, step by step: after each deferred verify every page
  equals the oracle's fold of the previous step (pages outside that commit
  bit-identical), this step's outputs and records equal ``oracle_verify`` from
  those pages, and the plan equals ``oracle_plan_single`` bit for bit; after
  the final flush the pages equal the oracle's last fold.
* Against the ordinary flow (verify, then commit: plan + fold + conv), bit for
  bit: outputs, records, plans, pages and conv states.

Batch changes between steps go through ``continue_pending`` (rows keyed by
request) and ``flush_deferred(rows=...)`` (the commits of requests that left),
and are checked against the oracle as well: a request that leaves with an
align-mode commit that crosses a block boundary, a new request taking a row,
a reordered batch, a batch that grows past the pending plan's rows, and a
step without a single token.

Bar: plan and page indexing bit-exact; FP32 pages within max-abs 1e-5
relative to the pages' max-abs (16-bit pages within 8e-3, one rounding);
outputs within 1e-2 norm-wise; corrections within 1e-5 norm-wise; keys
bit-exact; decays within 2 FP32 ulp.
"""

import pytest
import torch

import gdn_oracle as O
import sweep_cases as SC
from gdn_recoverssm_ascend import workloads as W
from gdn_recoverssm_ascend.kernels import (
    GDNRecoverSSMCommitContext,
    ReplayRecordBuffers,
    _fold_rows_spec,
    _settle_spec,
    continue_pending,
    gdn_recoverssm_verify,
    gdn_recoverssm_verify_deferred,
)
from gpu_helpers import (CORR_TOL, OUT_TOL, assert_norm_close, assert_state_close, retain_settings,
                         state_cache_retain)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(gpu_device):
    return gpu_device


def _check_pages(got, want, touched, what):
    """Pages outside `touched` bit-identical, the rest within the state bar."""
    got = got.cpu()
    untouched = [p for p in range(got.shape[0]) if p not in touched]
    assert torch.equal(got[untouched], want[untouched]), f"{what}: pages outside the commit changed"
    if want.dtype == torch.float32:
        assert_state_close(got, want, what)
    else:
        err = O.max_abs_rel(got, want)
        assert err <= 8e-3, f"{what}: max-abs error / max-abs = {err:.3g} > 8e-3"


def _check_verify(out, rec, r, what):
    """GPU outputs and records of one layer against an oracle VerifyResult."""
    got = out.cpu()[0]
    wm = r.out_written
    if bool(wm.any()):
        assert_norm_close(got[wm].double(), r.out[wm], OUT_TOL, f"{what} out")
    rw = r.record_written  # [R, Q]
    if not bool(rw.any()):
        return
    R = rw.shape[0]
    corr, key, decay = rec.correction[:R].cpu(), rec.key[:R].cpu(), rec.decay[:R].cpu()
    m_c = rw[:, None, :, None].expand_as(corr)
    assert_norm_close(corr[m_c].double(), r.correction[m_c], CORR_TOL, f"{what} correction")
    m_d = rw[:, None, :].expand_as(decay)
    torch.testing.assert_close(decay[m_d].double(), r.decay[m_d], rtol=3e-7, atol=0)
    m_k = rw[:, None, :, None].expand_as(key)
    assert torch.equal(key[m_k].float(), r.key[m_k].float()), f"{what}: keys must keep the input bits"


def _touched(plan, rows, num_pages):
    n, fin, bnd, blen = (plan[k][:rows] for k in ("commit_lens", "final", "boundary", "boundary_len"))
    pages = set()
    for i in range(rows):
        if int(n[i]) > 0:
            pages.add(int(fin[i]))
            if 0 < int(bnd[i]) < num_pages and int(bnd[i]) != int(fin[i]) and 0 < int(blen[i]) <= int(n[i]):
                pages.add(int(bnd[i]))
    return pages


def _oracle_fold(pages, results, plan, rows, num_pages, lengths=None):
    return O.oracle_fold(pages, [r.correction for r in results], [r.key for r in results],
                         [r.decay for r in results], source=plan["source"],
                         lengths=plan["commit_lens"] if lengths is None else lengths, final=plan["final"],
                         boundary=plan["boundary"], boundary_len=plan["boundary_len"], rows=rows,
                         num_blocks=num_pages, record_rows=rows, out_dtype=pages[0].dtype)


def _step_inputs(w, layer, T):
    i = w.inputs[layer]
    return i.g[:T], i.beta[:T], i.q[:, :T], i.k[:, :T], i.v[:, :T]


def _run_against_oracle(w, dev, acc_steps, qsl_steps):
    """The deferred flow over len(acc_steps) carried steps, each checked
    against the oracle as described in the module docstring."""
    s = w.spec
    L, B, Q, H, HV, K, V = s.layers, s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
    wd = w.to(dev)
    ckpts = [c.clone() for c in wd.checkpoints]
    convs = [c.clone() for c in wd.conv_states]
    recs = [[ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=wd.inputs[0].k.dtype)
             for _ in range(L)] for _ in range(2)]
    ctxs = [GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs[i], spec_query_len=Q, max_num_reqs=B)
            for i in range(2)]
    state_idx = wd.meta.state_indices.clone()
    computed = wd.meta.num_computed.clone()
    src_cpu = w.meta.state_indices.clone()
    c_cpu = w.meta.num_computed.clone()
    want = [c.clone() for c in w.checkpoints]
    touched = set()
    pending = None
    commits = crossings = 0
    for step, (acc, qsl) in enumerate(zip(acc_steps, qsl_steps)):
        i = step % 2
        T = int(qsl[-1])
        qd = qsl.to(dev)
        outs = []
        for layer in range(L):
            kw = dict(checkpoint_state=ckpts[layer], replay_cache=recs[i][layer], query_start_loc=qd,
                      state_indices=state_idx, spec_query_len=Q)
            args = _step_inputs(wd, layer, T)
            if pending is None:
                outs.append(gdn_recoverssm_verify(*args, **kw))
            else:
                outs.append(gdn_recoverssm_verify_deferred(*args, pending=pending[layer], **kw))
        torch.cuda.synchronize()
        cur = []
        for layer in range(L):
            _check_pages(ckpts[layer], want[layer], touched, f"step {step} layer {layer}: pages after the verify")
            cur.append(ckpts[layer].cpu())
        results = []
        for layer in range(L):
            ci = w.inputs[layer]
            r = O.oracle_verify(ci.q[:, :T], ci.k[:, :T], ci.v[:, :T], ci.g[:T], ci.beta[:T], cur[layer], qsl, src_cpu, Q)
            _check_verify(outs[layer], recs[i][layer], r, f"step {step} layer {layer}")
            results.append(r)
        pending = ctxs[i].commit_deferred(acc.to(dev), state_idx, qd, block_table=wd.meta.block_table,
                                          num_computed_tokens=computed, mamba_block_size=s.block_size)
        plan = O.oracle_plan_single(acc, src_cpu, qsl, spec_query_len=Q, num_blocks=w.num_pages,
                                    block_table=w.meta.block_table, num_computed=c_cpu, block_size=s.block_size)
        ctx = ctxs[i]
        for name, t in (("commit_lens", ctx.commit_lens), ("final", ctx.final_state_indices),
                        ("boundary", ctx.boundary_state_indices), ("boundary_len", ctx.boundary_recovery_lens)):
            assert t[:B].cpu().tolist() == plan[name].tolist(), f"step {step}: plan {name} differs"
        plan["source"] = src_cpu
        want = _oracle_fold(cur, results, plan, B, w.num_pages)
        touched = _touched(plan, B, w.num_pages)
        commits += int((plan["commit_lens"] > 0).sum())
        crossings += len(touched) - int((plan["commit_lens"] > 0).sum())
        n = plan["commit_lens"]
        src_cpu = torch.where(n > 0, plan["final"], src_cpu).to(torch.int32)
        c_cpu = (c_cpu + n).to(c_cpu.dtype)
        lens = ctx.commit_lens[:B]
        state_idx.copy_(torch.where(lens > 0, ctx.final_state_indices[:B], state_idx))
        computed.add_(lens.to(computed.dtype))
    ctxs[(len(acc_steps) - 1) % 2].flush_deferred()
    torch.cuda.synchronize()
    for layer in range(L):
        _check_pages(ckpts[layer], want[layer], touched, f"layer {layer}: pages after the flush")
    assert commits > 0 and crossings > 0, "the steps committed nothing or crossed no block boundary"


@pytest.mark.parametrize("seed,empty_row,state_dtype", [
    (5, None, torch.float32),
    (9, 3, torch.float32),
    (13, None, torch.bfloat16),
    (17, 2, torch.float16),
])
def test_deferred_commit_against_oracle(dev, seed, empty_row, state_dtype):
    """Four carried steps, align mode with boundary crossings and a padded
    row; with `empty_row`, step 2 gives that row no token while it carries a
    pending commit (the verify must fold it anyway)."""
    steps = 4
    w = W.make_workload("decode_loop_l48", layers=2, rows=10, key_heads=2, value_heads=4, key_dim=128, value_dim=128,
                        steps=steps, max_position=512, block_size=8, padded_rows=1, seed=seed,
                        state_dtype=state_dtype)
    s = w.spec
    print(f"deferred vs oracle: seed={seed} empty_row={empty_row} state={state_dtype}", flush=True)
    gen = torch.Generator().manual_seed(seed + 1)
    acc_steps = [W.sample_accepted(s, s.rows, gen) for _ in range(steps)]
    qsl_steps = [w.meta.query_start_loc.clone() for _ in range(steps)]
    if empty_row is not None:
        lens = torch.full((s.rows,), s.window, dtype=torch.int32)
        lens[empty_row] = 0
        q2 = torch.zeros(s.rows + 1, dtype=torch.int32)
        q2[1:] = torch.cumsum(lens, 0)
        qsl_steps[2] = q2
    _run_against_oracle(w, dev, acc_steps, qsl_steps)


def test_deferred_step_without_tokens(dev):
    """A step whose batch has no token at all while every row carries a
    pending commit: the launch still applies the commits (g, beta, q, k, v
    are empty tensors, so their pointers are null) and the pages equal the
    oracle's fold; the next step verifies from them."""
    steps = 3
    w = W.make_workload("decode_loop_l48", layers=1, rows=8, key_heads=2, value_heads=4, key_dim=128, value_dim=64,
                        steps=steps, max_position=256, block_size=8, padded_rows=1, seed=31)
    s = w.spec
    gen = torch.Generator().manual_seed(32)
    acc_steps = [torch.full((s.rows,), s.window, dtype=torch.int32)] + [W.sample_accepted(s, s.rows, gen)
                                                                        for _ in range(steps - 1)]
    qsl_steps = [w.meta.query_start_loc.clone(), torch.zeros(s.rows + 1, dtype=torch.int32),
                 w.meta.query_start_loc.clone()]
    _run_against_oracle(w, dev, acc_steps, qsl_steps)


def _flow(w, dev, acc_steps, qsl_steps, *, deferred, settle=False, move=None):
    """Verify + commit over the steps, ordinary or deferred. ``settle``: the
    deferred flow settles before every verify after the first step.
    ``move`` = (step, row, page): before that step's verifies the row's
    state index becomes `page` (a page no row uses), in both flows."""
    s = w.spec
    L, B, Q, H, HV, K, V = s.layers, s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
    wd = w.to(dev)
    ckpts = [c.clone() for c in wd.checkpoints]
    convs = [c.clone() for c in wd.conv_states]
    recs = [[ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=wd.inputs[0].k.dtype)
             for _ in range(L)] for _ in range(2)]
    ctxs = [GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs[i], spec_query_len=Q, max_num_reqs=B)
            for i in range(2)]
    state_idx = wd.meta.state_indices.clone()
    computed = wd.meta.num_computed.clone()
    pending = None
    history = []
    for step, (acc, qsl) in enumerate(zip(acc_steps, qsl_steps)):
        i = step % 2
        qsl = qsl.to(dev)
        if move is not None and move[0] == step:
            state_idx[move[1]] = move[2]
        if deferred and settle and pending is not None:
            ctxs[1 - i].settle_deferred(state_idx, pending[0].rows)
        outs = []
        for layer in range(L):
            T = int(qsl[-1])
            args = _step_inputs(wd, layer, T)
            kw = dict(checkpoint_state=ckpts[layer], replay_cache=recs[i][layer], query_start_loc=qsl,
                      state_indices=state_idx, spec_query_len=Q)
            if deferred and pending is not None:
                outs.append(gdn_recoverssm_verify_deferred(*args, pending=pending[layer], **kw))
            else:
                outs.append(gdn_recoverssm_verify(*args, **kw))
        commit_args = (acc.to(dev), state_idx, qsl)
        commit_kw = dict(block_table=wd.meta.block_table, num_computed_tokens=computed,
                         mamba_block_size=s.block_size)
        if deferred:
            pending = ctxs[i].commit_deferred(*commit_args, **commit_kw)
        else:
            ctxs[i].commit(*commit_args, **commit_kw)
        ctx = ctxs[i]
        lens = ctx.commit_lens[:B]
        state_idx.copy_(torch.where(lens > 0, ctx.final_state_indices[:B], state_idx))
        computed.add_(lens.to(computed.dtype))
        torch.cuda.synchronize()
        history.append(dict(
            out=[o.clone() for o in outs],
            corr=[r.correction.clone() for r in recs[i]], key=[r.key.clone() for r in recs[i]],
            decay=[r.decay.clone() for r in recs[i]],
            plan=[t[:B].clone() for t in (ctx.commit_lens, ctx.final_state_indices, ctx.boundary_state_indices,
                                          ctx.boundary_recovery_lens)],
            state_idx=state_idx.clone(),
        ))
    if deferred:
        ctxs[(len(acc_steps) - 1) % 2].flush_deferred()
    torch.cuda.synchronize()
    return history, ckpts, convs


def _assert_flows_equal(ref, got):
    (ref_h, ref_pages, ref_convs), (got_h, got_pages, got_convs) = ref, got
    for step, (a, b) in enumerate(zip(ref_h, got_h)):
        for name in ("out", "corr", "key", "decay", "plan"):
            for li, (x, y) in enumerate(zip(a[name], b[name])):
                assert torch.equal(x, y), f"step {step} {name} [{li}] differs"
        assert torch.equal(a["state_idx"], b["state_idx"])
    for li, (x, y) in enumerate(zip(ref_pages, got_pages)):
        assert torch.equal(x, y), f"layer {li}: pages differ after the flush"
    for li, (x, y) in enumerate(zip(ref_convs, got_convs)):
        assert torch.equal(x, y), f"layer {li}: conv states differ"
    assert sum(int((h["plan"][0] > 0).sum()) for h in ref_h) > 0


@pytest.mark.parametrize("seed,empty_row", [(5, None), (9, 3)])
def test_deferred_commit_equals_ordinary_flow(dev, seed, empty_row):
    steps = 4
    w = W.make_workload("decode_loop_l48", layers=2, rows=10, key_heads=2, value_heads=4, key_dim=128, value_dim=128,
                        steps=steps, max_position=512, block_size=8, padded_rows=1, seed=seed)
    s = w.spec
    gen = torch.Generator().manual_seed(seed + 1)
    acc_steps = [W.sample_accepted(s, s.rows, gen) for _ in range(steps)]
    qsl_steps = [w.meta.query_start_loc.clone() for _ in range(steps)]
    if empty_row is not None:
        lens = torch.full((s.rows,), s.window, dtype=torch.int32)
        lens[empty_row] = 0
        q2 = torch.zeros(s.rows + 1, dtype=torch.int32)
        q2[1:] = torch.cumsum(lens, 0)
        qsl_steps[2] = q2
    ref = _flow(w, dev, acc_steps, qsl_steps, deferred=False)
    got = _flow(w, dev, acc_steps, qsl_steps, deferred=True)
    _assert_flows_equal(ref, got)
    assert sum(int((h["plan"][2] > 0).sum()) for h in ref[0]) > 0
    # The cache hint changes only the ordinary verify of each flow's first step
    # (every row non-temporal, then the later half ordinary); the deferred
    # verify reads every row non-temporally whatever it says.
    for retain in retain_settings(s.rows, s.value_heads * s.value_dim * s.key_dim * 4)[:2]:
        with state_cache_retain(retain):
            _assert_flows_equal(ref, _flow(w, dev, acc_steps, qsl_steps, deferred=True))


@pytest.mark.parametrize("K,V,Q,H,HV,act,state", [
    (64, 100, 3, 1, 4, torch.bfloat16, torch.float32),
    (256, 64, 8, 2, 2, torch.bfloat16, torch.float32),
    (32, 192, 1, 2, 8, torch.float16, torch.float32),
    (136, 48, 5, 3, 6, torch.float32, torch.float32),
    (96, 16, 6, 1, 1, torch.bfloat16, torch.float32),
    (128, 128, 4, 2, 4, torch.bfloat16, torch.bfloat16),
    (64, 72, 3, 1, 2, torch.float16, torch.float16),
    (256, 40, 8, 2, 4, torch.float32, torch.bfloat16),
])
def test_deferred_commit_equals_ordinary_flow_shapes(dev, K, V, Q, H, HV, act, state):
    """The same equality over head dims off the 128 x 128 tile (partial
    64-row half tiles, K padded to whole chunks), windows 1-8, GQA ratios 1-4,
    every activation dtype and every state dtype."""
    steps = 3
    w = W.make_workload("decode_loop_l48", layers=2, rows=6, key_heads=H, value_heads=HV, key_dim=K, value_dim=V,
                        window=Q, act_dtype=act, state_dtype=state, steps=steps, max_position=256, block_size=8,
                        padded_rows=1, seed=K + V + Q)
    s = w.spec
    print(f"deferred shapes: K={K} V={V} Q={Q} H={H} HV={HV} act={act} state={state}", flush=True)
    gen = torch.Generator().manual_seed(K * V + Q)
    acc_steps = [W.sample_accepted(s, s.rows, gen) for _ in range(steps)]
    qsl_steps = [w.meta.query_start_loc.clone() for _ in range(steps)]
    ref = _flow(w, dev, acc_steps, qsl_steps, deferred=False)
    _assert_flows_equal(ref, _flow(w, dev, acc_steps, qsl_steps, deferred=True))
    with state_cache_retain(0):  # the first step's ordinary verify: every row non-temporal
        _assert_flows_equal(ref, _flow(w, dev, acc_steps, qsl_steps, deferred=True))


@pytest.mark.parametrize("case", range(SC.DEFERRED_CASES))
def test_random_deferred_flows(dev, case):
    """Seeded draws of the deferred flow's options together (head dims, GQA
    ratio, window, activation and state dtypes, rows, layers, steps, block
    size, a step in which one row has no token, a row given another page
    before a later step): the deferred flow, settling before every verify
    after the first step, equals the ordinary flow bit for bit, step by step,
    and after the final flush."""
    c = SC.deferred_case(case)
    print(f"deferred sweep case {case}: {c}", flush=True)
    w = W.make_workload("decode_loop_l48", layers=c["layers"], rows=c["rows"], key_heads=c["H"],
                        value_heads=c["HV"], key_dim=c["K"], value_dim=c["V"], window=c["Q"], act_dtype=c["act"],
                        state_dtype=c["state"], steps=c["steps"], max_position=256, block_size=c["block_size"],
                        padded_rows=1, seed=c["seed"])
    s = w.spec
    gen = torch.Generator().manual_seed(c["seed"] + 1)
    acc_steps = [W.sample_accepted(s, s.rows, gen) for _ in range(c["steps"])]
    acc_steps[0] = acc_steps[0].clamp(min=1)  # a small batch could otherwise commit nothing at all
    qsl_steps = [w.meta.query_start_loc.clone() for _ in range(c["steps"])]
    if c["empty_row"]:
        lens = torch.full((s.rows,), s.window, dtype=torch.int32)
        lens[case % s.rows] = 0
        q2 = torch.zeros(s.rows + 1, dtype=torch.int32)
        q2[1:] = torch.cumsum(lens, 0)
        qsl_steps[-1] = q2
    move = None
    if c["move"]:
        # a continued request given another page before a later step: a page
        # of the padded row's table, which no row reads or writes
        pad = int(w.extras["padded_rows"][0])
        pages = [int(p) for p in w.meta.block_table[pad].tolist() if 0 < int(p) < w.num_pages]
        rows = [r for r in range(s.rows) if r != pad]
        move = (1 + case % (c["steps"] - 1), rows[case % len(rows)], pages[0])
    print(f"deferred sweep case {case}: move {move}", flush=True)
    ref = _flow(w, dev, acc_steps, qsl_steps, deferred=False, move=move)
    _assert_flows_equal(ref, _flow(w, dev, acc_steps, qsl_steps, deferred=True, settle=True, move=move))


def _first_step(w, dev, acc):
    """Step 0 on the GPU: ordinary verify, then commit_deferred. Returns the
    device state, the pending commits, the oracle results and plan."""
    s = w.spec
    L, B, Q, H, HV, K, V = s.layers, s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
    wd = w.to(dev)
    ckpts = [c.clone() for c in wd.checkpoints]
    convs = [c.clone() for c in wd.conv_states]
    recs = [[ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=wd.inputs[0].k.dtype)
             for _ in range(L)] for _ in range(2)]
    ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs[0], spec_query_len=Q, max_num_reqs=2 * B)
    m = wd.meta
    for layer in range(L):
        gdn_recoverssm_verify(*_step_inputs(wd, layer, w.tokens), checkpoint_state=ckpts[layer],
                              replay_cache=recs[0][layer], query_start_loc=m.query_start_loc,
                              state_indices=m.state_indices, spec_query_len=Q)
    pending = ctx.commit_deferred(acc.to(dev), m.state_indices, m.query_start_loc, block_table=m.block_table,
                                  num_computed_tokens=m.num_computed, mamba_block_size=s.block_size)
    cm = w.meta
    results = [O.oracle_verify(i.q, i.k, i.v, i.g, i.beta, c, cm.query_start_loc, cm.state_indices, Q)
               for i, c in zip(w.inputs, w.checkpoints)]
    plan = O.oracle_plan_single(acc, cm.state_indices, cm.query_start_loc, spec_query_len=Q, num_blocks=w.num_pages,
                                block_table=cm.block_table, num_computed=cm.num_computed, block_size=s.block_size)
    plan["source"] = cm.state_indices.clone()
    torch.cuda.synchronize()
    for name, t in (("commit_lens", ctx.commit_lens), ("final", ctx.final_state_indices),
                    ("boundary", ctx.boundary_state_indices)):
        assert t[:B].cpu().tolist() == plan[name].tolist(), f"step 0: plan {name} differs"
    return dict(ckpts=ckpts, recs=recs, ctx=ctx, pending=pending, results=results, plan=plan)


def test_batch_change_with_flush(dev):
    """Step 1 keeps most requests in a shuffled order, drops two (one of them
    with an align-mode commit that writes a boundary snapshot) and admits a
    new request on a page of its own. The row map comes from
    ``continue_pending``; the verify applies the continued requests' commits
    and ``flush_deferred(rows=left)`` the departed ones'. Every page then
    equals the oracle's fold of step 0, the departed rows' final and boundary
    pages included, and step 1's outputs equal the oracle's verify from those
    pages (the new request's from its own unfolded page)."""
    w = W.make_workload("decode_loop_l48", layers=2, rows=12, key_heads=2, value_heads=4, key_dim=128, value_dim=128,
                        steps=2, max_position=512, block_size=8, padded_rows=1, seed=41)
    s = w.spec
    L, B, Q = s.layers, s.rows, s.window
    acc = torch.full((B,), Q, dtype=torch.int32)
    acc[::3] = 2
    st = _first_step(w, dev, acc)
    plan = st["plan"]
    n, fin, bnd = plan["commit_lens"], plan["final"], plan["boundary"]
    pad = int(w.extras["padded_rows"][0])
    crossing = [r for r in range(B) if int(n[r]) > 0 and int(bnd[r]) > 0 and int(bnd[r]) != int(fin[r])]
    plain = [r for r in range(B) if int(n[r]) > 0 and r not in crossing]
    assert crossing and plain, "the seed must give a crossing and a plain commit"
    leaving = [crossing[0], plain[0]]
    gen = torch.Generator().manual_seed(42)
    stay = [r for r in range(B) if r not in leaving and r != pad]
    stay = [stay[i] for i in torch.randperm(len(stay), generator=gen).tolist()]
    new_request = 1000
    next_requests = stay[:3] + [new_request] + stay[3:]
    B1 = len(next_requests)
    # Step-1 metadata: continued requests from their committed page and
    # position, the new request from the padded row's own (never written) page.
    src_col = w.extras["source_col"]
    table = w.meta.block_table
    new_page = int(table[pad, src_col[pad]])
    idx1 = torch.tensor([new_page if r == new_request else (int(fin[r]) if int(n[r]) > 0 else
                                                            int(w.meta.state_indices[r])) for r in next_requests],
                        dtype=torch.int32)
    qsl1 = torch.arange(B1 + 1, dtype=torch.int32) * Q
    inputs1 = [W.make_layer_inputs(s, B1 * Q, gen) for _ in range(L)]
    pending1, left = continue_pending(st["pending"], list(range(B)), next_requests)
    assert left == sorted(leaving + [pad])
    assert pending1[0].rows.cpu().tolist() == [-1 if r == new_request else r for r in next_requests]

    ckpts, recs, ctx = st["ckpts"], st["recs"], st["ctx"]
    qd, idx_d = qsl1.to(dev), idx1.to(dev)
    outs = []
    for layer in range(L):
        i = inputs1[layer]
        outs.append(gdn_recoverssm_verify_deferred(
            i.g.to(dev), i.beta.to(dev), i.q.to(dev), i.k.to(dev), i.v.to(dev), checkpoint_state=ckpts[layer],
            replay_cache=recs[1][layer], pending=pending1[layer], query_start_loc=qd, state_indices=idx_d,
            spec_query_len=Q))
    torch.cuda.synchronize()
    # The departed requests' final pages are still unwritten: no verify applied them.
    before = [c.cpu() for c in w.checkpoints]
    for layer in range(L):
        for r in leaving:
            assert torch.equal(ckpts[layer][int(fin[r])].cpu(), before[layer][int(fin[r])]), "a departed fold ran"
    ctx.flush_deferred(rows=left)
    torch.cuda.synchronize()
    want = _oracle_fold(before, st["results"], plan, B, w.num_pages)
    touched = _touched(plan, B, w.num_pages)
    for layer in range(L):
        _check_pages(ckpts[layer], want[layer], touched, f"layer {layer}: pages after verify + flush")
        for r in leaving:  # named explicitly: the departed rows' final (and boundary) pages
            pages = [int(fin[r])] + ([int(bnd[r])] if r in crossing else [])
            for p in pages:
                assert_state_close(ckpts[layer][p].cpu(), want[layer][p], f"layer {layer}: departed row {r} page {p}")
    for layer in range(L):
        i = inputs1[layer]
        r1 = O.oracle_verify(i.q, i.k, i.v, i.g, i.beta, want[layer], qsl1, idx1, Q)
        _check_verify(outs[layer], recs[1][layer], r1, f"step 1 layer {layer}")


def test_flush_of_listed_rows_folds_each_once(dev):
    """``flush_deferred(rows=...)`` launches the fold over the listed rows
    only (the fold's row list): rows given in any order and more than once
    are folded once each, and a device row list that is not strictly
    increasing folds a repeated row once (the kernel skips an entry not
    above the one before it). Pages equal the oracle's fold of exactly those
    rows; every other page, the other rows' final pages included, is
    unchanged."""
    w = W.make_workload("decode_loop_l48", layers=2, rows=12, key_heads=2, value_heads=4, key_dim=128, value_dim=128,
                        steps=2, max_position=512, block_size=8, padded_rows=1, seed=43)
    s = w.spec
    L, B, Q = s.layers, s.rows, s.window
    acc = torch.full((B,), Q, dtype=torch.int32)
    acc[1::3] = 1
    st = _first_step(w, dev, acc)
    plan, ctx, ckpts = st["plan"], st["ctx"], st["ckpts"]
    n = plan["commit_lens"]
    active = [r for r in range(B) if int(n[r]) > 0]
    assert len(active) >= 5
    a, b, c = active[0], active[2], active[4]
    print(f"listed flush: rows {a}, {b}, {c}", flush=True)
    ctx.flush_deferred(rows=[c, a, c])
    _fold_rows_spec(ctx._deferred_fold, torch.tensor([b, b], dtype=torch.int32, device=dev)).launch()
    torch.cuda.synchronize()
    lengths = torch.zeros_like(n)
    lengths[[a, b, c]] = n[[a, b, c]]
    before = [x.cpu() for x in w.checkpoints]
    want = _oracle_fold(before, st["results"], plan, B, w.num_pages, lengths=lengths)
    touched = _touched(dict(plan, commit_lens=lengths), B, w.num_pages)
    for layer in range(L):
        _check_pages(ckpts[layer], want[layer], touched, f"layer {layer}: pages after the listed flush")


def test_settle_folds_what_the_verify_does_not_apply(dev):
    """``settle_deferred`` decides on the device which pending rows the next
    verify will not apply and folds exactly those: here two departed requests
    (one whose commit writes a boundary snapshot) and a continued request
    whose next state index names another page than its pending final page.
    The verify then applies the rest. Every page equals the oracle's fold of
    step 0 (each commit folded once), and step 1's outputs equal the oracle's
    verify from those pages, the moved request's from its new, unfolded page."""
    w = W.make_workload("decode_loop_l48", layers=2, rows=12, key_heads=2, value_heads=4, key_dim=128, value_dim=128,
                        steps=2, max_position=512, block_size=8, padded_rows=1, seed=41)
    s = w.spec
    L, B, Q = s.layers, s.rows, s.window
    acc = torch.full((B,), Q, dtype=torch.int32)
    acc[::3] = 2
    st = _first_step(w, dev, acc)
    plan = st["plan"]
    n, fin, bnd = plan["commit_lens"], plan["final"], plan["boundary"]
    pad = int(w.extras["padded_rows"][0])
    crossing = [r for r in range(B) if int(n[r]) > 0 and int(bnd[r]) > 0 and int(bnd[r]) != int(fin[r])]
    plain = [r for r in range(B) if int(n[r]) > 0 and r not in crossing]
    assert crossing and len(plain) > 1, "the seed must give a crossing and two plain commits"
    leaving = [crossing[0], plain[0]]
    moved = plain[1]
    gen = torch.Generator().manual_seed(44)
    stay = [r for r in range(B) if r not in leaving and r != pad]
    stay = [stay[i] for i in torch.randperm(len(stay), generator=gen).tolist()]
    new_request = 1000
    next_requests = stay[:3] + [new_request] + stay[3:]
    B1 = len(next_requests)
    src_col = w.extras["source_col"]
    table = w.meta.block_table
    new_page = int(table[pad, src_col[pad]])
    moved_page = int(table[pad, src_col[pad] + 1])  # the padded row's next page: no row uses it
    assert moved_page > 0 and moved_page != new_page

    def next_index(r):
        if r == new_request:
            return new_page
        if r == moved:
            return moved_page
        return int(fin[r]) if int(n[r]) > 0 else int(w.meta.state_indices[r])

    idx1 = torch.tensor([next_index(r) for r in next_requests], dtype=torch.int32)
    qsl1 = torch.arange(B1 + 1, dtype=torch.int32) * Q
    inputs1 = [W.make_layer_inputs(s, B1 * Q, gen) for _ in range(L)]
    pending1, left = continue_pending(st["pending"], list(range(B)), next_requests)
    assert left == sorted(leaving + [pad])
    ckpts, recs, ctx = st["ckpts"], st["recs"], st["ctx"]
    qd, idx_d = qsl1.to(dev), idx1.to(dev)
    before = [c.cpu() for c in w.checkpoints]
    ctx.settle_deferred(idx_d, pending1[0].rows)
    torch.cuda.synchronize()
    settled = torch.tensor([1 if r in leaving or r == moved else 0 for r in range(B)], dtype=torch.int32)
    part = _oracle_fold(before, st["results"], plan, B, w.num_pages, lengths=plan["commit_lens"] * settled)
    touched_part = _touched({**plan, "commit_lens": plan["commit_lens"] * settled}, B, w.num_pages)
    for layer in range(L):
        _check_pages(ckpts[layer], part[layer], touched_part, f"layer {layer}: pages after the settle")
    outs = []
    for layer in range(L):
        i = inputs1[layer]
        outs.append(gdn_recoverssm_verify_deferred(
            i.g.to(dev), i.beta.to(dev), i.q.to(dev), i.k.to(dev), i.v.to(dev), checkpoint_state=ckpts[layer],
            replay_cache=recs[1][layer], pending=pending1[layer], query_start_loc=qd, state_indices=idx_d,
            spec_query_len=Q))
    torch.cuda.synchronize()
    want = _oracle_fold(before, st["results"], plan, B, w.num_pages)
    touched = _touched(plan, B, w.num_pages)
    for layer in range(L):
        _check_pages(ckpts[layer], want[layer], touched, f"layer {layer}: pages after settle + verify")
        i = inputs1[layer]
        r1 = O.oracle_verify(i.q, i.k, i.v, i.g, i.beta, want[layer], qsl1, idx1, Q)
        _check_verify(outs[layer], recs[1][layer], r1, f"step 1 layer {layer}")


def _settle(dev, lengths, finals, cap, num_rows, rows, nexts):
    """gdn_recoverssm_settle on the GPU for len(nexts) groups of `cap` plan
    rows; its outputs start poisoned. Returns (lengths, listed rows)."""
    lengths_d, finals_d = lengths.to(dev), finals.to(dev)
    out = torch.full(lengths.shape, -7, dtype=torch.int32, device=dev)
    rl = torch.full((max(num_rows, 1),), -9, dtype=torch.int32, device=dev)
    cnt = torch.full((1,), -5, dtype=torch.int32, device=dev)
    nexts_d = [None if x is None else x.to(dev) for x in nexts]
    _settle_spec(lengths_d, finals_d, cap, num_rows, rows.to(dev), nexts_d, out, rl, cnt).launch()
    torch.cuda.synchronize()
    n = int(cnt.cpu())
    assert 0 <= n <= num_rows
    got = out.cpu()
    # the plan keeps every length except those handed to the fold (marked 0)
    marked = lengths.clone()
    for g in range(len(nexts)):
        for r in range(num_rows):
            if int(got[g * cap + r]) > 0:
                marked[g * cap + r] = 0
    assert torch.equal(lengths_d.cpu(), marked), "the plan's lengths after the settle"
    return got, rl.cpu()[:n]


def _settled_by_definition(lengths, finals, cap, num_rows, rows, nexts):
    """Group g's pending row r < num_rows keeps its length unless some next
    row b has rows[b] == r and nexts[g][b] == its final page; entries past
    num_rows are kept. The listed rows: every r < num_rows with a length
    left in some group, ascending."""
    out = lengths.clone()
    for g, nxt in enumerate(nexts):
        if nxt is None:
            continue
        pairs = set(zip(rows[:nxt.shape[0]].tolist(), nxt.tolist()))  # (rows[b], nxt[b]) over the next rows
        for r in range(num_rows):
            if (r, int(finals[g * cap + r])) in pairs:
                out[g * cap + r] = 0
    listed = [r for r in range(num_rows) if any(int(out[g * cap + r]) > 0 for g in range(len(nexts)))]
    return out, listed


def test_settle_known_cases(dev):
    """What a settle folds, for hand-made batches: next row 0 continues
    pending row 2 on its final page (applied), next row 1 continues pending
    row 0 on another page (not applied), next row 2 is a new request, next
    row 3 applies pending row 3, pending row 1 left; the entry past the
    pending rows keeps its length and is not listed."""
    i32 = torch.int32
    lengths = torch.tensor([3, 2, 1, 4, 7], dtype=i32)
    finals = torch.tensor([10, 11, 12, 13, 14], dtype=i32)
    rows = torch.tensor([2, 0, -1, 3], dtype=i32)
    nxt = torch.tensor([12, 99, 5, 13], dtype=i32)
    out, listed = _settle(dev, lengths, finals, 5, 4, rows, [nxt])
    assert out.tolist() == [3, 2, 0, 0, 7] and listed.tolist() == [0, 1]
    # an empty next batch applies nothing; a zero length is not listed
    lengths0 = torch.tensor([3, 0, 1, 4, 7], dtype=i32)
    out, listed = _settle(dev, lengths0, finals, 5, 5, torch.tensor([-1], dtype=i32), [torch.zeros(0, dtype=i32)])
    assert out.tolist() == [3, 0, 1, 4, 7] and listed.tolist() == [0, 2, 3, 4]
    # a row map longer than the batch: only the batch's rows count; a row
    # index past the pending rows names no pending row (entry 4 is row 4,
    # past num_rows = 4, whose next index equals its final page)
    out, listed = _settle(dev, lengths, finals, 5, 4, torch.tensor([4, 1, 0, 2], dtype=i32),
                          [torch.tensor([14, 11], dtype=torch.int64)])
    assert out.tolist() == [3, 0, 1, 4, 7] and listed.tolist() == [0, 2, 3]
    # next state indices as a column of an int64 table (element stride 3)
    table = torch.tensor([[12, 0, 0], [99, 0, 0], [5, 0, 0], [13, 0, 0]], dtype=torch.int64)
    out, listed = _settle(dev, lengths, finals, 5, 4, rows, [table[:, 0]])
    assert out.tolist() == [3, 2, 0, 0, 7] and listed.tolist() == [0, 1]
    # two groups (plan rows g * 5 + r), a row listed when either group keeps
    # a length; a third group outside the next step keeps every length
    lengths3 = torch.cat([lengths, torch.tensor([0, 5, 6, 2, 1], dtype=i32), torch.tensor([1, 1, 0, 0, 9], dtype=i32)])
    finals3 = torch.cat([finals, torch.tensor([20, 21, 22, 23, 24], dtype=i32), finals])
    out, listed = _settle(dev, lengths3, finals3, 5, 4, rows,
                          [nxt, torch.tensor([22, 20, 9, 23], dtype=i32), None])
    assert out.tolist() == [3, 2, 0, 0, 7, 0, 5, 0, 0, 1, 1, 1, 0, 0, 9]
    assert listed.tolist() == [0, 1]


@pytest.mark.parametrize("seed", range(10))
def test_settle_random_batches(dev, seed):
    """Seeded batches, from a few rows to several times the kernel's 1024
    threads (plan, pending rows and next batch), 1-3 groups (some outside the
    next step), int32 or int64 next indices, contiguous or a strided column:
    lengths and listed rows equal the definition, row by row."""
    gen = torch.Generator().manual_seed(100 + seed)
    cap = [5, 300, 1500, 4000, 3000][seed % 5]
    groups = 1 + seed % 3
    num_rows = int(torch.randint(0, cap + 1, (1,), generator=gen))
    lengths = torch.randint(0, 5, (groups * cap,), generator=gen, dtype=torch.int32)
    finals = torch.randint(1, 50, (groups * cap,), generator=gen, dtype=torch.int32)
    nb = int(torch.randint(0, 2 * cap + 1, (1,), generator=gen))
    rows = torch.randint(-1, cap + 3, (nb + 3,), generator=gen, dtype=torch.int32)
    nexts = []
    for g in range(groups):
        if g == 2 and seed % 2:
            nexts.append(None)
            continue
        own = finals[g * cap + rows[:nb].clamp(0, cap - 1).long()]
        nxt = torch.where(torch.rand(nb, generator=gen) < 0.6, own,
                          torch.randint(1, 50, (nb,), generator=gen, dtype=torch.int32))
        if (seed + g) % 2:
            nxt = torch.stack([nxt.long(), torch.zeros_like(nxt.long())], 1)[:, 0]  # int64, stride 2
        nexts.append(nxt)
    print(f"settle seed {seed}: {groups} groups of {cap}, pending {num_rows}, next {nb}", flush=True)
    out, listed = _settle(dev, lengths, finals, cap, num_rows, rows, nexts)
    want, want_listed = _settled_by_definition(lengths, finals, cap, num_rows, rows, nexts)
    assert torch.equal(out, want), seed
    assert listed.tolist() == want_listed, seed


def test_flushes_and_settles_fold_each_row_once(dev):
    """A settle or a flush marks what it folds in the plan, so repeated and
    mixed calls fold every pending row once: a flush of row a, a flush of a
    and b, a settle in which a and b left and row c was given another page
    (folding c), the same settle again, then a flush of everything (the rows
    no verify has applied). The pages then equal the oracle's fold of the
    whole step, each commit applied once."""
    w = W.make_workload("decode_loop_l48", layers=2, rows=12, key_heads=2, value_heads=4, key_dim=128, value_dim=128,
                        steps=2, max_position=512, block_size=8, padded_rows=1, seed=47)
    s = w.spec
    L, B, Q = s.layers, s.rows, s.window
    acc = torch.full((B,), Q, dtype=torch.int32)
    acc[1::3] = 2
    st = _first_step(w, dev, acc)
    plan, ctx, ckpts = st["plan"], st["ctx"], st["ckpts"]
    n, fin = plan["commit_lens"], plan["final"]
    active = [r for r in range(B) if int(n[r]) > 0]
    assert len(active) >= 3
    a, b, c = active[0], active[1], active[2]
    pad = int(w.extras["padded_rows"][0])
    free_page = next(int(p) for p in w.meta.block_table[pad].tolist() if 0 < int(p) < w.num_pages)
    print(f"fold once: rows a={a} b={b} c={c}, c moves to page {free_page}", flush=True)
    before = [x.cpu() for x in w.checkpoints]
    ctx.flush_deferred(rows=[a])
    ctx.flush_deferred(rows=[a, b])
    # the next batch: a and b replaced by new requests, c on another page,
    # every other row on its final page
    rows = torch.arange(B, dtype=torch.int32)
    rows[a] = rows[b] = -1
    nxt = torch.where(n > 0, fin, torch.zeros_like(fin)).to(torch.int32)
    nxt[c] = free_page
    ctx.settle_deferred(nxt.to(dev), rows.to(dev))
    ctx.settle_deferred(nxt.to(dev), rows.to(dev))
    ctx.flush_deferred()
    torch.cuda.synchronize()
    assert int(ctx.commit_lens[:B].cpu().abs().sum()) == 0, "every pending row is marked folded"
    want = _oracle_fold(before, st["results"], plan, B, w.num_pages)
    touched = _touched(plan, B, w.num_pages)
    for layer in range(L):
        _check_pages(ckpts[layer], want[layer], touched, f"layer {layer}: pages after the flushes and settles")


def test_a_flushed_row_is_not_applied_again_by_the_verify(dev):
    """A row flushed before the next verify (its request continues on its
    final page) is marked folded, so that verify reads the folded final page
    instead of applying the commit a second time: after the flush of two
    continuing rows and every layer's deferred verify, the pages equal the
    oracle's fold of the whole step (each commit once) and the outputs equal
    the oracle's verify from those pages."""
    w = W.make_workload("decode_loop_l48", layers=2, rows=12, key_heads=2, value_heads=4, key_dim=128, value_dim=128,
                        steps=2, max_position=512, block_size=8, padded_rows=1, seed=53)
    s = w.spec
    L, B, Q = s.layers, s.rows, s.window
    acc = torch.full((B,), Q, dtype=torch.int32)
    acc[2::5] = 1
    st = _first_step(w, dev, acc)
    plan, ctx, ckpts, recs, pending = st["plan"], st["ctx"], st["ckpts"], st["recs"], st["pending"]
    n, fin = plan["commit_lens"], plan["final"]
    active = [r for r in range(B) if int(n[r]) > 0]
    assert len(active) >= 4
    flushed = [active[1], active[3]]
    print(f"flush before the verify: rows {flushed}", flush=True)
    before = [x.cpu() for x in w.checkpoints]
    ctx.flush_deferred(rows=flushed)
    idx1 = torch.where(n > 0, fin.to(torch.int32), w.meta.state_indices.to(torch.int32))
    gen = torch.Generator().manual_seed(54)
    inputs1 = [W.make_layer_inputs(s, B * Q, gen) for _ in range(L)]
    qd, idx_d = w.meta.query_start_loc.to(dev), idx1.to(dev)
    outs = []
    for layer in range(L):
        i = inputs1[layer]
        outs.append(gdn_recoverssm_verify_deferred(
            i.g.to(dev), i.beta.to(dev), i.q.to(dev), i.k.to(dev), i.v.to(dev), checkpoint_state=ckpts[layer],
            replay_cache=recs[1][layer], pending=pending[layer], query_start_loc=qd, state_indices=idx_d,
            spec_query_len=Q))
    torch.cuda.synchronize()
    want = _oracle_fold(before, st["results"], plan, B, w.num_pages)
    touched = _touched(plan, B, w.num_pages)
    for layer in range(L):
        _check_pages(ckpts[layer], want[layer], touched, f"layer {layer}: pages after the flush and the verify")
        i = inputs1[layer]
        r1 = O.oracle_verify(i.q, i.k, i.v, i.g, i.beta, want[layer], w.meta.query_start_loc, idx1, Q)
        _check_verify(outs[layer], recs[1][layer], r1, f"step 1 layer {layer}")


def test_deferred_step_graph_replay(dev):
    """The start of a deferred step recorded in a HIP graph: a settle (one
    continued row given another page, so it folds that row's commit through
    the counted row list) and every layer's deferred verify. Three replays,
    each from the same pages and plan with eager work in between, reproduce
    the eager launches bit for bit: pages, outputs, records and the plan's
    marks."""
    w = W.make_workload("decode_loop_l48", layers=2, rows=12, key_heads=2, value_heads=4, key_dim=128, value_dim=128,
                        steps=2, max_position=512, block_size=8, padded_rows=1, seed=49)
    s = w.spec
    L, B, Q, HV, V = s.layers, s.rows, s.window, s.value_heads, s.value_dim
    acc = torch.full((B,), Q, dtype=torch.int32)
    acc[::4] = 2
    st = _first_step(w, dev, acc)
    plan, ctx, ckpts, recs, pending = st["plan"], st["ctx"], st["ckpts"], st["recs"], st["pending"]
    n, fin = plan["commit_lens"], plan["final"]
    active = [r for r in range(B) if int(n[r]) > 0]
    assert len(active) >= 2
    moved = active[1]
    pad = int(w.extras["padded_rows"][0])
    free_page = next(int(p) for p in w.meta.block_table[pad].tolist() if 0 < int(p) < w.num_pages)
    si = torch.where(n > 0, fin.to(torch.int32), w.meta.state_indices.to(torch.int32))
    si[moved] = free_page
    si_d = si.to(dev)
    wd = w.to(dev)
    qsl = wd.meta.query_start_loc
    outs = [torch.empty(1, w.tokens, HV, V, dtype=wd.inputs[0].v.dtype, device=dev) for _ in range(L)]
    print(f"deferred graph replay: row {moved} moves to page {free_page}", flush=True)

    def run():
        ctx.settle_deferred(si_d, pending[0].rows)
        for layer in range(L):
            gdn_recoverssm_verify_deferred(*_step_inputs(wd, layer, w.tokens), checkpoint_state=ckpts[layer],
                                           replay_cache=recs[1][layer], pending=pending[layer],
                                           query_start_loc=qsl, state_indices=si_d, spec_query_len=Q,
                                           out=outs[layer])

    pages0 = [c.clone() for c in ckpts]
    lens0 = ctx.commit_lens.clone()

    def reset():
        for c, c0 in zip(ckpts, pages0):
            c.copy_(c0)
        ctx.commit_lens.copy_(lens0)
        for t in outs + [x for r in recs[1] for x in (r.correction, r.key, r.decay)]:
            t.fill_(-7.0)

    def results():
        return ([c.clone() for c in ckpts] + [o.clone() for o in outs] +
                [x.clone() for r in recs[1] for x in (r.correction, r.key, r.decay)] + [ctx.commit_lens.clone()])

    reset()
    run()
    torch.cuda.synchronize()
    want = results()
    assert int(ctx.commit_lens[moved]) == 0 and int(lens0[moved]) > 0, "the settle marks the row it folds"
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()  # warm the launch path on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for rep in range(3):
        reset()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, ref) in enumerate(zip(results(), want)):
            assert torch.equal(got, ref), f"replay {rep}: result {i} differs from the eager launches"


def test_counted_row_list_folds_the_counted_rows(dev):
    """A fold with a device row count (gdn_fold_ext.row_count) folds the
    first `count` entries of its row list, clamped to the list: count 2 of a
    list of 3 folds two rows, a count past the list folds the whole list,
    count 0 nothing. Pages equal the oracle's fold of those rows; every other
    page is unchanged."""
    w = W.make_workload("decode_loop_l48", layers=2, rows=12, key_heads=2, value_heads=4, key_dim=128, value_dim=128,
                        steps=2, max_position=512, block_size=8, padded_rows=1, seed=45)
    s = w.spec
    L, B, Q = s.layers, s.rows, s.window
    acc = torch.full((B,), Q, dtype=torch.int32)
    acc[2::4] = 2
    st = _first_step(w, dev, acc)
    plan, ctx, ckpts = st["plan"], st["ctx"], st["ckpts"]
    n = plan["commit_lens"]
    active = [r for r in range(B) if int(n[r]) > 0]
    assert len(active) >= 7
    lists = torch.tensor([active[0], active[2], active[4], active[5], active[6]], dtype=torch.int32, device=dev)
    before = [x.cpu() for x in w.checkpoints]
    folded = []
    for entries, count in ((lists[:3], 2), (lists[3:5], 7), (lists[3:5], 0)):
        print(f"counted fold: rows {entries.tolist()}, count {count}", flush=True)
        cnt = torch.tensor([count], dtype=torch.int32, device=dev)
        _fold_rows_spec(ctx._deferred_fold, entries, cnt, listed=entries.numel()).launch()
        folded += entries.tolist()[:count]
    torch.cuda.synchronize()
    lengths = torch.zeros_like(n)
    lengths[folded] = n[folded]
    want = _oracle_fold(before, st["results"], plan, B, w.num_pages, lengths=lengths)
    touched = _touched(dict(plan, commit_lens=lengths), B, w.num_pages)
    for layer in range(L):
        _check_pages(ckpts[layer], want[layer], touched, f"layer {layer}: pages after the counted folds")


def test_rows_past_the_pending_plan_do_not_apply(dev):
    """The pending plan covers `num_rows` rows, and plan entries past them
    (here: the rest of a full plan, as an older, larger step leaves them)
    look valid. Rows of a larger next batch at or past `num_rows`, whose state
    index equals such an entry's final page, must verify from their own page
    and fold nothing; rows below it apply their commits. A row whose state
    index is not its pending commit's final page (a new request in a
    continued row) also verifies from its own page."""
    from dataclasses import replace

    w = W.make_workload("decode_loop_l48", layers=1, rows=10, key_heads=2, value_heads=4, key_dim=128, value_dim=64,
                        steps=2, max_position=512, block_size=8, padded_rows=0, seed=51)
    s = w.spec
    B, Q = s.rows, s.window
    acc = torch.full((B,), Q, dtype=torch.int32)
    st = _first_step(w, dev, acc)
    plan = st["plan"]
    n, fin = plan["commit_lens"], plan["final"]
    src = w.meta.state_indices
    B0 = 6
    short = tuple(replace(p, num_rows=B0) for p in st["pending"])
    idx1 = torch.where(n > 0, fin, src).to(torch.int32)
    # One row below B0 keeps its pending row but names its source page, which
    # differs from its commit's final page.
    moved = [r for r in range(B0) if int(n[r]) > 0 and int(fin[r]) != int(src[r])]
    assert moved and all(int(n[r]) > 0 for r in range(B0, B)), "the seed must move a row to a new page"
    taken = moved[0]
    idx1[taken] = int(src[taken])
    gen = torch.Generator().manual_seed(52)
    inp = W.make_layer_inputs(s, B * Q, gen)
    qsl = w.meta.query_start_loc
    ckpts, recs = st["ckpts"], st["recs"]
    out = gdn_recoverssm_verify_deferred(inp.g.to(dev), inp.beta.to(dev), inp.q.to(dev), inp.k.to(dev),
                                         inp.v.to(dev), checkpoint_state=ckpts[0], replay_cache=recs[1][0],
                                         pending=short[0], query_start_loc=qsl.to(dev), state_indices=idx1.to(dev),
                                         spec_query_len=Q)
    torch.cuda.synchronize()
    applied = torch.tensor([1 if (r < B0 and r != taken) else 0 for r in range(B)], dtype=torch.int32)
    want = _oracle_fold([w.checkpoints[0]], st["results"][:1], plan, B, w.num_pages,
                        lengths=plan["commit_lens"] * applied)
    pages = _touched({**plan, "commit_lens": plan["commit_lens"] * applied}, B, w.num_pages)
    _check_pages(ckpts[0], want[0], pages, "pages after a verify with a short pending plan")
    r1 = O.oracle_verify(inp.q, inp.k, inp.v, inp.g, inp.beta, want[0], qsl, idx1, Q)
    _check_verify(out, recs[1][0], r1, "step 1")

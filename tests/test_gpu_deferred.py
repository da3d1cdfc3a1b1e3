"""The deferred commit: the fold of step k applied inside step k+1's verify
(``gdn_recoverssm_verify_deferred``) must give bit-for-bit what the ordinary
flow gives (verify, then commit: plan + conv + fold), step after step: the
same outputs and records every step and the same pages once the last pending
fold is flushed. The ordinary flow itself is checked against the oracle in
test_gpu_verify / test_gpu_commit / test_gpu_loop.
"""

import pytest
import torch

from gdn_recoverssm_ascend import workloads as W
from gdn_recoverssm_ascend.kernels import (
    GDNRecoverSSMCommitContext,
    ReplayRecordBuffers,
    gdn_recoverssm_verify,
    gdn_recoverssm_verify_deferred,
)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(gpu_device):
    return gpu_device


def _flow(w, dev, acc_steps, qsl_steps, *, deferred):
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
        outs = []
        for layer in range(L):
            inp = wd.inputs[layer]
            T = int(qsl[-1])
            args = (inp.g[:T], inp.beta[:T], inp.q[:, :T], inp.k[:, :T], inp.v[:, :T])
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
        # Step 2 has no token for one row that still carries a pending commit:
        # the deferred verify must fold it anyway.
        lens = torch.full((s.rows,), s.window, dtype=torch.int32)
        lens[empty_row] = 0
        q2 = torch.zeros(s.rows + 1, dtype=torch.int32)
        q2[1:] = torch.cumsum(lens, 0)
        qsl_steps[2] = q2
    ref, ref_pages, ref_convs = _flow(w, dev, acc_steps, qsl_steps, deferred=False)
    got, got_pages, got_convs = _flow(w, dev, acc_steps, qsl_steps, deferred=True)
    for step, (a, b) in enumerate(zip(ref, got)):
        for name in ("out", "corr", "key", "decay", "plan"):
            for li, (x, y) in enumerate(zip(a[name], b[name])):
                assert torch.equal(x, y), f"step {step} {name} [{li}] differs"
        assert torch.equal(a["state_idx"], b["state_idx"])
    for li, (x, y) in enumerate(zip(ref_pages, got_pages)):
        assert torch.equal(x, y), f"layer {li}: pages differ after the flush"
    for li, (x, y) in enumerate(zip(ref_convs, got_convs)):
        assert torch.equal(x, y), f"layer {li}: conv states differ"
    # the comparison is not vacuous: commits happened and crossed boundaries
    assert sum(int((h["plan"][0] > 0).sum()) for h in ref) > 0
    assert sum(int((h["plan"][2] > 0).sum()) for h in ref) > 0


@pytest.mark.parametrize("K,V,Q,H,HV,act", [
    (64, 100, 3, 1, 4, torch.bfloat16),
    (256, 64, 8, 2, 2, torch.bfloat16),
    (32, 192, 1, 2, 8, torch.float16),
    (136, 48, 5, 3, 6, torch.float32),
    (96, 16, 6, 1, 1, torch.bfloat16),
])
def test_deferred_commit_equals_ordinary_flow_shapes(dev, K, V, Q, H, HV, act):
    """The same equality over head dims off the 128 x 128 tile (partial
    64-row half tiles, K padded to whole chunks), windows 1-8, GQA ratios 1-4
    and every activation dtype."""
    steps = 3
    w = W.make_workload("decode_loop_l48", layers=2, rows=6, key_heads=H, value_heads=HV, key_dim=K, value_dim=V,
                        window=Q, act_dtype=act, steps=steps, max_position=256, block_size=8, padded_rows=1,
                        seed=K + V + Q)
    s = w.spec
    print(f"deferred shapes: K={K} V={V} Q={Q} H={H} HV={HV} act={act}", flush=True)
    gen = torch.Generator().manual_seed(K * V + Q)
    acc_steps = [W.sample_accepted(s, s.rows, gen) for _ in range(steps)]
    qsl_steps = [w.meta.query_start_loc.clone() for _ in range(steps)]
    ref, ref_pages, ref_convs = _flow(w, dev, acc_steps, qsl_steps, deferred=False)
    got, got_pages, got_convs = _flow(w, dev, acc_steps, qsl_steps, deferred=True)
    for step, (a, b) in enumerate(zip(ref, got)):
        for name in ("out", "corr", "key", "decay", "plan"):
            for li, (x, y) in enumerate(zip(a[name], b[name])):
                assert torch.equal(x, y), f"step {step} {name} [{li}] differs"
    for li, (x, y) in enumerate(zip(ref_pages, got_pages)):
        assert torch.equal(x, y), f"layer {li}: pages differ after the flush"
    for li, (x, y) in enumerate(zip(ref_convs, got_convs)):
        assert torch.equal(x, y), f"layer {li}: conv states differ"
    assert sum(int((h["plan"][0] > 0).sum()) for h in ref) > 0


def test_deferred_commit_with_reordered_rows(dev):
    """The next step's batch lists the rows in another order: the pending
    commit's arrays are indexed by the next step's row and ``rows`` points at
    the record row the pending step wrote (row b of the new batch is old row
    perm[b]). Outputs, records and folded pages equal the ordinary flow's."""
    from gdn_recoverssm_ascend.kernels import PendingCommit

    w = W.make_workload("decode_loop_l48", layers=1, rows=8, key_heads=2, value_heads=4, steps=2, max_position=256,
                        block_size=8, padded_rows=1, seed=21)
    s = w.spec
    B, Q, H, HV, K, V = s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
    gen = torch.Generator().manual_seed(22)
    acc0 = W.sample_accepted(s, B, gen)
    perm = torch.randperm(B, generator=gen)
    wd = w.to(dev)
    inp, m = wd.inputs[0], wd.meta
    kw = dict(block_table=m.block_table, num_computed_tokens=m.num_computed, mamba_block_size=s.block_size)
    results = []
    for deferred in (False, True):
        ckpt, conv = wd.checkpoints[0].clone(), wd.conv_states[0].clone()
        recs = [ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=inp.k.dtype) for _ in range(2)]
        ctx = GDNRecoverSSMCommitContext.from_tensors([conv], [ckpt], [recs[0]], spec_query_len=Q, max_num_reqs=B)
        idx0 = m.state_indices.clone()
        args = (inp.g, inp.beta, inp.q, inp.k, inp.v)
        gdn_recoverssm_verify(*args, checkpoint_state=ckpt, replay_cache=recs[0], query_start_loc=m.query_start_loc,
                              state_indices=idx0, spec_query_len=Q)
        if deferred:
            pend = ctx.commit_deferred(acc0.to(dev), idx0, m.query_start_loc, **kw)[0]
        else:
            ctx.commit(acc0.to(dev), idx0, m.query_start_loc, **kw)
        lens = ctx.commit_lens[:B]
        idx1 = torch.where(lens > 0, ctx.final_state_indices[:B], idx0)[perm.to(dev)].contiguous()
        kw1 = dict(checkpoint_state=ckpt, replay_cache=recs[1], query_start_loc=m.query_start_loc,
                   state_indices=idx1, spec_query_len=Q)
        if deferred:
            p = perm.to(dev)
            moved = PendingCommit(pend.rows[p].contiguous(), pend.source[p].contiguous(), pend.lengths[p].contiguous(),
                                  pend.final[p].contiguous(), pend.boundary[p].contiguous(),
                                  pend.boundary_len[p].contiguous(), pend.records)
            out = gdn_recoverssm_verify_deferred(*args, pending=moved, **kw1)
        else:
            out = gdn_recoverssm_verify(*args, **kw1)
        torch.cuda.synchronize()
        results.append([out.clone(), recs[1].correction.clone(), recs[1].key.clone(), recs[1].decay.clone(),
                        ckpt.clone()])
        if not deferred:
            assert int((lens > 0).sum()) > 0 and not torch.equal(perm, torch.arange(B))
    for name, a, b in zip(("out", "correction", "key", "decay", "pages"), *results):
        assert torch.equal(a, b), f"{name} differs"

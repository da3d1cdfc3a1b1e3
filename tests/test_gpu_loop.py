"""Carried state across speculative steps: verify every layer, commit (plan,
conv compaction, fold) once per step, move each row to its final page and
advance its position, three steps in a row, all against the CPU oracle run
step by step on the same inputs.

Bar: plan arrays and page movement bit-exact every step; bf16 outputs within
1e-2 norm-wise every step; FP32 pages within max-abs 1e-5 (relative to the
pages' max-abs) after every commit; conv histories bit-exact.
"""

import pytest
import torch

import gdn_oracle as O
from gdn_recoverssm_ascend import workloads as W
from gdn_recoverssm_ascend.kernels import GDNRecoverSSMCommitContext, ReplayRecordBuffers, gdn_recoverssm_verify
from gpu_helpers import OUT_TOL, assert_norm_close, assert_state_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(gpu_device):
    return gpu_device


@pytest.mark.parametrize("block_size", [8, 16])
def test_three_steps_with_carried_state(dev, block_size):
    steps = 3
    w = W.make_workload("decode_loop_l48", layers=2, rows=10, key_heads=2, value_heads=4, key_dim=64, value_dim=64,
                        steps=steps, max_position=256, block_size=block_size, padded_rows=1, seed=5)
    s = w.spec
    L, B, Q, H, HV, K, V = s.layers, s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
    m = w.meta
    gen = torch.Generator().manual_seed(11)
    acc_steps = [W.sample_accepted(s, B, gen) for _ in range(steps)]

    # CPU oracle state
    ck_cpu = [c.clone() for c in w.checkpoints]
    cv_cpu = [c.clone() for c in w.conv_states]
    src_cpu = m.state_indices.clone()
    c_cpu = m.num_computed.clone()

    # GPU state
    wd = w.to(dev)
    recs = [ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=wd.inputs[0].k.dtype) for _ in range(L)]
    ctx = GDNRecoverSSMCommitContext.from_tensors(wd.conv_states, wd.checkpoints, recs, spec_query_len=Q,
                                                  max_num_reqs=B)
    state_idx = wd.meta.state_indices.clone()
    computed = wd.meta.num_computed.clone()
    hist = wd.conv_states[0].shape[2] - Q + 1

    for step in range(steps):
        acc = acc_steps[step]
        outs = []
        for layer in range(L):
            inp = wd.inputs[layer]
            outs.append(gdn_recoverssm_verify(inp.g, inp.beta, inp.q, inp.k, inp.v,
                                              checkpoint_state=wd.checkpoints[layer], replay_cache=recs[layer],
                                              query_start_loc=wd.meta.query_start_loc, state_indices=state_idx,
                                              spec_query_len=Q))
        ctx.commit(acc.to(dev), state_idx, wd.meta.query_start_loc, block_table=wd.meta.block_table,
                   num_computed_tokens=computed, mamba_block_size=block_size)
        torch.cuda.synchronize()

        # oracle step
        res = []
        for layer in range(L):
            ci = w.inputs[layer]
            r = O.oracle_verify(ci.q, ci.k, ci.v, ci.g, ci.beta, ck_cpu[layer], m.query_start_loc, src_cpu, Q)
            res.append(r)
            got = outs[layer].cpu()[0]
            wmask = r.out_written
            assert_norm_close(got[wmask].double(), r.out[wmask], OUT_TOL, f"step {step} layer {layer} out")
        plan = O.oracle_plan_single(acc, src_cpu, m.query_start_loc, spec_query_len=Q, num_blocks=w.num_pages,
                                    block_table=m.block_table, num_computed=c_cpu, block_size=block_size)
        for name, t in (("commit_lens", ctx.commit_lens), ("final", ctx.final_state_indices),
                        ("boundary", ctx.boundary_state_indices), ("boundary_len", ctx.boundary_recovery_lens)):
            assert t[:B].cpu().tolist() == plan[name].tolist(), f"step {step}: plan {name} differs"
        ck_cpu = O.oracle_fold(ck_cpu, [r.correction for r in res], [r.key for r in res], [r.decay for r in res],
                               source=src_cpu, lengths=plan["commit_lens"], final=plan["final"],
                               boundary=plan["boundary"], boundary_len=plan["boundary_len"], rows=B,
                               num_blocks=w.num_pages, record_rows=B, out_dtype=torch.float32)
        cv_cpu = O.oracle_conv_compact(cv_cpu, source=src_cpu, lengths=plan["commit_lens"], final=plan["final"],
                                       boundary=plan["boundary"], boundary_len=plan["boundary_len"], history=hist,
                                       num_blocks=w.num_pages, rows=B, align=True)
        for layer in range(L):
            assert_state_close(wd.checkpoints[layer].cpu(), ck_cpu[layer], f"step {step} layer {layer} pages")
            assert torch.equal(wd.conv_states[layer].cpu(), cv_cpu[layer]), f"step {step} layer {layer} conv"
            ck_cpu[layer] = wd.checkpoints[layer].cpu()  # continue both from the same pages

        # carry: committed rows move to their final page and advance by n
        n = plan["commit_lens"]
        committed = n > 0
        src_cpu = torch.where(committed, plan["final"], src_cpu).to(torch.int32)
        c_cpu = (c_cpu + n).to(c_cpu.dtype)
        lens = ctx.commit_lens[:B]
        state_idx.copy_(torch.where(lens > 0, ctx.final_state_indices[:B], state_idx))
        computed.add_(lens.to(computed.dtype))
        assert state_idx.cpu().tolist() == src_cpu.tolist()
        assert computed.cpu().tolist() == c_cpu.tolist()

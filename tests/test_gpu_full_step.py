"""One whole speculative step at the full sizes of the benchmark configurations
(B=64 from a 512-page pool, B=256 align mode with boundary crossings and
padded rows, B=256 plain decode at Q=1, B=256 at Q=8 with skewed acceptance)
and at two extremes (2048 rows of small heads; K=256, V=1024 at Q=8):
verify over every row, then the commit (plan + fold in one launch, conv
compaction), against the CPU oracle run over every row on the same inputs.

Bar: plan arrays and conv histories bit-exact; bf16 outputs within 1e-2
norm-wise; FP32 pages the commit targets within max-abs 1e-5 relative to the
pages' max-abs; every other page bit-identical.
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


EXTREMES = {
    # many rows with small heads: 2048 rows, 2 value heads of 32 x 32, Q=2
    "rows_2048": ("pool512_b64", dict(rows=2048, key_heads=1, value_heads=2, key_dim=32, value_dim=32, window=2,
                                      pool_pages=2100)),
    # the largest heads the kernels take: K=256, V=1024 (eight verify tiles), Q=8, align mode
    "k256_v1024_q8": ("align_b256", dict(rows=3, key_heads=1, value_heads=2, key_dim=256, value_dim=1024, window=8,
                                         padded_rows=0, crossing_fraction=1.0)),
}


@pytest.mark.parametrize("name", ["pool512_b64", "align_b256", "decode_q1_b256", "skewed_q8_b256", *EXTREMES])
def test_full_step_against_oracle(dev, name):
    base, over = EXTREMES.get(name, (name, {}))
    w = W.make_workload(base, gen_device=dev.type, **over)
    s = w.spec
    B, Q, H, HV, K, V = s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
    align = w.meta.block_table is not None
    print(f"full step {name}: B={B} Q={Q} pages={w.num_pages} align={align}", flush=True)
    # Host copies for the oracle, taken before the step changes the pages.
    cpu = lambda t: None if t is None else t.cpu()  # noqa: E731
    ck0 = w.checkpoints[0].cpu()
    conv0 = [c.cpu() for c in w.conv_states]
    ci = w.inputs[0]
    cq, ckk, cv, cg, cb = (t.cpu() for t in (ci.q, ci.k, ci.v, ci.g, ci.beta))
    m = w.meta
    qsl, idx, acc = cpu(m.query_start_loc), cpu(m.state_indices), cpu(m.accepted)
    table, computed = cpu(m.block_table), cpu(m.num_computed)

    wd = w.to(dev)
    inp = wd.inputs[0]
    rec = ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=inp.k.dtype)
    ctx = GDNRecoverSSMCommitContext.from_tensors(wd.conv_states, wd.checkpoints, [rec], spec_query_len=Q,
                                                  max_num_reqs=B)
    out = gdn_recoverssm_verify(inp.g, inp.beta, inp.q, inp.k, inp.v, checkpoint_state=wd.checkpoints[0],
                                replay_cache=rec, query_start_loc=wd.meta.query_start_loc,
                                state_indices=wd.meta.state_indices, spec_query_len=Q)
    ctx.commit(wd.meta.accepted, wd.meta.state_indices, wd.meta.query_start_loc,
               block_table=wd.meta.block_table if align else None,
               num_computed_tokens=wd.meta.num_computed if align else None,
               mamba_block_size=m.block_size if align else None)
    torch.cuda.synchronize()
    assert [sp.name for sp in ctx._last_specs] == ["plan_fold", "conv"]

    res = O.oracle_verify(cq, ckk, cv, cg, cb, ck0, qsl, idx, Q)
    got_out = out.cpu()[0]
    wm = res.out_written
    assert_norm_close(got_out[wm].double(), res.out[wm], OUT_TOL, f"{name} out")

    plan = O.oracle_plan_single(acc, idx, qsl, spec_query_len=Q, num_blocks=w.num_pages, block_table=table,
                                num_computed=computed, block_size=m.block_size if align else None)
    for key, t in (("commit_lens", ctx.commit_lens), ("final", ctx.final_state_indices),
                   ("boundary", ctx.boundary_state_indices), ("boundary_len", ctx.boundary_recovery_lens)):
        assert t[:B].cpu().tolist() == plan[key].tolist(), f"{name}: plan {key} differs"
    n = plan["commit_lens"]
    assert int((n > 0).sum()) > 0
    if align:
        assert int(plan["boundary_len"].gt(0).sum()) > 0, "align mode must exercise boundary snapshots"

    want = O.oracle_fold([ck0], [res.correction], [res.key], [res.decay], source=idx,
                         lengths=n, final=plan["final"], boundary=plan["boundary"],
                         boundary_len=plan["boundary_len"], rows=B, num_blocks=w.num_pages, record_rows=B,
                         out_dtype=torch.float32)[0]
    got = wd.checkpoints[0].cpu()
    targeted = sorted({int(p) for p in plan["final"][n > 0]} | {int(p) for p in plan["boundary"][n > 0] if int(p) > 0})
    untouched = torch.ones(got.shape[0], dtype=torch.bool)
    untouched[targeted] = False
    assert torch.equal(got[untouched], ck0[untouched]), f"{name}: pages outside the commit changed"
    assert_state_close(got[targeted], want[targeted], f"{name} committed pages")

    hist = conv0[0].shape[2] - Q + 1
    want_conv = O.oracle_conv_compact(conv0, source=idx, lengths=n, final=plan["final"],
                                      boundary=plan["boundary"], boundary_len=plan["boundary_len"], history=hist,
                                      num_blocks=w.num_pages, rows=B, align=align)
    assert torch.equal(wd.conv_states[0].cpu(), want_conv[0]), f"{name}: conv states differ"

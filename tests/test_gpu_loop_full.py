"""The decode loop at its full size: 48 GDN layers (H=16, HV=32, K=V=128),
B=128 rows, Q=4, align mode (block size 64), 64 carried speculative steps
with fresh accepted lengths each step: every layer's verify, then one commit
(plan + fold in one launch, then the conv compaction) across all layers.

Checked every step of the ordinary flow (verify, then commit):
* the plan arrays against ``oracle_plan_single`` for all rows, bit for bit;
* for a seeded subset of (layer, row) pairs, the row's outputs and records
  against ``oracle_verify`` from the row's pre-step page, and its final (and
  boundary) page against ``oracle_fold`` of those records;
* every page outside the step's commit bit-identical, by a per-page digest
  (the int64 sum of the page's 32-bit words, which any change of a single
  word alters).
The deferred flow (each step's fold applied by the next step's verify, the
last one flushed) runs the same 64 steps from the same seeded start and must
give bit-identical outputs, plans and final pages (digests of each).

Bar: plan indexing bit-exact; outputs within 1e-2 norm-wise; corrections
within 1e-5 norm-wise; keys bit-exact; FP32 pages within max-abs 1e-5
relative to the pages' max-abs.
"""

import pytest
import torch

import gdn_oracle as O
from gdn_recoverssm_ascend import workloads as W
from gdn_recoverssm_ascend.kernels import (
    GDNRecoverSSMCommitContext,
    ReplayRecordBuffers,
    gdn_recoverssm_verify,
    gdn_recoverssm_verify_deferred,
)
from gpu_helpers import CORR_TOL, OUT_TOL, assert_norm_close, assert_state_close

pytestmark = pytest.mark.gpu

SEED = 0
ACCEPT_SEED = 7
PAIRS_PER_STEP = (2, 3)  # layers x rows checked against the oracle each step


@pytest.fixture(scope="module")
def dev(gpu_device):
    return gpu_device


def _digest(pages: torch.Tensor) -> torch.Tensor:
    """Per-page int64 sum of the page's 32-bit words (on the device)."""
    return pages.view(pages.shape[0], -1).view(torch.int32).sum(dim=1, dtype=torch.int64)


def _check_pair(w, outs, recs, layer, row, src_tile, qsl, src, plan, ckpt_after, step):
    """Outputs, records and committed pages of one (layer, row) against the
    oracle run on that row alone from its pre-step page."""
    s = w.spec
    Q = s.window
    b0, b1 = int(qsl[row]), int(qsl[row + 1])
    inp = w.inputs[layer]
    sl = slice(b0, b1)
    q, k, v = inp.q[:, sl].cpu(), inp.k[:, sl].cpu(), inp.v[:, sl].cpu()
    g, beta = inp.g[sl].cpu(), inp.beta[sl].cpu()
    n, fin, bnd, blen = (int(plan[x][row]) for x in ("commit_lens", "final", "boundary", "boundary_len"))
    page = int(src[row])
    pool = torch.zeros((2,) + tuple(src_tile.shape), dtype=src_tile.dtype)
    pool[1] = src_tile
    r = O.oracle_verify(q, k, v, g, beta, pool, torch.tensor([0, b1 - b0]), torch.tensor([1]), Q)
    what = f"step {step} layer {layer} row {row}"
    got = outs[layer][0, sl].cpu()
    assert_norm_close(got.double(), r.out, OUT_TOL, f"{what} out")
    rw = r.record_written[0]
    rec = recs[layer]
    for t in range(Q):
        if not bool(rw[t]):
            continue
        assert_norm_close(rec.correction[row, :, t].cpu().double(), r.correction[0, :, t], CORR_TOL,
                          f"{what} correction {t}")
        assert torch.equal(rec.key[row, :, t].cpu().float(), r.key[0, :, t].float()), f"{what} key {t}"
    if n == 0:
        return 0
    # The fold of this row in a pool of its own pages: source, final, boundary.
    crossing = 0 < bnd < w.num_pages and bnd != fin and 0 < blen <= n
    ids = [page, fin] + ([bnd] if crossing else [])
    mini = torch.zeros((len(set(ids)) + 1,) + tuple(src_tile.shape), dtype=src_tile.dtype)
    index = {p: i + 1 for i, p in enumerate(dict.fromkeys(ids))}
    mini[index[page]] = src_tile
    want = O.oracle_fold([mini], [r.correction], [r.key], [r.decay], source=torch.tensor([index[page]]),
                         lengths=torch.tensor([n]), final=torch.tensor([index[fin]]),
                         boundary=torch.tensor([index[bnd] if crossing else 0]), boundary_len=torch.tensor([blen]),
                         rows=1, num_blocks=mini.shape[0], record_rows=1, out_dtype=torch.float32)[0]
    assert_state_close(ckpt_after[fin].cpu(), want[index[fin]], f"{what} final page")
    if crossing:
        assert_state_close(ckpt_after[bnd].cpu(), want[index[bnd]], f"{what} boundary page")
    return 1


def _run(dev, *, deferred, check):
    w = W.make_workload("decode_loop_l48", seed=SEED, gen_device="cuda")
    s = w.spec
    L, B, Q, H, HV, K, V = s.layers, s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
    assert (L, B, Q, H, HV, K, V, s.block_size, s.steps) == (48, 128, 4, 16, 32, 128, 128, 64, 64)
    wd = w.to(dev)
    ckpts, convs = wd.checkpoints, wd.conv_states
    sets = 2 if deferred else 1
    recs = [[ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=wd.inputs[0].k.dtype)
             for _ in range(L)] for _ in range(sets)]
    ctxs = [GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs[i], spec_query_len=Q, max_num_reqs=B)
            for i in range(sets)]
    m = wd.meta
    state_idx = m.state_indices.clone()
    computed = m.num_computed.clone()
    src_cpu = w.meta.state_indices.clone()
    c_cpu = w.meta.num_computed.clone()
    qsl_cpu = w.meta.query_start_loc
    outs = [torch.empty(1, w.tokens, HV, V, dtype=wd.inputs[0].v.dtype, device=dev) for _ in range(L)]
    gen = torch.Generator().manual_seed(ACCEPT_SEED)
    pick = torch.Generator().manual_seed(ACCEPT_SEED + 1)
    valid_rows = [r for r in range(B) if int(src_cpu[r]) > 0]
    out_digests, plan_rows, checked = [], [], 0
    pending = None
    before = [_digest(c) for c in ckpts] if check else None
    for step in range(s.steps):
        acc = W.sample_accepted(s, B, gen)
        i = step % sets
        pairs = []
        if check:
            layers = torch.randperm(L, generator=pick)[:PAIRS_PER_STEP[0]].tolist()
            rows = [valid_rows[j] for j in torch.randperm(len(valid_rows), generator=pick)[:PAIRS_PER_STEP[1]]]
            pairs = [(la, r, ckpts[la][int(src_cpu[r])].cpu()) for la in layers for r in rows]
        for layer in range(L):
            inp = wd.inputs[layer]
            kw = dict(checkpoint_state=ckpts[layer], replay_cache=recs[i][layer], query_start_loc=m.query_start_loc,
                      state_indices=state_idx, spec_query_len=Q, out=outs[layer])
            if pending is None:
                gdn_recoverssm_verify(inp.g, inp.beta, inp.q, inp.k, inp.v, **kw)
            else:
                gdn_recoverssm_verify_deferred(inp.g, inp.beta, inp.q, inp.k, inp.v, pending=pending[layer], **kw)
        commit_kw = dict(block_table=m.block_table, num_computed_tokens=computed, mamba_block_size=m.block_size)
        if deferred:
            pending = ctxs[i].commit_deferred(acc.to(dev), state_idx, m.query_start_loc, **commit_kw)
        else:
            ctxs[i].commit(acc.to(dev), state_idx, m.query_start_loc, **commit_kw)
        ctx = ctxs[i]
        plan_dev = [t[:B].clone() for t in (ctx.commit_lens, ctx.final_state_indices, ctx.boundary_state_indices,
                                            ctx.boundary_recovery_lens)]
        torch.cuda.synchronize()
        out_digests.append(torch.stack([_digest(o[0]).sum() for o in outs]).cpu())
        plan_rows.append(torch.stack(plan_dev).cpu())
        if check:
            plan = O.oracle_plan_single(acc, src_cpu, qsl_cpu, spec_query_len=Q, num_blocks=w.num_pages,
                                        block_table=w.meta.block_table, num_computed=c_cpu, block_size=s.block_size)
            for j, name in enumerate(("commit_lens", "final", "boundary", "boundary_len")):
                assert plan_rows[-1][j].tolist() == plan[name].tolist(), f"step {step}: plan {name} differs"
            touched = set()
            for r in range(B):
                if int(plan["commit_lens"][r]) > 0:
                    touched.add(int(plan["final"][r]))
                    bnd = int(plan["boundary"][r])
                    if 0 < bnd < w.num_pages and bnd != int(plan["final"][r]) and int(plan["boundary_len"][r]) > 0:
                        touched.add(bnd)
            keep = torch.ones(w.num_pages, dtype=torch.bool)
            keep[list(touched)] = False
            after = [_digest(c) for c in ckpts]
            for layer in range(L):
                assert torch.equal(after[layer].cpu()[keep], before[layer].cpu()[keep]), \
                    f"step {step} layer {layer}: pages outside the commit changed"
            before = after
            for la, r, tile in pairs:
                checked += _check_pair(w, outs, recs[i], la, r, tile, qsl_cpu, src_cpu, plan, ckpts[la], step)
            n = plan["commit_lens"]
            src_cpu = torch.where(n > 0, plan["final"], src_cpu).to(torch.int32)
            c_cpu = (c_cpu + n).to(c_cpu.dtype)
        lens = ctx.commit_lens[:B]
        state_idx.copy_(torch.where(lens > 0, ctx.final_state_indices[:B], state_idx))
        computed.add_(lens.to(computed.dtype))
        if step % 8 == 7:
            print(f"decode loop {'deferred' if deferred else 'ordinary'}: step {step + 1}/{s.steps}", flush=True)
    if deferred:
        ctxs[(s.steps - 1) % sets].flush_deferred()
    torch.cuda.synchronize()
    final_pages = torch.stack([_digest(c) for c in ckpts]).cpu()
    conv = torch.stack([_digest(c) for c in convs]).cpu()
    del w, wd, ckpts, convs, recs, ctxs, outs, pending
    torch.cuda.empty_cache()
    return dict(out=out_digests, plan=plan_rows, pages=final_pages, conv=conv, checked=checked)


def test_decode_loop_l48_full_size(dev):
    ref = _run(dev, deferred=False, check=True)
    assert ref["checked"] > 32, "too few committed (layer, row) pairs were checked against the oracle"
    got = _run(dev, deferred=True, check=False)
    for step, (a, b) in enumerate(zip(ref["plan"], got["plan"])):
        assert torch.equal(a, b), f"step {step}: deferred plan differs"
    for step, (a, b) in enumerate(zip(ref["out"], got["out"])):
        assert torch.equal(a, b), f"step {step}: deferred outputs differ"
    assert torch.equal(ref["pages"], got["pages"]), "deferred pages differ after the flush"
    assert torch.equal(ref["conv"], got["conv"]), "deferred conv states differ"

"""The torch operators ``torch.ops.gdn_recoverssm_hip.verify`` / ``fold``
(the reference's native op ABI, csrc/ops.cpp:243-257) against the Python API
on the same inputs: called with the 28-field verify config and the 17-field
fold config that the API builds, they must produce bit-identical outputs,
records and pages (they launch the same kernels through the C ABI)."""

import pytest
import torch

import sweep_cases as SC
from gdn_recoverssm_ascend import torch_ops  # noqa: F401  (registers the operators)
from gdn_recoverssm_ascend import workloads as W
from gdn_recoverssm_ascend.kernels import GDNRecoverSSMCommitContext, ReplayRecordBuffers, gdn_recoverssm_verify

pytestmark = pytest.mark.gpu
OPS = torch.ops.gdn_recoverssm_hip


@pytest.fixture(scope="module")
def dev(gpu_device):
    return gpu_device


def _workload(dev, **kw):
    spec = dict(rows=12, key_heads=2, value_heads=4, padded_rows=1, seed=3)
    spec.update(kw)
    return W.make_workload("align_b256", **spec).to(dev)


def test_verify_operator_equals_api(dev, **kw):
    w = _workload(dev, **kw)
    s, m, inp = w.spec, w.meta, w.inputs[0]
    B, Q, H, HV, K, V = s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
    runs = []
    for via_op in (False, True):
        rec = ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=inp.k.dtype)
        out = torch.full((1, w.tokens, HV, V), -7.0, dtype=inp.v.dtype, device=dev)
        specs = []
        gdn_recoverssm_verify(inp.g, inp.beta, inp.q, inp.k, inp.v, checkpoint_state=w.checkpoints[0],
                              replay_cache=rec, query_start_loc=m.query_start_loc, state_indices=m.state_indices,
                              spec_query_len=Q, out=out, _collect=specs)
        spec = specs[0]
        if via_op:
            OPS.verify(inp.q, inp.k, inp.v, inp.g, inp.beta, w.checkpoints[0], rec.correction, rec.key, rec.decay,
                       out, m.query_start_loc, m.state_indices, list(spec.config), spec.scale)
        else:
            spec.launch()
        torch.cuda.synchronize()
        runs.append([t.clone() for t in (out, rec.correction, rec.key, rec.decay)])
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    assert bool((runs[0][0] != -7.0).any())


def test_fold_operator_equals_api(dev, _any_commit=True, **kw):
    w = _workload(dev, **kw)
    s, m = w.spec, w.meta
    B, Q, H, HV, K, V = s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
    gen = torch.Generator(device=dev).manual_seed(5)
    rec = ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=torch.bfloat16)
    rec.correction.copy_(torch.randn(rec.correction.shape, generator=gen, device=dev))
    rec.key.copy_(torch.randn(rec.key.shape, generator=gen, device=dev).to(torch.bfloat16))
    rec.decay.copy_(torch.rand(rec.decay.shape, generator=gen, device=dev) * 0.5 + 0.5)
    ctx = GDNRecoverSSMCommitContext.from_tensors(w.conv_states, w.checkpoints, [rec], spec_query_len=Q,
                                                  max_num_reqs=B)
    specs = []
    ctx.commit(m.accepted, m.state_indices, m.query_start_loc, block_table=m.block_table,
               num_computed_tokens=m.num_computed, mamba_block_size=m.block_size, commit_conv=False,
               _collect=specs, _fold_source=m.state_indices)
    plan, fold = specs[0], specs[-1]
    assert [sp.name for sp in specs] == ["plan", "fold"]
    plan.launch()
    pages0 = w.checkpoints[0].clone()
    OPS.fold(w.checkpoints[0], rec.correction, rec.key, rec.decay, ctx.state_base_addrs, ctx.state_block_strides,
             ctx.correction_base_addrs, ctx.correction_block_strides, ctx.key_base_addrs, ctx.key_block_strides,
             ctx.decay_base_addrs, ctx.decay_block_strides, torch.empty(0, dtype=torch.int32, device=dev),
             m.state_indices, ctx.commit_lens, ctx.final_state_indices, ctx.boundary_state_indices,
             ctx.boundary_recovery_lens, list(fold.config))
    torch.cuda.synchronize()
    via_op = w.checkpoints[0].clone()
    w.checkpoints[0].copy_(pages0)
    fold.launch()
    torch.cuda.synchronize()
    assert torch.equal(via_op, w.checkpoints[0])
    if _any_commit:
        assert not torch.equal(via_op, pages0)  # the step committed something


def _random_shape(case):
    c = SC.deferred_case(case)
    print(f"operator sweep case {case}: {c}", flush=True)
    return dict(rows=c["rows"], key_heads=c["H"], value_heads=c["HV"], key_dim=c["K"], value_dim=c["V"],
                window=c["Q"], act_dtype=c["act"], state_dtype=c["state"], block_size=max(c["block_size"], c["Q"]),
                seed=c["seed"])


@pytest.mark.parametrize("case", range(SC.DEFERRED_CASES))
def test_random_operators_equal_api(dev, case):
    """Both operators over seeded random shapes (head dims, GQA ratio, window,
    activation and state dtypes, rows, block size): bit-identical to the API's
    own launches."""
    shape = _random_shape(case)
    test_verify_operator_equals_api(dev, **shape)
    test_fold_operator_equals_api(dev, _any_commit=False, **shape)  # a small batch may accept nothing

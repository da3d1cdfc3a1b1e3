"""Compile-only preparation (the reference's startup path, kernels.py:1741-1822
and grouped_commit.py:955-1016): every signature the serving step will use is
built and checked against the loaded library without a single launch, and
the prepared grouped bucket is adopted by the first real commit.
"""

from types import SimpleNamespace

import pytest
import torch

from gdn_recoverssm_ascend import kernels as Kmod
from gdn_recoverssm_ascend.grouped_commit import GroupedCommitCoordinator, prepare_grouped_commit
from gdn_recoverssm_ascend.kernels import GDNRecoverSSMCommitContext, ReplayRecordBuffers

pytestmark = pytest.mark.gpu

LAUNCHES = ("verify", "plan", "conv", "fold", "plan_fold", "publish")


@pytest.fixture(scope="module")
def dev(gpu_device):
    return gpu_device


def _launches():
    c = Kmod.counts()
    return {k: c.get(k, 0) for k in LAUNCHES}


def _context(dev, rows=4, HV=4, H=2, Q=4, K=128, V=128, NB=12, dtype=torch.bfloat16):
    convs = [torch.zeros(NB, 16, 3 + Q - 1, dtype=dtype, device=dev) for _ in range(2)]
    ckpts = [torch.randn(NB, HV, V, K, device=dev) for _ in range(2)]
    recs = [ReplayRecordBuffers.allocate(rows, HV, H, Q, V, K, device=dev, key_dtype=dtype) for _ in range(2)]
    return GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=Q, max_num_reqs=rows)


@pytest.mark.parametrize("align", [False, True])
def test_prepare_compiles_every_row_count_without_launching(dev, align):
    ctx = _context(dev)
    pages = [c.clone() for c in ctx.checkpoints]
    before = _launches()
    rows = ctx.prepare(capacity=8, state_table_width=4, request_mapping=True, device=dev, align_mode=align,
                       mamba_block_size=8 if align else None)
    torch.cuda.synchronize()
    assert rows == [1, 2, 3, 4]  # bounded by the record rows, not the capacity
    assert _launches() == before
    assert Kmod.counts().get("prepared_plan_fold", 0) > 0 and Kmod.counts().get("prepared_conv", 0) > 0
    assert all(torch.equal(a, b) for a, b in zip(pages, ctx.checkpoints))


def test_prepare_verify_covers_value_layouts_and_beta_dtypes(dev):
    ctx = _context(dev)
    before = _launches()
    report = ctx.prepare_verify(activation_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert _launches() == before
    # contiguous and combined-QKV value views, FP32 and activation-typed beta
    assert len(report) == 4
    assert {r["value_token_stride"] for r in report} == {4 * 128, 2 * 2 * 128 + 4 * 128}
    assert {r["beta_dtype"] for r in report} == {str(torch.float32), str(torch.bfloat16)}


def _builder(ctx, mode="none", block_size=8):
    return SimpleNamespace(
        _get_context=lambda: ctx,
        vllm_config=SimpleNamespace(cache_config=SimpleNamespace(mamba_cache_mode=mode)),
        kv_cache_spec=SimpleNamespace(block_size=block_size),
    )


def test_prepare_grouped_commit_is_adopted_by_the_coordinator(dev):
    contexts = [_context(dev) for _ in range(4)]
    builders = [_builder(c) for c in contexts]
    before = _launches()
    n = prepare_grouped_commit(builders)
    torch.cuda.synchronize()
    assert _launches() == before
    # buckets of three and one context, each prepared as (plan + fold, conv)
    assert n == 2 * 2
    assert builders[0]._prepared_group_bucket is builders[2]._prepared_group_bucket
    assert builders[3]._prepared_group_bucket is not builders[0]._prepared_group_bucket

    # the first real commit of the same groups uses the prepared buckets
    rows = 4
    metas = []
    for b, c in zip(builders, contexts):
        payload = SimpleNamespace(
            state_indices=torch.tensor([1, 2, 3, 4], dtype=torch.int32, device=dev),
            query_start_loc=torch.arange(rows + 1, dtype=torch.int32, device=dev) * 4,
            request_indices=torch.arange(rows, dtype=torch.int64, device=dev),
            block_table=None, num_computed_tokens=None, block_size=None,
            request_rows=tuple(range(rows)), query_lens=(4,) * rows,
        )
        metas.append(SimpleNamespace(recoverssm_commit=payload, recoverssm_builder=b, recoverssm_context=c))
    coord = GroupedCommitCoordinator()
    sampled = torch.zeros(rows, dtype=torch.int32, device=dev)  # nothing accepted: pages stay as they are
    pages = [p.clone() for c in contexts for p in c.checkpoints]
    coord.commit(metas, sampled, torch.arange(rows, dtype=torch.int32, device=dev),
                 torch.zeros(rows, dtype=torch.int32, device=dev), torch.zeros(rows, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    assert set(map(id, coord._buckets.values())) == {id(builders[0]._prepared_group_bucket),
                                                    id(builders[3]._prepared_group_bucket)}
    assert coord.last_launch_count == 4
    assert all(torch.equal(a, b) for a, b in zip(pages, [p for c in contexts for p in c.checkpoints]))

"""Compile-only preparation (the reference's startup path, kernels.py:1741-1822
and grouped_commit.py:955-1016): every signature the serving step will use is
built and checked against the loaded library without a single launch, and
the prepared grouped bucket is adopted by the first real commit.
"""

import json
import os
from types import SimpleNamespace

import pytest
import torch

from gdn_recoverssm_ascend import kernels as Kmod
from gdn_recoverssm_ascend.grouped_commit import (
    CommitEntry,
    GroupedCommitBucket,
    GroupedCommitCoordinator,
    prepare_grouped_commit,
)
from gdn_recoverssm_ascend.kernels import GDNRecoverSSMCommitContext, ReplayRecordBuffers, gdn_recoverssm_verify

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_known_answers.json")

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


def test_native_config_prefixes_match_reference(dev):
    """The verify and fold configs the host layer builds for the launch setups
    of the reference's backend tests (tests/test_ascendc_backend.py:38-77 and
    :118-168): field prefixes, the column-view index stride and the default
    scale, built without a launch."""
    gold = json.load(open(GOLDEN))["native_config_prefixes"]
    bf = torch.bfloat16
    q = torch.zeros((1, 8, 1, 128), dtype=bf, device=dev)
    value = torch.zeros((1, 8, 3, 128), dtype=bf, device=dev)
    record = ReplayRecordBuffers.allocate(2, 3, 1, 4, 128, 128, device=dev, key_dtype=bf)
    specs = []
    before = _launches()
    gdn_recoverssm_verify(torch.zeros((1, 8, 3), device=dev), torch.zeros((1, 8, 3), device=dev), q, q.clone(), value,
                          checkpoint_state=torch.zeros((4, 3, 128, 128), device=dev), replay_cache=record,
                          query_start_loc=torch.tensor([0, 4, 8], dtype=torch.int32, device=dev),
                          state_indices=torch.ones((2, 4), dtype=torch.int32, device=dev)[:, 0], spec_query_len=4,
                          _collect=specs)
    cfg = specs[0].config
    assert len(cfg) == 28
    assert list(cfg[:8]) == gold["verify_prefix"]
    assert cfg[-1] == gold["verify_index_stride_column_view"]
    assert specs[0].scale == pytest.approx(128 ** -0.5)

    contexts = []
    for _ in range(2):
        rec = ReplayRecordBuffers.allocate(2, 3, 1, 4, 128, 128, device=dev, key_dtype=bf)
        contexts.append(GDNRecoverSSMCommitContext.from_tensors(
            [torch.zeros((4, 8, 6), device=dev)], [torch.zeros((4, 3, 128, 128), device=dev)], [rec],
            spec_query_len=4, max_num_reqs=2))
    entries = []
    for ctx in contexts:
        p = SimpleNamespace(
            state_indices=torch.tensor([1, 2], dtype=torch.int32, device=dev),
            query_start_loc=torch.tensor([0, 4, 8], dtype=torch.int32, device=dev),
            request_indices=torch.tensor([0, 1], dtype=torch.int64, device=dev),
            block_table=None, num_computed_tokens=None, block_size=None, request_rows=(0, 1), query_lens=(4, 4),
        )
        entries.append(CommitEntry(None, p, ctx))
    bucket = GroupedCommitBucket(tuple(contexts))
    persistent = torch.zeros(2, dtype=torch.int32, device=dev)
    fold = bucket.make_specs(entries, torch.ones(2, dtype=torch.int32, device=dev), persistent.clone(),
                             persistent.clone(), persistent.clone(), fuse_plan_fold=False)[-1]
    assert fold.name == "fold" and len(fold.config) == 17
    assert list(fold.config[:9]) == gold["fold_prefix"]
    assert _launches() == before

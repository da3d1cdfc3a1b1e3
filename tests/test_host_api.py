"""Host side of the Python API, on the CPU (no launch): record geometry and
byte counts, and the argument checks that raise ValueError before anything is
submitted (the reference's error contract, kernels.py:143-151; record
geometry kernels.py:166-294; grouped checks grouped_commit.py:483-610 and
:925-942).

Known answers: 193.125 / 169.125 MiB of records for 128 rows x 48 layers,
HV=12, H=4, Q=4, K=V=128 with FP32 / BF16 keys
(tests/test_record_buffers.py:112-129 of the reference), and the geometry /
dtype rejections of its :153-160.
"""

from types import SimpleNamespace

import pytest
import torch

import sweep_cases as SC

from gdn_recoverssm_ascend import kernels as Kmod
from gdn_recoverssm_ascend.grouped_commit import CommitEntry, GroupedCommitBucket, GroupedCommitCoordinator
from gdn_recoverssm_ascend.kernels import (
    GDNRecoverSSMCommitContext,
    ReplayRecordBuffers,
    gdn_recoverssm_verify,
    record_geometry_bytes,
    record_nbytes,
)


def test_record_geometry_known_answers():
    kw = dict(rows=128, num_layers=48, num_value_heads=12, num_key_heads=4, window=4, key_dim=128, value_dim=128)
    assert record_geometry_bytes(**kw, key_dtype=torch.float32) == 193.125 * 1024**2
    assert record_geometry_bytes(**kw, key_dtype=torch.bfloat16) == 169.125 * 1024**2
    # the closed form, term by term: corrections, keys (one per key head), decays
    r, L, HV, H, Q, K, V = 3, 2, 6, 2, 4, 8, 8
    assert record_geometry_bytes(r, L, HV, H, Q, K, V, torch.float16) == r * L * Q * (HV * V * 4 + H * K * 2 + HV * 4)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_record_planes_and_key_roundtrip(dtype):
    rec = ReplayRecordBuffers.allocate(2, 6, 2, 4, 8, 8, device="cpu", key_dtype=dtype)
    assert tuple(rec.correction.shape) == (2, 6, 4, 8) and rec.correction.dtype == torch.float32
    assert tuple(rec.key.shape) == (2, 2, 4, 8) and rec.key.dtype == dtype  # shared by three value heads
    assert tuple(rec.decay.shape) == (2, 6, 4) and rec.decay.dtype == torch.float32
    assert tuple(rec.shape) == (2, 6, 4, 8 + 8 + 1)
    assert record_nbytes(rec) == record_geometry_bytes(2, 1, 6, 2, 4, 8, 8, dtype)
    values = torch.randn(rec.key.shape, generator=torch.Generator().manual_seed(231)).to(dtype)
    rec.key.copy_(values)
    assert torch.equal(rec.key.float(), values.float())


def test_record_geometry_and_dtype_rejected():
    with pytest.raises(ValueError, match="geometry"):
        ReplayRecordBuffers.allocate(2, 6, 4, 4, 8, 8, device="cpu")  # 6 value heads over 4 key heads
    with pytest.raises(ValueError, match="geometry"):
        ReplayRecordBuffers.allocate(2, 6, 2, 9, 8, 8, device="cpu")  # window above 8
    with pytest.raises(ValueError, match="FP16, BF16 or FP32"):
        ReplayRecordBuffers.allocate(2, 6, 2, 4, 8, 8, device="cpu", key_dtype=torch.float64)


def _verify_inputs(dtype=torch.bfloat16):
    B, Q, H, HV, K, V, NB = 2, 4, 2, 6, 8, 8, 4
    return dict(
        g=torch.zeros(B * Q, HV),
        beta=torch.ones(B * Q, HV),
        q=torch.zeros(1, B * Q, H, K, dtype=dtype),
        k=torch.zeros(1, B * Q, H, K, dtype=dtype),
        v=torch.zeros(1, B * Q, HV, V, dtype=dtype),
        checkpoint_state=torch.zeros(NB, HV, V, K),
        replay_cache=ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device="cpu", key_dtype=dtype),
        query_start_loc=torch.tensor([0, 4, 8], dtype=torch.int32),
        state_indices=torch.tensor([1, 2], dtype=torch.int32),
        spec_query_len=Q,
    )


@pytest.mark.parametrize(
    "change,match",
    [
        (lambda d: d.update(k=d["k"][:, :, :1]), "q and k shapes differ"),
        (lambda d: d.update(spec_query_len=0), "spec_query_len"),
        (lambda d: d.update(spec_query_len=9), "spec_query_len"),
        (lambda d: d.update(checkpoint_state=torch.zeros(4, 6, 8, 16)), "checkpoint shape"),
        (lambda d: d.update(g=torch.zeros(8, 5)), "gate or beta shape"),
        (lambda d: d.update(v=d["v"].float()), "share one activation dtype"),
        (lambda d: d.update(q=torch.zeros(1, 8, 4, 8, dtype=torch.bfloat16),
                            k=torch.zeros(1, 8, 4, 8, dtype=torch.bfloat16)), "multiple of the q/k heads"),
        (lambda d: d.update(state_indices=torch.tensor([[1, 2]], dtype=torch.int32)), "one-dimensional"),
        (lambda d: d.update(query_start_loc=torch.tensor([0, 4, 8, 12], dtype=torch.int32),
                            state_indices=torch.tensor([1], dtype=torch.int32)), "query metadata is incompatible"),
        # lossy key records (tests/test_record_buffers.py:193-222 of the reference)
        (lambda d: d.update(qk_already_normalized=False), "already-normalized"),
        (lambda d: d.update(q=d["q"].half(), k=d["k"].half(), v=d["v"].half()), "already-normalized"),
        (lambda d: None, "HIP device"),  # well-formed, but there is no CPU path
    ],
)
def test_verify_rejects_before_any_launch(change, match):
    d = _verify_inputs()
    change(d)
    before = dict(Kmod.counts())
    with pytest.raises(ValueError, match=match):
        gdn_recoverssm_verify(**d)
    assert dict(Kmod.counts()) == before


def _context(dtype=torch.bfloat16, rows=3, layers=2):
    HV, H, Q, K, V, NB, C = 6, 2, 4, 8, 8, 16, 5
    convs = [torch.zeros(NB, C, 3 + Q - 1, dtype=dtype) for _ in range(layers)]
    ckpts = [torch.zeros(NB, HV, V, K) for _ in range(layers)]
    recs = [ReplayRecordBuffers.allocate(rows, HV, H, Q, V, K, device="cpu", key_dtype=dtype) for _ in range(layers)]
    return GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=Q, max_num_reqs=rows)


def test_context_geometry_from_tensors():
    ctx = _context()
    assert ctx.record_bytes == record_geometry_bytes(3, 2, 6, 2, 4, 8, 8, torch.bfloat16)
    assert sum(record_nbytes(r) for r in ctx.records) == ctx.record_bytes
    assert ctx.num_key_heads == 2 and ctx.record_layout == "soa" and ctx.key_dtype == torch.bfloat16
    assert tuple(ctx.records[0].shape) == (3, 6, 4, 17)


def test_commit_rejects_before_any_launch():
    ctx = _context()
    acc = torch.ones(3, dtype=torch.int32)
    idx = torch.tensor([1, 2, 3], dtype=torch.int32)
    qsl = torch.tensor([0, 4, 8, 12], dtype=torch.int32)
    before = dict(Kmod.counts())
    with pytest.raises(ValueError, match="align metadata is incomplete"):
        ctx.commit(acc, idx, qsl, block_table=torch.ones(3, 2, dtype=torch.int32))
    with pytest.raises(ValueError, match="commit metadata is incompatible"):
        ctx.commit(acc, idx, qsl[:3])
    with pytest.raises(ValueError, match="cover one speculative window"):
        ctx.commit(acc, idx, qsl, block_table=torch.ones(3, 2, dtype=torch.int32),
                   num_computed_tokens=torch.zeros(3, dtype=torch.int32), mamba_block_size=2)
    with pytest.raises(ValueError, match="HIP device"):  # well-formed, but there is no CPU path
        ctx.commit(acc, idx, qsl)
    assert dict(Kmod.counts()) == before


def _entry(ctx, *, align=False, block_size=8):
    rows = 3
    payload = SimpleNamespace(
        state_indices=torch.tensor([1, 2, 3], dtype=torch.int32),
        query_start_loc=torch.tensor([0, 4, 8, 12], dtype=torch.int32),
        request_indices=torch.arange(rows, dtype=torch.int64),
        block_table=torch.ones(rows, 4, dtype=torch.int32) if align else None,
        num_computed_tokens=torch.zeros(rows, dtype=torch.int32) if align else None,
        block_size=block_size if align else None,
        request_rows=tuple(range(rows)),
        query_lens=(4, 4, 4),
    )
    meta = SimpleNamespace(recoverssm_commit=payload, recoverssm_builder=SimpleNamespace(), recoverssm_context=ctx)
    return CommitEntry(meta, payload, ctx)


def test_grouped_bucket_rejects_before_any_launch():
    ctx = _context()
    bucket = GroupedCommitBucket((ctx,))
    sampled = torch.ones(3, dtype=torch.int32)
    mapping = torch.arange(3, dtype=torch.int32)
    cols = torch.zeros(4, dtype=torch.int32)
    accepted = torch.zeros(4, dtype=torch.int32)
    before = dict(Kmod.counts())
    with pytest.raises(ValueError, match="must not alias"):
        bucket.make_specs((_entry(ctx),), sampled, mapping, cols, sampled)
    with pytest.raises(ValueError, match="different KV epoch"):
        bucket.make_specs((_entry(_context()),), sampled, mapping, cols, accepted)
    with pytest.raises(ValueError, match="HIP device"):  # well-formed, but there is no CPU path
        bucket.make_specs((_entry(ctx),), sampled, mapping, cols, accepted)
    with pytest.raises(ValueError, match="one to three contexts"):
        GroupedCommitBucket(tuple(_context() for _ in range(4)))
    assert dict(Kmod.counts()) == before


def test_coordinator_rejects_mixed_and_disagreeing_groups():
    inputs = (torch.ones(3, dtype=torch.int32), torch.arange(3, dtype=torch.int32), torch.zeros(4, dtype=torch.int32),
              torch.zeros(4, dtype=torch.int32))
    before = dict(Kmod.counts())
    mixed = [_entry(_context(), align=True), _entry(_context(), align=False)]
    with pytest.raises(ValueError, match="cannot mix align and none"):
        GroupedCommitCoordinator().commit([e.metadata for e in mixed], *inputs)
    disagree = [_entry(_context(), align=True, block_size=8), _entry(_context(), align=True, block_size=16)]
    with pytest.raises(ValueError, match="must agree"):
        GroupedCommitCoordinator().commit([e.metadata for e in disagree], *inputs)
    assert dict(Kmod.counts()) == before


@pytest.mark.parametrize("case", range(SC.VERIFY_CASES))
def test_verify_sweep_cases_pass_host_validation(case):
    """Every seeded verify configuration of the GPU sweep is accepted by the
    host checks (on the CPU the call stops only at the device check)."""
    import test_gpu_verify as TV

    c = SC.verify_case(case)
    p = c["problem"]
    P = TV._problem(p["B"], p["H"], p["HV"], p["K"], p["V"], p["Q"], qlens=p["qlens"], seed=p["seed"], act=p["act"],
                    state_dtype=p["state_dtype"], null_rows=p["null_rows"], oob_rows=p["oob_rows"],
                    normalise=p["normalise"])
    with pytest.raises(ValueError, match="HIP device"):
        TV._run_and_check(P, torch.device("cpu"), **c["run"])


@pytest.mark.parametrize("case", range(SC.COMMIT_CASES))
def test_commit_sweep_cases_pass_host_validation(case):
    """The same for the seeded commit configurations."""
    import test_gpu_commit as TC

    c = SC.commit_case(case)
    B, Q, align = c["B"], c["Q"], c["align"]
    G = TC._group(B, c["H"], c["HV"], c["K"], c["V"], Q, c["L"], align=align, seed=c["seed"], Bk=c["Bk"],
                  key_dtype=c["key_dtype"], state_dtype=c["state_dtype"], packed=c["packed"], qlens=c["qlens"])
    ckpts, convs, recs = TC._to_dev(G, torch.device("cpu"))
    ctx = GDNRecoverSSMCommitContext.from_tensors(convs, ckpts, recs, spec_query_len=Q, max_num_reqs=B + 3)
    with pytest.raises(ValueError, match="HIP device"):
        ctx.commit(G["acc"], G["src"], G["qsl"], block_table=G["table"] if align else None,
                   num_computed_tokens=G["C"] if align else None, mamba_block_size=G["Bk"])

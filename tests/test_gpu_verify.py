"""GPU parity of the verify kernel against the CPU oracle (float64).

Bar: bf16 outputs within 1e-2 norm-wise; FP32 corrections within 1e-5
norm-wise; keys bit-exact; decays within 2 ulp; checkpoint bit-identical after
verify; records and outputs outside the written set untouched.
"""

import pytest
import torch

import gdn_oracle as O
from gdn_recoverssm_ascend import workloads as W
from gdn_recoverssm_ascend.kernels import ReplayRecordBuffers, gdn_recoverssm_verify
import sweep_cases as SC
from gpu_helpers import CORR_TOL, OUT_TOL, assert_norm_close, retain_settings, state_cache_retain

pytestmark = pytest.mark.gpu

SENT = -77.0


def _problem(B, H, HV, K, V, Q, *, qlens=None, seed=0, act=torch.bfloat16, state_dtype=torch.float32,
             null_rows=(), oob_rows=(), normalise=True, pages=None):
    gen = torch.Generator().manual_seed(seed)
    qlens = torch.full((B,), Q) if qlens is None else torch.tensor(qlens)
    qsl = torch.zeros(B + 1, dtype=torch.int32)
    qsl[1:] = torch.cumsum(qlens, 0)
    T = int(qsl[-1])
    spec = W.get_spec("plumbing_b4", rows=B, key_heads=H, value_heads=HV, key_dim=K, value_dim=V, window=Q, act_dtype=act)
    inp = W.make_layer_inputs(spec, T, gen)
    if not normalise:
        inp.q = (torch.randn(inp.q.shape, generator=gen) * 2).to(act)
        inp.k = (torch.randn(inp.k.shape, generator=gen) * 2).to(act)
    NB = pages or (B + 2)
    ckpt = (torch.randn(NB, HV, V, K, generator=gen) * 0.1).to(state_dtype)
    idx = (torch.randperm(NB - 1, generator=gen)[:B] + 1).to(torch.int32)
    for r in null_rows:
        idx[r] = -1
    for r in oob_rows:
        idx[r] = NB + 3
    return dict(inp=inp, qsl=qsl, idx=idx, ckpt=ckpt, T=T, B=B, H=H, HV=HV, K=K, V=V, Q=Q)


def _run_and_check(P, dev, *, key_dtype=None, record_rows=None, packed=False, l2norm=False, idx_dtype=torch.int32,
                   column_view=False, out_dtype=None, beta_dtype=torch.float32, scale=None):
    inp, Q, B, H, HV, K, V, T = P["inp"], P["Q"], P["B"], P["H"], P["HV"], P["K"], P["V"], P["T"]
    R = record_rows or B
    key_dtype = key_dtype or (torch.float32 if l2norm else inp.k.dtype)
    q, k, v = inp.q.to(dev), inp.k.to(dev), inp.v.to(dev)
    g, beta = inp.g.to(dev), inp.beta.to(beta_dtype).to(dev)
    ckpt = P["ckpt"].to(dev)
    qsl = P["qsl"].to(idx_dtype).to(dev)
    if column_view:
        table = torch.zeros(B, Q + 3, dtype=idx_dtype, device=dev)
        table[:, 0] = P["idx"].to(idx_dtype).to(dev)
        idx = table[:, 0]
    else:
        idx = P["idx"].to(idx_dtype).to(dev)
    def launch():
        if packed:
            rec = torch.full((R, HV, Q, V + K + 1), SENT, dtype=torch.float32, device=dev)
        else:
            rec = ReplayRecordBuffers(
                torch.full((R, HV, Q, V), SENT, dtype=torch.float32, device=dev),
                torch.full((R, H, Q, K), SENT, dtype=key_dtype, device=dev),
                torch.full((R, HV, Q), SENT, dtype=torch.float32, device=dev),
            )
        out = torch.full((1, T, HV, V), SENT, dtype=out_dtype or v.dtype, device=dev)
        ret = gdn_recoverssm_verify(
            g, beta, q, k, v, checkpoint_state=ckpt, replay_cache=rec, query_start_loc=qsl, state_indices=idx,
            spec_query_len=Q, qk_already_normalized=not l2norm, out=out, scale=scale,
        )
        torch.cuda.synchronize()
        assert ret is out
        planes = (rec,) if packed else (rec.correction, rec.key, rec.decay)
        return out, rec, planes

    before = ckpt.clone()
    out, rec, planes = launch()
    assert torch.equal(ckpt, before), "verify must never write the checkpoint"
    # The same launch with the state read non-temporally (row-run loads
    # turned into the operand layout through LDS) for every row, then for the
    # earlier half: the same bits as the ordinary loads.
    for retain in retain_settings(B, HV * V * K * ckpt.element_size())[:2]:
        with state_cache_retain(retain):
            out2, _, planes2 = launch()
        assert torch.equal(out2, out), f"outputs differ with {retain} retained state bytes"
        for a_, b_ in zip(planes2, planes):
            assert torch.equal(a_, b_), f"records differ with {retain} retained state bytes"
    res = O.oracle_verify(
        inp.q, inp.k, inp.v, inp.g, inp.beta.to(beta_dtype), P["ckpt"], P["qsl"], P["idx"], Q, scale=scale,
        qk_already_normalized=not l2norm, record_rows=R, packed_key_per_value_head=packed,
    )
    got_out = out.cpu()[0]
    w = res.out_written
    assert torch.all(got_out[~w] == SENT), "outputs outside the window were written"
    assert_norm_close(got_out[w].double(), res.out[w], OUT_TOL, "out")
    if packed:
        rc = rec.cpu()
        corr, key, decay = rc[..., :V], rc[..., V:V + K], rc[..., V + K]
    else:
        corr, key, decay = rec.correction.cpu(), rec.key.cpu(), rec.decay.cpu()
    rw = res.record_written  # [R, Q]
    m_c = rw[:, None, :, None].expand_as(corr)
    assert torch.all(corr[~m_c] == SENT), "correction written outside the valid set"
    assert_norm_close(corr[m_c].double(), res.correction[m_c], CORR_TOL, "correction")
    m_d = rw[:, None, :].expand_as(decay)
    assert torch.all(decay[~m_d] == SENT)
    torch.testing.assert_close(decay[m_d].double(), res.decay[m_d], rtol=3e-7, atol=0)
    m_k = rw[:, None, :, None].expand_as(key)
    assert torch.all(key[~m_k] == SENT)
    if l2norm:
        torch.testing.assert_close(key[m_k].double(), res.key[m_k].double(), rtol=2e-6, atol=1e-7)
    else:
        assert torch.equal(key[m_k].float(), res.key[m_k].float()), "keys must keep the input bits"
    return res


@pytest.fixture(scope="module")
def dev(gpu_device):
    return gpu_device


def test_plumbing_config_full(dev):
    w = W.make_workload("plumbing_b4")
    P = dict(inp=w.inputs[0], qsl=w.meta.query_start_loc, idx=w.meta.state_indices.clone(), ckpt=w.checkpoints[0],
             T=w.tokens, B=4, H=2, HV=4, K=64, V=64, Q=4)
    _run_and_check(P, dev)


@pytest.mark.parametrize("Q", [1, 2, 3, 4, 5, 8])
def test_every_window_length(dev, Q):
    _run_and_check(_problem(5, 2, 4, 128, 128, Q, seed=Q), dev)


@pytest.mark.parametrize("K,V", [(64, 64), (128, 128), (256, 128), (128, 96), (64, 192), (32, 16)])
def test_head_dims(dev, K, V):
    _run_and_check(_problem(3, 1, 2, K, V, 4, seed=K + V), dev)


def test_ragged_null_and_out_of_range_rows(dev):
    P = _problem(8, 2, 4, 128, 128, 4, qlens=[4, 0, 2, 4, 1, 3, 4, 4], null_rows=(3,), oob_rows=(6,))
    res = _run_and_check(P, dev)
    assert not bool(res.record_written[3].any()) and not bool(res.record_written[6].any())


def test_record_rows_smaller_than_batch(dev):
    _run_and_check(_problem(6, 2, 4, 128, 128, 4), dev, record_rows=4)


def test_packed_record_layout(dev):
    _run_and_check(_problem(4, 2, 4, 128, 128, 4, qlens=[4, 3, 4, 2]), dev, packed=True)


def test_in_kernel_l2norm(dev):
    _run_and_check(_problem(4, 2, 4, 128, 128, 4, normalise=False), dev, l2norm=True)


def test_fp32_key_records_and_beta_in_activation_dtype(dev):
    _run_and_check(_problem(4, 2, 4, 128, 128, 4), dev, key_dtype=torch.float32, beta_dtype=torch.bfloat16)


def test_int64_metadata_and_column_view_indices(dev):
    _run_and_check(_problem(5, 2, 4, 128, 128, 4), dev, idx_dtype=torch.int64, column_view=True)


def test_fp16_activations_and_fp32_output(dev):
    P = _problem(4, 2, 4, 128, 128, 4, act=torch.float16)
    _run_and_check(P, dev, out_dtype=torch.float32, scale=0.3)


@pytest.mark.parametrize("state_dtype", [torch.bfloat16, torch.float16])
def test_low_precision_state(dev, state_dtype):
    _run_and_check(_problem(4, 2, 4, 128, 128, 4, state_dtype=state_dtype), dev)


def test_gqa_ratio_one_and_four(dev):
    _run_and_check(_problem(3, 4, 4, 128, 128, 4), dev)
    _run_and_check(_problem(3, 2, 8, 128, 128, 4), dev)


def test_empty_batch_returns_without_launch(dev):
    P = _problem(2, 1, 2, 128, 128, 4, qlens=[0, 0])
    q = torch.zeros(1, 0, 1, 128, dtype=torch.bfloat16, device=dev)
    v = torch.zeros(1, 0, 2, 128, dtype=torch.bfloat16, device=dev)
    g = torch.zeros(0, 2, device=dev)
    rec = ReplayRecordBuffers.allocate(2, 2, 1, 4, 128, 128, device=dev, key_dtype=torch.bfloat16)
    out = gdn_recoverssm_verify(g, g, q, q, v, checkpoint_state=P["ckpt"].to(dev), replay_cache=rec,
                                query_start_loc=P["qsl"].to(dev), state_indices=P["idx"].to(dev), spec_query_len=4)
    assert out.shape == (1, 0, 2, 128)


@pytest.mark.parametrize("name,rows", [("pool512_b64", None), ("align_b256", 40), ("decode_q1_b256", 40),
                                       ("skewed_q8_b256", 24)])
def test_baseline_workloads(dev, name, rows):
    """Full-size launches; the oracle checks a seeded subset of rows."""
    w = W.make_workload(name, gen_device=dev.type)
    spec = w.spec
    B, Q, H, HV, K, V = spec.rows, spec.window, spec.key_heads, spec.value_heads, spec.key_dim, spec.value_dim
    wd = w.to(dev)
    inp = wd.inputs[0]
    rec = ReplayRecordBuffers(
        torch.full((B, HV, Q, V), SENT, device=dev), torch.full((B, H, Q, K), SENT, dtype=torch.bfloat16, device=dev),
        torch.full((B, HV, Q), SENT, device=dev),
    )
    out = torch.full((1, w.tokens, HV, V), SENT, dtype=torch.bfloat16, device=dev)
    ckpt = wd.checkpoints[0]
    gdn_recoverssm_verify(inp.g, inp.beta, inp.q, inp.k, inp.v, checkpoint_state=ckpt, replay_cache=rec,
                          query_start_loc=wd.meta.query_start_loc, state_indices=wd.meta.state_indices, spec_query_len=Q,
                          out=out)
    torch.cuda.synchronize()
    # Every row non-temporal, and every row ordinary: the same bits as the
    # default split.
    for retain in retain_settings(B, HV * V * K * 4)[::2]:
        rec2 = ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=torch.bfloat16)
        for t in (rec2.correction, rec2.key, rec2.decay):
            t.fill_(SENT)
        out2 = torch.full_like(out, SENT)
        with state_cache_retain(retain):
            gdn_recoverssm_verify(inp.g, inp.beta, inp.q, inp.k, inp.v, checkpoint_state=ckpt, replay_cache=rec2,
                                  query_start_loc=wd.meta.query_start_loc, state_indices=wd.meta.state_indices,
                                  spec_query_len=Q, out=out2)
        torch.cuda.synchronize()
        assert torch.equal(out2, out), f"{name}: outputs differ with {retain} retained state bytes"
        for a_, b_ in zip((rec2.correction, rec2.key, rec2.decay), (rec.correction, rec.key, rec.decay)):
            assert torch.equal(a_, b_), f"{name}: records differ with {retain} retained state bytes"
    sel = list(range(B)) if rows is None else sorted(torch.randperm(B, generator=torch.Generator().manual_seed(1))[:rows].tolist())
    if "padded_rows" in w.extras:
        sel = sorted(set(sel) | set(w.extras["padded_rows"].tolist()[:2]))
    qsl = w.meta.query_start_loc
    idx = w.meta.state_indices
    pages = [int(idx[r]) for r in sel]
    valid_pages = [p for p in pages if p > 0]
    ck_cpu = torch.zeros(len(valid_pages) + 1, HV, V, K)
    remap = {}
    for j, p in enumerate(valid_pages):
        ck_cpu[j + 1] = ckpt[p].cpu()
        remap[p] = j + 1
    sub_idx = torch.tensor([remap.get(p, -1) for p in pages], dtype=torch.int32)
    toks = torch.cat([torch.arange(int(qsl[r]), int(qsl[r + 1])) for r in sel])
    lens = torch.tensor([int(qsl[r + 1] - qsl[r]) for r in sel])
    sub_qsl = torch.zeros(len(sel) + 1, dtype=torch.int32)
    sub_qsl[1:] = torch.cumsum(lens, 0)
    ci = w.inputs[0]
    cq, ck, cv, cg, cb = (t.cpu() for t in (ci.q, ci.k, ci.v, ci.g, ci.beta))
    res = O.oracle_verify(cq[:, toks], ck[:, toks], cv[:, toks], cg[toks], cb[toks], ck_cpu, sub_qsl, sub_idx, Q)
    got_out = out[0, toks.to(dev)].cpu()
    assert_norm_close(got_out.double(), res.out, OUT_TOL, f"{name} out")
    sel_t = torch.tensor(sel, device=dev)
    corr = rec.correction[sel_t].cpu()
    m = res.record_written[:, None, :, None].expand_as(corr)
    assert_norm_close(corr[m].double(), res.correction[m], CORR_TOL, f"{name} correction")
    assert torch.all(corr[~m] == SENT)
    keys = rec.key[sel_t].cpu()
    mk = res.record_written[:, None, :, None].expand_as(keys)
    assert torch.equal(keys[mk].float(), res.key[mk].float())


def test_verify_graph_replay(dev):
    """A verify launch recorded in a HIP graph: every replay, with eager work
    in between, reproduces the eager launch bit for bit."""
    P = _problem(6, 2, 4, 128, 128, 4, qlens=[4, 3, 4, 2, 0, 4], null_rows=(1,))
    inp, B, H, HV, K, V, Q, T = P["inp"], P["B"], P["H"], P["HV"], P["K"], P["V"], P["Q"], P["T"]
    q, k, v, g, beta = (t.to(dev) for t in (inp.q, inp.k, inp.v, inp.g, inp.beta))
    ckpt, qsl, idx = P["ckpt"].to(dev), P["qsl"].to(dev), P["idx"].to(dev)
    rec = ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=k.dtype)
    out = torch.empty(1, T, HV, V, dtype=v.dtype, device=dev)

    def run():
        gdn_recoverssm_verify(g, beta, q, k, v, checkpoint_state=ckpt, replay_cache=rec, query_start_loc=qsl,
                              state_indices=idx, spec_query_len=Q, out=out)

    def reset():
        for t in (out, rec.correction, rec.key, rec.decay):
            t.fill_(SENT)

    reset()
    run()
    torch.cuda.synchronize()
    want = [t.clone() for t in (out, rec.correction, rec.key, rec.decay)]
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()  # warm the launch path on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        run()
    for _ in range(3):
        reset()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, ref in zip((out, rec.correction, rec.key, rec.decay), want):
            assert torch.equal(got, ref), "graph replay differs from the eager launch"


def _gated_check(dev, P, ab_dtype, param_dtype, seed=21):
    from gdn_recoverssm_ascend.kernels import gdn_recoverssm_verify_gated

    inp, B, H, HV, K, V, Q, T = P["inp"], P["B"], P["H"], P["HV"], P["K"], P["V"], P["Q"], P["T"]
    gen = torch.Generator().manual_seed(seed)
    a = (torch.randn(T, HV, generator=gen) * 3).to(ab_dtype)
    b = (torch.randn(T, HV, generator=gen) * 2).to(ab_dtype)
    A_log = torch.randn(HV, generator=gen).to(param_dtype)
    dt_bias = torch.randn(HV, generator=gen).to(param_dtype)
    a[0, 0] = 30.0  # the linear branch of softplus
    def launch():
        rec = ReplayRecordBuffers(
            torch.full((B, HV, Q, V), SENT, device=dev), torch.full((B, H, Q, K), SENT, device=dev),
            torch.full((B, HV, Q), SENT, device=dev),
        )
        out = torch.full((1, T, HV, V), SENT, dtype=inp.v.dtype, device=dev)
        gdn_recoverssm_verify_gated(a.to(dev), b.to(dev), inp.q.to(dev), inp.k.to(dev), inp.v.to(dev),
                                    A_log=A_log.to(dev), dt_bias=dt_bias.to(dev), checkpoint_state=P["ckpt"].to(dev),
                                    replay_cache=rec, query_start_loc=P["qsl"].to(dev),
                                    state_indices=P["idx"].to(dev), spec_query_len=Q, out=out)
        torch.cuda.synchronize()
        return out, rec

    out, rec = launch()
    with state_cache_retain(0):
        out2, rec2 = launch()
    assert torch.equal(out2, out)
    for a_, b_ in zip((rec2.correction, rec2.key, rec2.decay), (rec.correction, rec.key, rec.decay)):
        assert torch.equal(a_, b_), "gated records differ with the state read non-temporally"
    g, beta = O.oracle_gating(a, b, A_log, dt_bias)
    res = O.oracle_verify(inp.q, inp.k, inp.v, g, beta, P["ckpt"], P["qsl"], P["idx"], Q, qk_already_normalized=False)
    w = res.out_written
    got = out.cpu()[0]
    assert torch.all(got[~w] == SENT)
    assert_norm_close(got[w].double(), res.out[w], OUT_TOL, "gated out")
    rw = res.record_written
    corr = rec.correction.cpu()
    m_c = rw[:, None, :, None].expand_as(corr)
    assert_norm_close(corr[m_c].double(), res.correction[m_c], CORR_TOL, "gated correction")
    decay = rec.decay.cpu()
    m_d = rw[:, None, :].expand_as(decay)
    # decay = exp(g) carries g's FP32 rounding times |g|: allow 2 ulps of g
    # (2 * 2^-23 * |g|) on top of the exponential's own error. Below FP32's
    # normal range a decay is a subnormal, spaced 2^-149 apart (or 0 under
    # it: exp(-120) is 0 in FP32), so two of those spacings are allowed too.
    want_d = res.decay[m_d]
    tol = want_d * (3e-6 + 2.4e-7 * (-torch.log(want_d)).abs()) + 2.0 * 2.0**-149
    got_d = decay[m_d].double()
    bad = (got_d - want_d).abs() > tol
    assert not bool(bad.any()), "gated decay: " + ", ".join(
        f"got {float(x):.6e} want {float(y):.6e} g {float(z):.4f}"
        for x, y, z in zip(got_d[bad][:4], want_d[bad][:4], torch.log(want_d[bad][:4])))
    key = rec.key.cpu()
    m_k = rw[:, None, :, None].expand_as(key)
    torch.testing.assert_close(key[m_k].double(), res.key[m_k].double(), rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("ab_dtype,param_dtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.float32),
                                                  (torch.bfloat16, torch.bfloat16)])
def test_gated_verify_fuses_gating_and_l2norm(dev, ab_dtype, param_dtype):
    """gdn_recoverssm_verify_gated from raw a, b, q, k against the oracle fed
    the oracle's own gating of the same raw inputs."""
    P = _problem(5, 2, 4, 128, 128, 4, qlens=[4, 3, 4, 0, 2], null_rows=(3,), normalise=False)
    _gated_check(dev, P, ab_dtype, param_dtype)


@pytest.mark.parametrize("K,V,Q,H,HV,act", [
    (64, 100, 3, 1, 4, torch.bfloat16),
    (256, 48, 8, 2, 2, torch.float16),
    (32, 192, 1, 3, 6, torch.float32),
    (136, 16, 6, 1, 1, torch.bfloat16),
])
def test_gated_verify_shapes(dev, K, V, Q, H, HV, act):
    """The gated verify at head dims off the 128 x 128 tile, windows 1-8, GQA
    ratios 1-4 and every activation dtype (a, b in the activation dtype)."""
    gen = torch.Generator().manual_seed(K + V)
    qlens = [int(x) for x in torch.randint(0, Q + 1, (4,), generator=gen)]
    qlens[0] = Q
    P = _problem(4, H, HV, K, V, Q, qlens=qlens, oob_rows=(2,), normalise=False, act=act, seed=K * V)
    _gated_check(dev, P, act, torch.float32, seed=Q)


@pytest.mark.parametrize("case", range(SC.GATED_CASES))
def test_random_gated(dev, case):
    """Seeded draws of the gated verify's options together, against the
    oracle fed the oracle's own gating of the same raw inputs."""
    c = SC.gated_case(case)
    print(f"gated sweep case {case}: {c}", flush=True)
    P = _problem(c["B"], c["H"], c["HV"], c["K"], c["V"], c["Q"], qlens=c["qlens"], null_rows=c["null_rows"],
                 oob_rows=c["oob_rows"], normalise=False, act=c["act"], state_dtype=c["state"], seed=c["seed"])
    _gated_check(dev, P, c["ab"], c["param"], seed=c["seed"] + 1)


@pytest.mark.parametrize("case", range(SC.VERIFY_CASES))
def test_random_configurations(dev, case):
    """Seeded draws of every verify option together: head dims, GQA ratio,
    window, ragged / null / out-of-range rows, activation, state, key, beta
    and output dtypes, packed records, in-kernel L2 norm, index dtypes and
    column views, record rows below the batch, explicit scale."""
    c = SC.verify_case(case)
    p = c["problem"]
    print(f"verify sweep case {case}: {p} {c['run']}", flush=True)
    P = _problem(p["B"], p["H"], p["HV"], p["K"], p["V"], p["Q"], qlens=p["qlens"], seed=p["seed"], act=p["act"],
                 state_dtype=p["state_dtype"], null_rows=p["null_rows"], oob_rows=p["oob_rows"],
                 normalise=p["normalise"])
    _run_and_check(P, dev, **c["run"])


def test_launches_follow_the_current_stream(dev):
    """Every launch goes on torch's current stream (csrc/ops.cpp:142-153 of the
    reference runs on the device's current stream): a verify issued inside
    ``torch.cuda.stream(s)`` behind a spin kernel on s is still pending on s
    after the default stream has drained, and then matches the same verify
    run on the default stream."""
    P = _problem(4, 2, 4, 128, 128, 4, seed=77)
    inp, B, H, HV, K, V, Q, T = P["inp"], P["B"], P["H"], P["HV"], P["K"], P["V"], P["Q"], P["T"]
    args = (inp.g.to(dev), inp.beta.to(dev), inp.q.to(dev), inp.k.to(dev), inp.v.to(dev))
    kw = dict(checkpoint_state=P["ckpt"].to(dev), query_start_loc=P["qsl"].to(dev),
              state_indices=P["idx"].to(dev), spec_query_len=Q)
    outs = []
    for side in (False, True):
        rec = ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=inp.k.dtype)
        torch.cuda.synchronize()
        if side:
            s = torch.cuda.Stream(device=dev)
            with torch.cuda.stream(s):
                torch.cuda._sleep(20_000_000)
                out = gdn_recoverssm_verify(*args, replay_cache=rec, **kw)
            torch.cuda.default_stream(dev).synchronize()
            assert not s.query(), "the verify did not queue behind the side stream's spin kernel"
            s.synchronize()
        else:
            out = gdn_recoverssm_verify(*args, replay_cache=rec, **kw)
            torch.cuda.synchronize()
        outs.append((out.clone(), rec.correction.clone()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])

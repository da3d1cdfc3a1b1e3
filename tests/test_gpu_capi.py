"""The C ABI on its own: a native program (tests/capi/capi_step.cpp, built by
the build step) allocates device buffers with hipMalloc, calls
gdn_recoverssm_verify, gdn_recoverssm_plan_fold and
gdn_recoverssm_conv_compact the way a non-Python
serving runtime would, and writes the results back. Nothing of the Python
package runs on the device in this test; the program is started as a child
process and its outputs are checked against the CPU oracle.

Problem: an align-mode step (prefix-cache block table, boundary crossings,
padded rows) at K=V=128, Q=4, 16 rows, 2 key heads, 4 value heads, with the
conv states of the same pages compacted from the plan the commit stored.
Bar: plan arrays and conv states bit-exact; bf16 outputs within 1e-2
norm-wise; corrections within 1e-5 norm-wise; keys bit-exact; decays within
3e-7 relative; committed FP32 pages within max-abs 1e-5 relative; every other
page bit-identical.
"""

import os
import subprocess

import numpy as np
import pytest
import torch

import gdn_oracle as O
from gdn_recoverssm_ascend import workloads as W
from gpu_helpers import CORR_TOL, OUT_TOL, assert_norm_close, assert_state_close

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "capi", "capi_step")


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy()
    return t.numpy()


def _read(path, dtype, shape):
    a = np.fromfile(path, dtype=dtype)
    t = torch.from_numpy(a.copy())
    if dtype == np.int16:
        t = t.view(torch.bfloat16)
    return t.reshape(shape)


@pytest.mark.parametrize("seed", [5, 11])
def test_native_caller_step_against_oracle(tmp_path, seed):
    assert os.path.exists(EXE), "tests/capi/capi_step is missing: run __graft_entry__.build() first"
    w = W.make_workload("align_b256", seed=seed, rows=16, key_heads=2, value_heads=4, padded_rows=2)
    s, m = w.spec, w.meta
    B, Q, H, HV, K, V = s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
    inp = w.inputs[0]
    T = int(m.query_start_loc[-1])
    NB, Wd = w.num_pages, int(m.block_table.shape[1])
    scale = K ** -0.5
    print(f"native C-ABI step: seed={seed} B={B} T={T} pages={NB} table width={Wd}", flush=True)

    d = str(tmp_path)
    conv = w.conv_states[0]
    CD, CW = int(conv.shape[1]), int(conv.shape[2])
    meta = dict(B=B, T=T, H=H, HV=HV, K=K, V=V, Q=Q, NB=NB, W=Wd, BS=m.block_size, CD=CD, CW=CW, SCALE=scale)
    with open(os.path.join(d, "meta.txt"), "w") as f:
        f.writelines(f"{k} {v!r}\n" for k, v in meta.items())
    i32 = lambda t: t.to(torch.int32)  # noqa: E731
    arrays = dict(q=inp.q, k=inp.k, v=inp.v, g=inp.g.float(), beta=inp.beta.float(), state=w.checkpoints[0], conv=conv,
                  qsl=i32(m.query_start_loc), idx=i32(m.state_indices), accepted=i32(m.accepted),
                  table=i32(m.block_table), computed=i32(m.num_computed))
    for name, t in arrays.items():
        _bits(t).tofile(os.path.join(d, f"{name}.bin"))

    r = subprocess.run([EXE, d], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=120)
    print(r.stdout.decode(errors="replace"), flush=True)
    assert r.returncode == 0, f"capi_step exited with {r.returncode}"

    rd = lambda n, dt, sh: _read(os.path.join(d, f"out_{n}.bin"), dt, sh)  # noqa: E731
    res = O.oracle_verify(inp.q, inp.k, inp.v, inp.g, inp.beta, w.checkpoints[0], m.query_start_loc,
                          m.state_indices, Q, scale=scale)
    out = rd("out", np.int16, (T, HV, V))
    wm = res.out_written
    assert_norm_close(out[wm].double(), res.out[wm], OUT_TOL, "out")
    assert torch.all(out[~wm] == 0), "outputs outside the windows were written"
    rw = res.record_written  # [B, Q]
    corr = rd("corr", np.float32, (B, HV, Q, V))
    m_c = rw[:, None, :, None].expand_as(corr)
    assert_norm_close(corr[m_c].double(), res.correction[m_c], CORR_TOL, "correction")
    assert torch.all(corr[~m_c] == 0)
    key = rd("key", np.int16, (B, H, Q, K))
    m_k = rw[:, None, :, None].expand_as(key)
    assert torch.equal(key[m_k].float(), res.key[m_k].float()), "keys must keep the input bits"
    decay = rd("decay", np.float32, (B, HV, Q))
    m_d = rw[:, None, :].expand_as(decay)
    torch.testing.assert_close(decay[m_d].double(), res.decay[m_d], rtol=3e-7, atol=0)

    plan = O.oracle_plan_single(m.accepted, m.state_indices, m.query_start_loc, spec_query_len=Q, num_blocks=NB,
                                block_table=m.block_table, num_computed=m.num_computed, block_size=m.block_size)
    valid = plan["align_valid"].bool()
    want_source = torch.where(valid, m.state_indices.to(torch.int32), torch.zeros(B, dtype=torch.int32))
    for name, want in (("source", want_source), ("lens", plan["commit_lens"]), ("final", plan["final"]),
                       ("boundary", plan["boundary"]), ("blen", plan["boundary_len"]),
                       ("valid", plan["align_valid"]), ("col", plan["align_col"])):
        got = rd(name, np.int32, (B,))
        assert got.tolist() == want.tolist(), f"plan {name} differs"
    n = plan["commit_lens"]
    assert int((n > 0).sum()) > 0 and int(plan["boundary_len"].gt(0).sum()) > 0, "the step must commit and cross"

    want = O.oracle_fold([w.checkpoints[0]], [res.correction], [res.key], [res.decay], source=m.state_indices,
                         lengths=n, final=plan["final"], boundary=plan["boundary"],
                         boundary_len=plan["boundary_len"], rows=B, num_blocks=NB, record_rows=B,
                         out_dtype=torch.float32)[0]
    got = rd("state", np.float32, (NB, HV, V, K))
    ck0 = w.checkpoints[0]
    targeted = sorted({int(p) for p in plan["final"][n > 0]} | {int(p) for p in plan["boundary"][n > 0] if int(p) > 0})
    untouched = torch.ones(NB, dtype=torch.bool)
    untouched[targeted] = False
    assert torch.equal(got[untouched], ck0[untouched]), "pages outside the commit changed"
    assert_state_close(got[targeted], want[targeted], "committed pages")

    want_conv = O.oracle_conv_compact([conv], source=m.state_indices, lengths=n, final=plan["final"],
                                      boundary=plan["boundary"], boundary_len=plan["boundary_len"],
                                      history=CW - Q + 1, num_blocks=NB, rows=B, align=True)[0]
    assert torch.equal(rd("conv", np.int16, (NB, CD, CW)), want_conv), "conv states differ"

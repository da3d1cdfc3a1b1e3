"""Shared helpers for the GPU parity tests: run the HIP path and the CPU oracle
on the same seeded inputs and compare them to the stated tolerances.

Tolerances (the bar for this path):
* integer plan outputs, slot / accepted-length / align-boundary indexing: bit-exact;
* FP32 state: max |gpu - oracle| <= 1e-5 * max |oracle| (infinity norm of the pages);
* FP32 records (correction): norm-wise relative error <= 1e-5;
* bf16 outputs: norm-wise relative error <= 1e-2;
* bf16 keys and FP32 decays written by verify: bit-exact keys, decay within 2 ulp.
"""

from __future__ import annotations

import contextlib

import torch

import gdn_oracle as O

STATE_TOL = 1e-5
CORR_TOL = 1e-5
OUT_TOL = 1e-2


def sub_workload(inputs, qsl, state_indices, rows):
    """Gather the token windows of `rows` into a compact problem (CPU tensors)."""
    qsl = qsl.cpu().long()
    idx = state_indices.cpu()
    segs = [torch.arange(int(qsl[r]), int(qsl[r + 1])) for r in rows]
    toks = torch.cat(segs) if segs else torch.zeros(0, dtype=torch.long)
    lens = torch.tensor([len(s) for s in segs])
    new_qsl = torch.zeros(len(rows) + 1, dtype=torch.long)
    new_qsl[1:] = torch.cumsum(lens, 0)
    pick = lambda t, dim=1: t.cpu().index_select(dim, toks)  # noqa: E731
    return dict(
        q=pick(inputs.q), k=pick(inputs.k), v=pick(inputs.v), g=pick(inputs.g, 0), beta=pick(inputs.beta, 0),
        qsl=new_qsl, idx=idx[list(rows)], toks=toks,
    )


def assert_state_close(got: torch.Tensor, want: torch.Tensor, what: str = "state"):
    err = O.max_abs_rel(got, want)
    assert err <= STATE_TOL, f"{what}: max-abs error / max-abs = {err:.3g} > {STATE_TOL}"


def assert_norm_close(got: torch.Tensor, want: torch.Tensor, tol: float, what: str):
    err = O.rel_err_norm(got, want)
    assert err <= tol, f"{what}: norm-wise relative error {err:.3g} > {tol}"


@contextlib.contextmanager
def state_cache_retain(nbytes: int):
    """Verify launches inside read all but the last `nbytes` of their state
    non-temporally (gdn_recoverssm_set_state_cache_retain); restored after."""
    import gdn_recoverssm_ascend as G

    prev = G.set_state_cache_retain(nbytes)
    try:
        yield
    finally:
        G.set_state_cache_retain(prev)


def retain_settings(rows: int, row_state_bytes: int) -> tuple[int, ...]:
    """Settings that run a verify's state loads through each body: every row
    non-temporal (0), the later half ordinary, every row ordinary."""
    return (0, (rows // 2) * row_state_bytes, 1 << 50)

"""Pins the CPU oracle's verify and fold against known answers and closed forms.

Every check here is independent of the oracle's own loop: hand-computed values
transcribed from the reference tests (tests/golden/reference_known_answers.json),
a triangular-solve formulation of the delta rule, and the closed-form fold
S_n = G_n S_0 + sum_t (G_n / G_t) c_t k_t^T.
"""

import json
import math
import os

import pytest
import torch

import gdn_oracle as O

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))


def test_verify_hand_case_matches_reference_known_answer():
    case = GOLD["verify_hand_case"]
    hv, d = case["value_heads"], case["dim"]
    q = torch.tensor(case["q"], dtype=torch.float64).reshape(1, 2, 1, d)
    k = torch.tensor(case["k"], dtype=torch.float64).reshape(1, 2, 1, d)
    v = torch.tensor(case["v"], dtype=torch.float64)[:, None, :].expand(2, hv, d).reshape(1, 2, hv, d)
    g = torch.full((2, hv), case["g"], dtype=torch.float64)
    beta = torch.full((2, hv), case["beta"], dtype=torch.float64)
    ckpt = torch.zeros(2, hv, d, d, dtype=torch.float64)
    res = O.oracle_verify(
        q, k, v, g, beta, ckpt, torch.tensor([0, 2]), torch.tensor([1]), 2,
        scale=case["scale"], keep_states=True,
    )
    want = torch.tensor(case["expected_out"], dtype=torch.float64)
    assert torch.equal(res.out, want[:, None, :].expand(2, hv, d))
    assert torch.equal(res.correction[0].permute(1, 0, 2), want[:, None, :].expand(2, hv, d))
    assert torch.equal(res.decay, torch.full((1, hv, 2), case["expected_decay"], dtype=torch.float64))
    # prefix states: after token 0 only column 0 is populated (test_ascendc_selftest_oracle.py:30-33)
    s1 = res.states[0][0]
    assert torch.equal(s1[:, :, 0], want[0][None, :].expand(hv, d))
    assert torch.count_nonzero(s1[:, :, 1]) == 0
    assert torch.equal(res.states[1][0][:, :, 1], want[1][None, :].expand(hv, d))


def _fold_one(ckpt, corr, key, decay, n, final=1, boundary=0, blen=0):
    return O.oracle_fold(
        [ckpt], [corr], [key], [decay],
        source=torch.tensor([1]), lengths=torch.tensor([n]), final=torch.tensor([final]),
        boundary=torch.tensor([boundary]), boundary_len=torch.tensor([blen]),
        rows=1, num_blocks=ckpt.shape[0], record_rows=1,
    )[0]


def test_fold_hand_case_matches_reference_known_answer():
    case = GOLD["fold_hand_case"]
    hv = case["value_heads"]
    ckpt = torch.full((2, hv, 2, 2), case["initial"], dtype=torch.float64)
    keys = torch.tensor(case["keys"], dtype=torch.float64).reshape(1, 1, 2, 2)
    corr = torch.tensor(case["corrections"], dtype=torch.float64)[None, None].expand(1, hv, 2, 2).clone()
    decay = torch.full((1, hv, 2), case["decay"], dtype=torch.float64)
    out = _fold_one(ckpt, corr, keys, decay, case["accepted"])
    want = torch.tensor(case["expected"], dtype=torch.float64)
    assert torch.equal(out[1], want[None].expand(hv, 2, 2))
    # n == 0 leaves the checkpoint bit-identical
    zero = _fold_one(ckpt, corr, keys, decay, 0)
    assert torch.equal(zero, ckpt)


def test_alias_case_single_pass_boundary():
    case = GOLD["alias_scalar_case"]
    ckpt = torch.zeros(3, 1, 1, 1, dtype=torch.float64)
    ckpt[1] = case["h0"]
    n = case["accepted"]
    corr = torch.full((1, 1, n, 1), case["correction"], dtype=torch.float64)
    key = torch.full((1, 1, n, 1), case["key"], dtype=torch.float64)
    decay = torch.full((1, 1, n), case["decay"], dtype=torch.float64)
    # final lands in the source page (1); the boundary snapshot goes to page 2
    out = _fold_one(ckpt, corr, key, decay, n, final=1, boundary=2, blen=case["boundary_len"])
    assert float(out[1]) == case["expected_final"]
    assert float(out[2]) == case["expected_boundary"]
    # the two-pass shape (boundary folded again from the overwritten page) differs
    h = case["expected_final"]
    for _ in range(case["boundary_len"]):
        h = h * case["decay"] + case["correction"] * case["key"]
    assert h == case["two_pass_bug_value"] != case["expected_boundary"]


def _random_case(seed, T, H, HV, K, V, dtype=torch.float64):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(1, T, H, K, generator=gen, dtype=dtype)
    k = torch.randn(1, T, H, K, generator=gen, dtype=dtype)
    q = q / q.norm(dim=-1, keepdim=True)
    k = k / k.norm(dim=-1, keepdim=True)
    v = torch.randn(1, T, HV, V, generator=gen, dtype=dtype)
    beta = torch.sigmoid(torch.randn(T, HV, generator=gen, dtype=dtype))
    g = -torch.nn.functional.softplus(torch.randn(T, HV, generator=gen, dtype=dtype))
    return q, k, v, g, beta


def _triangular_reference(s0, q, k, v, g, beta, scale):
    """Independent chunk form of the gated delta rule for one (row, head).

    With G_t = prod_{s<=t} exp(g_s), the corrections solve the unit lower
    triangular system  c_t + beta_t * sum_{s<t} (G_t/G_s)(k_s.k_t) c_s
                        = beta_t (v_t - G_t S_0 k_t),
    and o_t = G_t S_0 q_t + sum_{s<=t} (G_t/G_s)(k_s.q_t) c_s.
    s0 [V, K]; q, k [Q, K]; v [Q, V]; g, beta [Q]. Returns (out [Q,V], c [Q,V]).
    """
    Q = q.shape[0]
    G = torch.cumprod(torch.exp(g), 0)
    ratio = G[:, None] / G[None, :]  # [t, s]
    A = torch.tril(ratio * (k @ k.T).T, diagonal=-1)  # A[t,s] = G_t/G_s k_s.k_t
    M = torch.eye(Q, dtype=s0.dtype) + beta[:, None] * A
    rhs = beta[:, None] * (v - G[:, None] * (k @ s0.T))
    c = torch.linalg.solve_triangular(M, rhs, upper=False)
    qs = q * scale
    W = torch.tril(ratio * (k @ qs.T).T)  # W[t,s] = G_t/G_s k_s.q_t, s<=t
    out = G[:, None] * (qs @ s0.T) + W @ c
    return out, c


@pytest.mark.parametrize("Q", [1, 2, 4, 8])
def test_verify_matches_triangular_chunk_form(Q):
    B, H, HV, K, V = 3, 2, 4, 16, 8
    T = B * Q
    q, k, v, g, beta = _random_case(Q, T, H, HV, K, V)
    gen = torch.Generator().manual_seed(100 + Q)
    ckpt = torch.randn(B + 1, HV, V, K, generator=gen, dtype=torch.float64) * 0.1
    qsl = torch.arange(B + 1) * Q
    idx = torch.arange(1, B + 1)
    ckpt_copy = ckpt.clone()
    res = O.oracle_verify(q, k, v, g, beta, ckpt, qsl, idx, Q, scale=0.37)
    assert torch.equal(ckpt, ckpt_copy), "verify must not modify the checkpoint"
    for b in range(B):
        for hv in range(HV):
            h = hv // (HV // H)
            sl = slice(b * Q, (b + 1) * Q)
            out, c = _triangular_reference(
                ckpt[b + 1, hv], q[0, sl, h], k[0, sl, h], v[0, sl, hv], g[sl, hv], beta[sl, hv], 0.37
            )
            torch.testing.assert_close(res.out[sl, hv], out, rtol=1e-11, atol=1e-12)
            torch.testing.assert_close(res.correction[b, hv], c, rtol=1e-11, atol=1e-12)
            torch.testing.assert_close(res.decay[b, hv], torch.exp(g[sl, hv]), rtol=0, atol=0)
            assert torch.equal(res.key[b, h], k[0, sl, h])


def test_fold_equals_verify_prefix_state_and_closed_form():
    B, H, HV, K, V, Q = 2, 1, 2, 8, 8, 5
    T = B * Q
    q, k, v, g, beta = _random_case(7, T, H, HV, K, V)
    ckpt = torch.randn(B + 1, HV, V, K, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    res = O.oracle_verify(q, k, v, g, beta, ckpt, torch.arange(B + 1) * Q, torch.arange(1, B + 1), Q, keep_states=True)
    for n in range(Q + 1):
        pages = torch.arange(1, B + 1)
        folded = O.oracle_fold(
            [ckpt], [res.correction], [res.key], [res.decay],
            source=pages, lengths=torch.full((B,), n), final=pages,
            boundary=torch.zeros(B, dtype=torch.long), boundary_len=torch.zeros(B, dtype=torch.long),
            rows=B, num_blocks=B + 1, record_rows=B,
        )[0]
        for b in range(B):
            want = ckpt[b + 1] if n == 0 else res.states[n - 1][b]
            if n == 0:
                assert torch.equal(folded[b + 1], want)
            torch.testing.assert_close(folded[b + 1], want, rtol=1e-12, atol=1e-12)
            key_hv = res.key[b][torch.arange(HV) // (HV // H)]
            closed = O.fold_closed_form(ckpt[b + 1], res.correction[b], key_hv, res.decay[b], n)
            torch.testing.assert_close(folded[b + 1], closed, rtol=1e-11, atol=1e-12)


def test_verify_null_padding_and_record_rows():
    B, H, HV, K, V, Q = 4, 1, 2, 8, 4, 3
    T = B * Q
    q, k, v, g, beta = _random_case(11, T, H, HV, K, V)
    ckpt = torch.randn(5, HV, V, K, dtype=torch.float64)
    # row 1 null (-1), row 2 out of range (>= NB), row 3 short (qlen 1) and beyond record_rows
    idx = torch.tensor([1, -1, 9, 3])
    qsl = torch.tensor([0, 3, 6, 9, 10])
    res = O.oracle_verify(q, k, v, g, beta, ckpt, qsl, idx, Q, record_rows=3)
    assert torch.count_nonzero(res.out[3:9]) == 0  # null rows emit zeros
    assert bool(res.out_written[3:9].all())
    assert not bool(res.record_written[1].any()) and not bool(res.record_written[2].any())
    assert bool(res.record_written[0].all())
    assert not bool(res.out_written[10:].any())  # tokens beyond the row's window are untouched
    assert bool(res.out_written[9].all())  # row 3 token 0 computed but not recorded (row >= R)


def test_in_kernel_l2norm_matches_prenormalised_inputs():
    B, H, HV, K, V, Q = 2, 2, 4, 16, 8, 4
    T = B * Q
    gen = torch.Generator().manual_seed(5)
    q = torch.randn(1, T, H, K, generator=gen, dtype=torch.float64) * 3
    k = torch.randn(1, T, H, K, generator=gen, dtype=torch.float64) * 3
    v = torch.randn(1, T, HV, V, generator=gen, dtype=torch.float64)
    g = -torch.rand(T, HV, generator=gen, dtype=torch.float64)
    beta = torch.rand(T, HV, generator=gen, dtype=torch.float64)
    ckpt = torch.randn(B + 1, HV, V, K, generator=gen, dtype=torch.float64)
    qsl, idx = torch.arange(B + 1) * Q, torch.arange(1, B + 1)
    a = O.oracle_verify(q, k, v, g, beta, ckpt, qsl, idx, Q, qk_already_normalized=False)
    qn = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6)
    kn = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    b = O.oracle_verify(qn, kn, v, g, beta, ckpt, qsl, idx, Q)
    torch.testing.assert_close(a.out, b.out, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(a.key, b.key, rtol=1e-12, atol=1e-12)


def test_record_bytes_closed_form():
    rb = GOLD["record_bytes"]
    args = [rb[k] for k in ("rows", "num_layers", "num_value_heads", "num_key_heads", "window", "key_dim", "value_dim")]
    assert O.record_geometry_bytes(*args, 4) == rb["expected_fp32_key_mib"] * 1024**2
    assert O.record_geometry_bytes(*args, 2) == rb["expected_bf16_key_mib"] * 1024**2


def test_fold_boundary_only_when_distinct_and_within_window():
    ckpt = (torch.arange(4, dtype=torch.float64).reshape(4, 1, 1, 1) + 1) * 10
    corr = torch.ones(1, 1, 4, 1, dtype=torch.float64)
    key = torch.ones(1, 1, 4, 1, dtype=torch.float64)
    dec = torch.full((1, 1, 4), 0.5, dtype=torch.float64)
    # boundary == final: no separate snapshot
    out = _fold_one(ckpt, corr, key, dec, 2, final=2, boundary=2, blen=1)
    assert float(out[2]) == (20 * 0.5 + 1) * 0.5 + 1 and float(out[3]) == 40
    # boundary length beyond n: never reached
    out = _fold_one(ckpt, corr, key, dec, 2, final=2, boundary=3, blen=3)
    assert float(out[3]) == 40
    # a null boundary is ignored
    out = _fold_one(ckpt, corr, key, dec, 2, final=2, boundary=0, blen=1)
    assert float(out[0]) == 10
    # a distinct valid boundary inside the window gets the snapshot after blen tokens
    out = _fold_one(ckpt, corr, key, dec, 2, final=2, boundary=3, blen=1)
    assert float(out[3]) == 20 * 0.5 + 1 and float(out[2]) == (20 * 0.5 + 1) * 0.5 + 1


def test_gating_matches_library_softplus_and_sigmoid():
    gen = torch.Generator().manual_seed(4)
    a = torch.randn(37, 6, generator=gen, dtype=torch.float64) * 8
    b = torch.randn(37, 6, generator=gen, dtype=torch.float64) * 4
    A_log = torch.randn(6, generator=gen, dtype=torch.float64)
    dt_bias = torch.randn(6, generator=gen, dtype=torch.float64)
    for sb, thr in ((1.0, 20.0), (2.0, 5.0)):
        g, beta = O.oracle_gating(a, b, A_log, dt_bias, softplus_beta=sb, softplus_threshold=thr)
        want_g = -torch.exp(A_log)[None, :] * torch.nn.functional.softplus(a + dt_bias, beta=sb, threshold=thr)
        torch.testing.assert_close(g, want_g, rtol=1e-13, atol=1e-13)
        torch.testing.assert_close(beta, torch.sigmoid(b), rtol=1e-14, atol=1e-14)


def test_gating_hand_values():
    # softplus(0) = ln 2, beta(0) = 1/2; above the threshold softplus is the identity.
    z = torch.zeros(1, 2, dtype=torch.float64)
    g, beta = O.oracle_gating(z, z, torch.zeros(2, dtype=torch.float64), torch.tensor([0.0, 25.0], dtype=torch.float64))
    assert abs(float(g[0, 0]) + math.log(2.0)) < 1e-15 and float(g[0, 1]) == -25.0
    assert float(beta[0, 0]) == 0.5

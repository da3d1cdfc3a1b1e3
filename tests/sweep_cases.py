"""Seeded random configurations for the parity sweeps: every option of the
verify and commit entry points drawn together, inside the limits the host
API accepts (K <= 256 and a multiple of the 16-byte chunk's element count,
Q <= 8, GQA ratio dividing the value heads). The same draws feed the CPU test
that checks each case passes the host validation and the GPU tests that
check it against the oracle.
"""

from __future__ import annotations

import os
import random

import torch

# GDN_SWEEP_SCALE=k draws k times as many cases (the default suite keeps 1).
_SCALE = max(1, int(os.environ.get("GDN_SWEEP_SCALE", "1")))
VERIFY_CASES = 24 * _SCALE
COMMIT_CASES = 16 * _SCALE
DEFERRED_CASES = 6 * _SCALE
COORDINATOR_CASES = 6 * _SCALE
GATED_CASES = 6 * _SCALE


def verify_case(i: int) -> dict:
    rng = random.Random(7001 + i)
    state_dtype = rng.choice([torch.float32, torch.float32, torch.bfloat16, torch.float16])
    chunk = 4 if state_dtype == torch.float32 else 8
    K = rng.choice([k for k in (16, 32, 40, 64, 96, 128, 136, 192, 256) if k % chunk == 0])
    V = rng.choice([8, 16, 48, 64, 100, 128, 192, 256])
    H = rng.choice([1, 2, 3])
    HV = H * rng.choice([1, 2, 4])
    Q = rng.randint(1, 8)
    B = rng.randint(1, 7)
    qlens = [rng.randint(0, Q) for _ in range(B)]
    qlens[0] = max(qlens[0], 1)  # at least one token (the empty batch has a test of its own)
    rows = list(range(B))
    rng.shuffle(rows)
    null_rows = tuple(rows[: rng.randint(0, 1)])
    oob_rows = tuple(rows[1 : 1 + rng.randint(0, 1)])
    act = rng.choice([torch.bfloat16, torch.float16, torch.float32])
    packed = rng.random() < 0.25
    l2norm = rng.random() < 0.25
    key_dtype = None
    if not packed and not l2norm:
        key_dtype = rng.choice([None, torch.float32])
    return dict(
        problem=dict(B=B, H=H, HV=HV, K=K, V=V, Q=Q, qlens=qlens, seed=100 + i, act=act, state_dtype=state_dtype,
                     null_rows=null_rows, oob_rows=oob_rows, normalise=not l2norm),
        run=dict(key_dtype=key_dtype, record_rows=rng.randint(max(1, B - 2), B), packed=packed, l2norm=l2norm,
                 idx_dtype=rng.choice([torch.int32, torch.int64]), column_view=rng.random() < 0.5,
                 out_dtype=rng.choice([None, torch.float32]),
                 beta_dtype=rng.choice([torch.float32, act]), scale=rng.choice([None, 0.25])),
    )


def commit_case(i: int) -> dict:
    rng = random.Random(9001 + i)
    state_dtype = rng.choice([torch.float32, torch.float32, torch.bfloat16, torch.float16])
    chunk = 4 if state_dtype == torch.float32 else 8
    K = rng.choice([k for k in (16, 32, 40, 64, 96, 128, 136, 192, 256) if k % chunk == 0])
    V = rng.choice([8, 16, 48, 64, 100, 128, 192, 256])
    H = rng.choice([1, 2, 3])
    HV = H * rng.choice([1, 2, 4])
    Q = rng.randint(1, 8)
    B = rng.randint(2, 9)
    packed = rng.random() < 0.3
    key_dtype = torch.float32 if packed else rng.choice([torch.bfloat16, torch.float16, torch.float32])
    return dict(B=B, H=H, HV=HV, K=K, V=V, Q=Q, L=rng.randint(1, 3), align=rng.random() < 0.5, seed=500 + i,
                Bk=rng.choice([Q, 8, 16]) if Q <= 8 else 16, key_dtype=key_dtype, state_dtype=state_dtype,
                packed=packed, qlens=[rng.randint(0, Q) for _ in range(B)], padded=rng.randint(0, 1))


def deferred_case(i: int) -> dict:
    """A carried decode-loop workload for the deferred flow: head dims, GQA
    ratio, window, dtypes, rows, layers, steps and block size drawn together."""
    rng = random.Random(9001 + i)
    state = rng.choice([torch.float32, torch.float32, torch.bfloat16, torch.float16])
    chunk = 4 if state == torch.float32 else 8
    K = rng.choice([k for k in (16, 32, 40, 64, 96, 128, 136, 192, 256) if k % chunk == 0])
    V = rng.choice([8, 16, 40, 64, 100, 128, 192, 256])
    H = rng.choice([1, 2, 3])
    HV = H * rng.choice([1, 2, 4])
    Q = rng.randint(1, 8)
    return dict(K=K, V=V, Q=Q, H=H, HV=HV,
                act=rng.choice([torch.bfloat16, torch.float16, torch.float32]), state=state,
                rows=rng.randint(2, 12), layers=rng.randint(1, 3), steps=rng.randint(2, 4),
                block_size=rng.choice([b for b in (4, 8, 16) if b >= Q]),  # a block covers one window
                seed=rng.randint(0, 10_000),
                empty_row=rng.random() < 0.3,
                move=rng.random() < 0.5)


def coordinator_case(i: int) -> dict:
    """One grouped commit through the coordinator: 1-7 cache groups on the
    same rows, each with its own layer count and record layout (typed keys in
    the activation dtype or FP32, or packed records), head dims, window and
    state dtype shared by the step."""
    rng = random.Random(11001 + i)
    state = rng.choice([torch.float32, torch.float32, torch.bfloat16, torch.float16])
    chunk = 4 if state == torch.float32 else 8
    K = rng.choice([k for k in (16, 32, 40, 64, 96, 128, 136, 192, 256) if k % chunk == 0])
    H = rng.choice([1, 2, 3])
    n = rng.randint(1, 7)
    return dict(n_groups=n, align=rng.random() < 0.6, B=rng.randint(2, 8), H=H, HV=H * rng.choice([1, 2, 4]), K=K,
                V=rng.choice([8, 16, 40, 64, 100, 128]), Q=rng.randint(1, 8), state=state,
                layers=[rng.randint(1, 3) for _ in range(n)],
                layouts=[rng.choice(["bf16", "bf16", "f32", "packed"]) for _ in range(n)],
                seed=rng.randint(0, 10_000))


def gated_case(i: int) -> dict:
    """The gated verify (gating and q/k L2 norm fused in): head dims, GQA
    ratio, window, ragged / null / out-of-range rows, activation and state
    dtypes, raw a / b in the activation dtype or FP32, A_log / dt_bias in any
    float dtype."""
    rng = random.Random(13001 + i)
    state = rng.choice([torch.float32, torch.float32, torch.bfloat16, torch.float16])
    chunk = 4 if state == torch.float32 else 8
    K = rng.choice([k for k in (16, 32, 40, 64, 96, 128, 136, 192, 256) if k % chunk == 0])
    H = rng.choice([1, 2, 3])
    Q = rng.randint(1, 8)
    B = rng.randint(1, 7)
    qlens = [rng.randint(0, Q) for _ in range(B)]
    qlens[0] = max(qlens[0], 1)
    rows = list(range(B))
    rng.shuffle(rows)
    act = rng.choice([torch.bfloat16, torch.float16, torch.float32])
    return dict(B=B, H=H, HV=H * rng.choice([1, 2, 4]), K=K, V=rng.choice([8, 16, 48, 64, 100, 128, 192, 256]), Q=Q,
                qlens=qlens, null_rows=tuple(rows[: rng.randint(0, 1)]), oob_rows=tuple(rows[1: 1 + rng.randint(0, 1)]),
                act=act, state=state, ab=rng.choice([act, torch.float32]),
                param=rng.choice([torch.float32, torch.bfloat16, torch.float16]), seed=rng.randint(0, 10_000))

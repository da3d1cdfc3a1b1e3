"""CPU oracle for the RecoverSSM verify / plan / fold / conv-compaction path.

TEST INFRASTRUCTURE ONLY. Nothing in the shipped package imports this module:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and only as the checker (or as the timed CPU baseline),
never as the thing measured on the GPU.

Each function restates the reference algorithm in plain torch on the CPU,
batched over rows and heads and sequential over the speculative tokens, in the
dtype the caller asks for (float64 for parity, float32 for the CPU timing leg).
Citations are ``file:line`` inside the reference plugin
(``plugin/gdn_recoverssm_ascend``):

* ``oracle_verify``        -> kernels.py:554-697 (verify body), :700-856 (host)
* ``oracle_plan_single``   -> kernels.py:975-1072 (``_prepare_commit_plan_kernel``)
* ``oracle_plan_grouped``  -> grouped_commit.py:109-222 (``_grouped_plan_kernel``)
* ``oracle_fold``          -> kernels.py:1222-1324, grouped_commit.py:377-480
* ``oracle_conv_compact``  -> kernels.py:1104-1169, grouped_commit.py:256-322
* ``oracle_publish``       -> grouped_commit.py:531-560
* ``oracle_gating``        -> docs/reference/recoverssm_gdn_upstream.py:135-151 (fused gating
  of the gated verify; vLLM's ``fused_gdn_gating`` formula, called at spec_forward.py:91-93)

How each part is pinned (see tests/test_oracle_*.py):

* verify: hand-computed known answers (plugin/tests/test_ascendc_selftest_oracle.py:16-36),
  the independent closed form S_t = g_t S_0 + sum_s (g_t/g_s) c_s k_s^T evaluated
  in float64, the "checkpoint is read-only" and "null rows emit zeros" invariants;
* fold: the known answers of test_ascendc_selftest_oracle.py:39-53 and
  test_math_oracle.py:206-235, "fold(n) == verify state after n tokens",
  "n == 0 is bit-identical";
* plan: the (C, Bk, n, W) tuples of test_math_oracle.py:238-250 and the grouped
  vectors of test_grouped_commit.py:173-292 / :626-637, plus a brute-force
  comparison against a per-token simulation of block ownership;
* conv compaction: index identities against hand-built histories;
* publish: the persistent-column vectors of test_grouped_commit.py:173-253;
* gating: torch's own ``softplus(x, beta, threshold)`` and ``sigmoid`` (library
  routines with the same switch-over rule) and hand values (softplus(0) = ln 2,
  the linear branch above the threshold).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

# vLLM reserves physical page 0 as the null block (csrc/ops.cpp:97).
NULL_BLOCK_ID = 0


# ---------------------------------------------------------------------------
# Verify
# ---------------------------------------------------------------------------


@dataclass
class VerifyResult:
    out: torch.Tensor  # [T, HV, V] compute dtype (caller rounds to bf16)
    correction: torch.Tensor  # [R, HV, Q, V]
    key: torch.Tensor  # [R, H, Q, K] (values as written; packed: [R, HV, Q, K])
    decay: torch.Tensor  # [R, HV, Q]
    out_written: torch.Tensor  # [T, HV] bool: which (token, head) rows the kernel writes
    record_written: torch.Tensor  # [R, Q] bool: which record slots the kernel writes
    states: list  # per token t: [B, HV, V, K] state after token t (valid rows)


def oracle_verify(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    checkpoint: torch.Tensor,
    query_start_loc: torch.Tensor,
    state_indices: torch.Tensor,
    spec_query_len: int,
    *,
    scale: float | None = None,
    qk_already_normalized: bool = True,
    record_rows: int | None = None,
    packed_key_per_value_head: bool = False,
    dtype: torch.dtype = torch.float64,
    keep_states: bool = False,
) -> VerifyResult:
    """Restates kernels.py:554-697 for every (row, value head) at once.

    Shapes follow the host API (kernels.py:717-727): q, k ``[1, T, H, K]``;
    v ``[1, T, HV, V]``; g, beta ``[T, HV]`` (any shape with T*HV elements);
    checkpoint ``[NB, HV, V, K]``; query_start_loc ``[B+1]``; state_indices ``[B]``.

    Per token t of row b (kernels.py:608-659):
      decay = exp(g); q <- q*scale; S' = S*decay; c = (v - S'k)*beta;
      S = S' + c k^T; o = S q. Invalid tokens (t >= query_len, token outside
      [0, T)) leave S unchanged and write nothing (kernels.py:612, :653).
    Null / out-of-range slots write zeros to ``out`` for t < query_len and never
    touch the records (kernels.py:569-583). Records are row-indexed and written
    only for ``b < record_rows`` (kernels.py:594-607). The key record holds the raw
    (already normalised) k, or the in-kernel normalised k when
    ``qk_already_normalized`` is False (kernels.py:677).
    """
    _, T, H, K = q.shape
    HV, V = v.shape[-2], v.shape[-1]
    Q = int(spec_query_len)
    B = int(state_indices.shape[0])
    NB = int(checkpoint.shape[0])
    R = int(record_rows if record_rows is not None else B)
    ratio = HV // H
    if scale is None:
        scale = K**-0.5
    qf = q.reshape(T, H, K).to(dtype)
    kf = k.reshape(T, H, K).to(dtype)
    vf = v.reshape(T, HV, V).to(dtype)
    gf = g.reshape(T, HV).to(dtype)
    bf = beta.reshape(T, HV).to(dtype)
    if not qk_already_normalized:
        # kernels.py:645-648: x * rsqrt(sum(x*x) + 1e-6)
        qf = qf * torch.rsqrt((qf * qf).sum(-1, keepdim=True) + 1e-6)
        kf = kf * torch.rsqrt((kf * kf).sum(-1, keepdim=True) + 1e-6)
    key_src = kf if not qk_already_normalized else k.reshape(T, H, K)
    qs = qf * scale

    qsl = query_start_loc.to(torch.int64)
    idx = state_indices.to(torch.int64)
    bos = qsl[:B]
    eos = qsl[1 : B + 1]
    qlen = eos - bos
    null = (idx <= NULL_BLOCK_ID) | (idx >= NB)

    out = torch.zeros(T, HV, V, dtype=dtype)
    out_written = torch.zeros(T, HV, dtype=torch.bool)
    key_heads = HV if packed_key_per_value_head else H
    correction = torch.zeros(R, HV, Q, V, dtype=dtype)
    key_rec = torch.zeros(R, key_heads, Q, K, dtype=key_src.dtype if qk_already_normalized else dtype)
    decay_rec = torch.zeros(R, HV, Q, dtype=dtype)
    record_written = torch.zeros(R, Q, dtype=torch.bool)

    safe_idx = torch.where(null, torch.zeros_like(idx), idx)
    state = checkpoint.to(dtype)[safe_idx].clone()  # [B, HV, V, K]
    head_of = torch.arange(HV) // ratio
    states = []
    for t in range(Q):
        tok = bos + t
        in_range = (t < qlen) & (tok >= 0) & (tok < T)
        tok_c = tok.clamp(0, max(T - 1, 0))
        if T == 0:
            break
        valid = in_range & ~null  # rows whose state advances
        # Null rows: zero outputs (kernels.py:574-583).
        zero_rows = in_range & null
        if bool(zero_rows.any()):
            out[tok_c[zero_rows]] = 0
            out_written[tok_c[zero_rows]] = True
        if not bool(valid.any()):
            if keep_states:
                states.append(state.clone())
            continue
        qt = qs[tok_c][:, head_of, :]  # [B, HV, K]
        kt = kf[tok_c][:, head_of, :]
        vt = vf[tok_c]  # [B, HV, V]
        decay = torch.exp(gf[tok_c])  # [B, HV]
        bt = bf[tok_c]
        new_state = state * decay[:, :, None, None]
        corr = (vt - (new_state * kt[:, :, None, :]).sum(-1)) * bt[:, :, None]
        new_state = new_state + corr[:, :, :, None] * kt[:, :, None, :]
        m = valid[:, None, None, None]
        state = torch.where(m, new_state, state)
        o = (state * qt[:, :, None, :]).sum(-1)  # [B, HV, V]
        vr = valid.nonzero().flatten()
        out[tok_c[vr]] = o[vr]
        out_written[tok_c[vr]] = True
        rec = vr[vr < R]
        if rec.numel():
            correction[rec, :, t] = corr[rec]
            decay_rec[rec, :, t] = decay[rec]
            record_written[rec, t] = True
            ksrc = key_src[tok_c[rec]]  # [n, H, K]
            if packed_key_per_value_head:
                key_rec[rec, :, t] = ksrc[:, head_of, :].to(key_rec.dtype)
            else:
                key_rec[rec, :, t] = ksrc.to(key_rec.dtype)
        if keep_states:
            states.append(state.clone())
    return VerifyResult(out, correction, key_rec, decay_rec, out_written, record_written, states)


# ---------------------------------------------------------------------------
# Commit plan (integer, bit-exact)
# ---------------------------------------------------------------------------


def _floordiv(a: int, b: int) -> int:
    """Integer division as the Triton kernels do it on int32/int64 (C truncation).

    Only reached with non-negative operands for every value that is stored
    unmasked (the plan clamps with max(.., 0) first), so floor and truncation
    agree there; negative ``num_computed`` only feeds masked values.
    """
    q = abs(a) // abs(b)
    return q if (a >= 0) == (b >= 0) else -q


@dataclass
class PlanRow:
    commit_len: int
    final: int
    boundary: int
    boundary_len: int
    valid: int
    col: int
    source: int


def oracle_plan_row(
    *,
    source: int,
    accepted: int,
    bos: int,
    eos: int,
    spec_query_len: int,
    num_blocks: int,
    align: bool,
    table_row: list | None = None,
    num_computed: int | None = None,
    block_size: int | None = None,
    grouped: bool,
) -> PlanRow:
    """One plan row: kernels.py:975-1072 (single) / grouped_commit.py:147-207.

    ``grouped`` selects the grouped kernel's extra canonicalisation: the plan
    stores the source (NULL when invalid) and an invalid boundary becomes NULL
    (grouped_commit.py:194-204), and a negative ``num_computed`` masks the
    boundary load (grouped_commit.py:183-187).
    """
    Q = spec_query_len
    qlen = eos - bos
    count = min(max(accepted, 0), qlen)
    count = min(count, Q)
    final = source
    boundary = NULL_BLOCK_ID
    boundary_len = 0
    col = 0
    computed_ok = True
    if align:
        W = len(table_row)
        C = int(num_computed)
        computed_ok = C >= 0
        position = C + count
        col = min(_floordiv(max(position - 1, 0), block_size), W - 1)
        final = int(table_row[col])
        next_boundary = (_floordiv(C, block_size) + 1) * block_size
        crossed = position >= next_boundary
        boundary_len = next_boundary - C
        boundary_col = _floordiv(next_boundary, block_size) - 1
        load = crossed and 0 <= boundary_col < W
        if grouped:
            load = load and computed_ok
        boundary = int(table_row[boundary_col]) if load else NULL_BLOCK_ID
    geometry = bos >= 0 and bos <= eos and qlen <= Q
    valid = (
        geometry
        and NULL_BLOCK_ID < source < num_blocks
        and NULL_BLOCK_ID < final < num_blocks
        and count > 0
        and count <= qlen
        and computed_ok
    )
    boundary_ok = NULL_BLOCK_ID < boundary < num_blocks
    if align:
        boundary_len = boundary_len if boundary_ok else 0
    if grouped:
        boundary = boundary if boundary_ok else NULL_BLOCK_ID
    return PlanRow(
        commit_len=count if valid else 0,
        final=final if valid else NULL_BLOCK_ID,
        boundary=boundary if valid else NULL_BLOCK_ID,
        boundary_len=boundary_len if valid else 0,
        valid=int(valid),
        col=col,
        source=source if valid else NULL_BLOCK_ID,
    )


def _i(x, i, stride=1):
    return int(x.reshape(-1)[i * stride]) if x.dim() else int(x)


def oracle_plan_single(
    num_accepted,
    state_indices,
    query_start_loc,
    *,
    spec_query_len: int,
    num_blocks: int,
    request_indices=None,
    block_table=None,
    num_computed=None,
    block_size=None,
) -> dict:
    """kernels.py:975-1072 for every row; returns int32 arrays keyed like the context."""
    rows = int(state_indices.shape[0])
    align = block_table is not None
    res = {k: [] for k in ("commit_lens", "final", "boundary", "boundary_len", "align_valid", "align_col")}
    for r in range(rows):
        request = int(request_indices[r]) if request_indices is not None else r
        pr = oracle_plan_row(
            source=int(state_indices[r]),
            accepted=int(num_accepted[request]),
            bos=int(query_start_loc[r]),
            eos=int(query_start_loc[r + 1]),
            spec_query_len=spec_query_len,
            num_blocks=num_blocks,
            align=align,
            table_row=block_table[request].tolist() if align else None,
            num_computed=int(num_computed[request]) if align else None,
            block_size=block_size,
            grouped=False,
        )
        res["commit_lens"].append(pr.commit_len)
        res["final"].append(pr.final)
        res["boundary"].append(pr.boundary)
        res["boundary_len"].append(pr.boundary_len)
        res["align_valid"].append(pr.valid)
        res["align_col"].append(pr.col)
    return {k: torch.tensor(v, dtype=torch.int32) for k, v in res.items()}


def oracle_plan_grouped(
    sampled,
    groups: list,
    *,
    spec_query_len: int,
    capacity: int,
    rows: int,
    align: bool,
    idx_mapping=None,
    persistent_cols=None,
    persistent_accepted=None,
    publish_align: bool = True,
) -> dict:
    """grouped_commit.py:109-222. ``groups`` is a list of dicts with keys
    state_indices, query_start_loc, request_indices, block_table, num_computed,
    block_size, num_blocks. Returns the seven plan arrays of size
    ``len(groups) * capacity`` (rows beyond ``rows`` are left at -12345 so that a
    test can see the kernel never writes them) and applies the publication to
    copies of the persistent arrays."""
    G = len(groups)
    size = G * capacity
    plan = {k: [-12345] * size for k in ("source", "length", "final", "boundary", "boundary_len", "valid", "col")}
    cols = persistent_cols.clone() if persistent_cols is not None else None
    acc = persistent_accepted.clone() if persistent_accepted is not None else None
    for row in range(rows):
        all_valid = True
        shared_col = -1
        shared_request = -1
        for gi, grp in enumerate(groups):
            request = int(grp["request_indices"][row])
            pr = oracle_plan_row(
                source=int(grp["state_indices"][row]),
                accepted=int(sampled[request]),
                bos=int(grp["query_start_loc"][row]),
                eos=int(grp["query_start_loc"][row + 1]),
                spec_query_len=spec_query_len,
                num_blocks=int(grp["num_blocks"]),
                align=align,
                table_row=grp["block_table"][request].tolist() if align else None,
                num_computed=int(grp["num_computed"][request]) if align else None,
                block_size=int(grp["block_size"]) if align else None,
                grouped=True,
            )
            off = gi * capacity + row
            plan["source"][off] = pr.source
            plan["length"][off] = pr.commit_len
            plan["final"][off] = pr.final
            plan["boundary"][off] = pr.boundary
            plan["boundary_len"][off] = pr.boundary_len
            plan["valid"][off] = pr.valid
            plan["col"][off] = pr.col
            if gi == 0:
                shared_col, shared_request = pr.col, request
            else:
                all_valid = all_valid and pr.col == shared_col and request == shared_request
            all_valid = all_valid and bool(pr.valid)
        if align and publish_align and cols is not None:
            slot = int(idx_mapping[shared_request])
            if all_valid and slot >= 0:
                cols[slot] = shared_col
                acc[slot] = 1
    out = {k: torch.tensor(v, dtype=torch.int32) for k, v in plan.items()}
    out["persistent_cols"] = cols
    out["persistent_accepted"] = acc
    return out


def oracle_publish(buckets: list, request_indices, idx_mapping, persistent_cols, persistent_accepted, rows: int):
    """grouped_commit.py:531-560: AND-valid publication across buckets.

    ``buckets`` is a list of (valid[int32], col[int32], capacity, group_count).
    """
    cols = persistent_cols.clone()
    acc = persistent_accepted.clone()
    first_cols = buckets[0][1]
    for row in range(rows):
        valid = True
        shared_col = int(first_cols[row])
        for valid_arr, col_arr, capacity, group_count in buckets:
            for gi in range(group_count):
                off = gi * capacity + row
                valid = valid and int(valid_arr[off]) != 0
                valid = valid and int(col_arr[off]) == shared_col
        request = int(request_indices[row])
        slot = int(idx_mapping[request])
        if valid and slot >= 0:
            cols[slot] = shared_col
            acc[slot] = 1
    return cols, acc


# ---------------------------------------------------------------------------
# Fold
# ---------------------------------------------------------------------------


def oracle_fold(
    checkpoints: list,
    corrections: list,
    keys: list,
    decays: list,
    *,
    source,
    lengths,
    final,
    boundary,
    boundary_len,
    layer_groups=None,
    plan_capacity: int | None = None,
    rows: int,
    num_blocks: int,
    record_rows: int,
    dtype: torch.dtype = torch.float64,
    out_dtype: torch.dtype | None = None,
) -> list:
    """kernels.py:1222-1324 / grouped_commit.py:377-480 for every layer.

    Per (layer l, row b, value head): skipped unless the source and final pages
    are valid, n > 0 and b < record_rows (kernels.py:1232-1242). Otherwise
    h = checkpoint[source] (one load, before any store), then for t < n
    h = h*decay_t + c_t k_t^T, storing the boundary snapshot when t+1 equals the
    boundary length and the boundary page is valid and differs from the final
    page (kernels.py:1251-1256, :1313-1319); finally checkpoint[final] = h.
    Returns new checkpoint tensors (inputs are not modified). ``source`` etc. are
    plan arrays indexed by ``layer_groups[l] * plan_capacity + b``.
    """
    L = len(checkpoints)
    if layer_groups is None:
        layer_groups = [0] * L
    cap = plan_capacity if plan_capacity is not None else rows
    results = []
    for li in range(L):
        ckpt = checkpoints[li]
        sdt = out_dtype or ckpt.dtype
        new = ckpt.clone()
        HV = ckpt.shape[1]
        H = keys[li].shape[1]
        ratio = HV // H
        head_of = torch.arange(HV) // ratio
        base = int(layer_groups[li]) * cap
        # Gather the work: valid rows in this layer.
        todo = []
        for b in range(rows):
            p = base + b
            src = int(source[p])
            n = int(lengths[p])
            fin = int(final[p])
            if not (NULL_BLOCK_ID < src < num_blocks and n > 0 and NULL_BLOCK_ID < fin < num_blocks and b < record_rows):
                continue
            todo.append((b, src, n, fin, int(boundary[p]), int(boundary_len[p])))
        if not todo:
            results.append(new)
            continue
        bs = torch.tensor([t[0] for t in todo])
        srcs = torch.tensor([t[1] for t in todo])
        h = ckpt[srcs].to(dtype)  # every load happens before any store
        ns = torch.tensor([t[2] for t in todo])
        nmax = int(ns.max())
        corr = corrections[li][bs].to(dtype)  # [n, HV, Q, V]
        key = keys[li][bs].to(dtype)[:, head_of]  # [n, HV, Q, K]
        dec = decays[li][bs].to(dtype)  # [n, HV, Q]
        snaps = {}
        for t in range(nmax):
            active = (ns > t)[:, None, None, None]
            upd = h * dec[:, :, t, None, None] + corr[:, :, t, :, None] * key[:, :, t, None, :]
            h = torch.where(active, upd, h)
            for j, (_, _, n, fin, bidx, blen) in enumerate(todo):
                store_b = NULL_BLOCK_ID < bidx < num_blocks and bidx != fin and blen > 0
                if store_b and t + 1 == blen and t < n:
                    snaps[j] = (bidx, h[j].clone())
        for j, (bidx, hb) in snaps.items():
            new[bidx] = hb.to(sdt)
        for j, (_, _, _, fin, _, _) in enumerate(todo):
            new[fin] = h[j].to(sdt)
        results.append(new)
    return results


def fold_closed_form(s0, corr, key, decay, n):
    """Independent closed form S_n = G_n S_0 + sum_t (G_n/G_t) c_t k_t^T.

    docs/GDN-RecoverSSM-实现方案.md:93-99. Shapes: s0 [HV,V,K]; corr [HV,Q,V];
    key [HV,Q,K] (already expanded over value heads); decay [HV,Q]. float64.
    """
    s0 = s0.double()
    if n == 0:
        return s0.clone()
    d = decay.double()[:, :n]
    gam = torch.cumprod(d, dim=1)  # G_1..G_n
    gn = gam[:, -1]
    acc = gn[:, None, None] * s0
    for t in range(n):
        w = gn / gam[:, t]
        acc = acc + w[:, None, None] * corr.double()[:, t, :, None] * key.double()[:, t, None, :]
    return acc


# ---------------------------------------------------------------------------
# Conv-state compaction
# ---------------------------------------------------------------------------


def oracle_conv_compact(
    conv_states: list,
    *,
    source,
    lengths,
    final,
    boundary,
    boundary_len,
    history: int,
    num_blocks: int,
    rows: int,
    align: bool,
    layer_groups=None,
    plan_capacity: int | None = None,
) -> list:
    """kernels.py:1104-1169 / grouped_commit.py:256-322.

    conv state is ``[blocks, dim, window]`` (dim-first view). For a row with a
    valid final page and n > 0: final[:, :hist] = src[:, n-1 : n-1+hist]; in
    align mode, when the boundary page is valid,
    boundary[:, :hist] = src[:, blen-1 : blen-1+hist]. Both reads use the
    original source (all loads precede the stores of the same tile).
    """
    L = len(conv_states)
    if layer_groups is None:
        layer_groups = [0] * L
    cap = plan_capacity if plan_capacity is not None else rows
    out = []
    for li in range(L):
        cs = conv_states[li]
        new = cs.clone()
        base = int(layer_groups[li]) * cap
        pending = []
        for b in range(rows):
            p = base + b
            src = int(source[p])
            n = int(lengths[p])
            fin = int(final[p])
            if not (src > NULL_BLOCK_ID and n != 0 and NULL_BLOCK_ID < fin < num_blocks):
                continue
            fv = cs[src, :, n - 1 : n - 1 + history].clone()
            bv = None
            bidx = int(boundary[p])
            if align and NULL_BLOCK_ID < bidx < num_blocks:
                blen = int(boundary_len[p])
                bv = cs[src, :, blen - 1 : blen - 1 + history].clone()
            pending.append((fin, fv, bidx, bv))
        for fin, fv, bidx, bv in pending:
            if bv is not None:
                new[bidx, :, :history] = bv
            new[fin, :, :history] = fv
        out.append(new)
    return out


# ---------------------------------------------------------------------------
# Fused gating (gated verify)
# ---------------------------------------------------------------------------


def oracle_gating(a, b, A_log, dt_bias, *, softplus_beta: float = 1.0, softplus_threshold: float = 20.0,
                  dtype: torch.dtype = torch.float64):
    """docs/reference/recoverssm_gdn_upstream.py:135-151 for every token and head.

    a, b: [T, HV] raw gate projections; A_log, dt_bias: [HV]. Returns
    (g, beta) with g = -exp(A_log) * softplus(a + dt_bias), where
    softplus(x) = log(1 + exp(sb*x)) / sb if sb*x <= threshold else x, and
    beta = sigmoid(b), in ``dtype``.
    """
    x = a.to(dtype) + dt_bias.to(dtype)[None, :]
    bx = softplus_beta * x
    sp = torch.where(bx <= softplus_threshold, torch.log(1 + torch.exp(bx)) / softplus_beta, x)
    g = -torch.exp(A_log.to(dtype))[None, :] * sp
    beta = 1 / (1 + torch.exp(-b.to(dtype)))
    return g, beta


# ---------------------------------------------------------------------------
# Byte model and helpers
# ---------------------------------------------------------------------------


def record_geometry_bytes(rows, num_layers, num_value_heads, num_key_heads, window, key_dim, value_dim, key_bytes):
    """kernels.py:258-294 closed form (bytes of one step's typed records)."""
    return rows * num_layers * window * (num_value_heads * value_dim * 4 + num_key_heads * key_dim * key_bytes + num_value_heads * 4)


def l2_normalise(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """FLA l2norm_fwd semantics: x * rsqrt(sum(x^2) + eps) along the last dim."""
    xf = x.float()
    return xf * torch.rsqrt((xf * xf).sum(-1, keepdim=True) + eps)


def rel_err_norm(got: torch.Tensor, want: torch.Tensor) -> float:
    got = got.double()
    want = want.double()
    den = max(float(want.norm()), 1e-30)
    return float((got - want).norm()) / den


def max_abs_rel(got: torch.Tensor, want: torch.Tensor) -> float:
    """max |got - want| divided by max |want| (the state's infinity norm)."""
    got = got.double()
    want = want.double()
    den = max(float(want.abs().max()) if want.numel() else 0.0, 1e-30)
    return float((got - want).abs().max()) / den if want.numel() else 0.0


__all__ = [
    "NULL_BLOCK_ID",
    "VerifyResult",
    "oracle_verify",
    "oracle_plan_row",
    "oracle_plan_single",
    "oracle_plan_grouped",
    "oracle_publish",
    "oracle_fold",
    "fold_closed_form",
    "oracle_conv_compact",
    "record_geometry_bytes",
    "l2_normalise",
    "rel_err_norm",
    "max_abs_rel",
    "math",
]

"""RecoverSSM for Gated DeltaNet on AMD Instinct MI355X (gfx950).

Host side of the verify and single-context commit path. The public names,
argument meaning and error behaviour follow the reference plugin's
``gdn_recoverssm_ascend/kernels.py`` so that its callers
(``layer_patch._verify`` and the commit proxy) run unchanged:

* ``gdn_recoverssm_verify`` -- verify a speculative window from the read-only
  checkpoint (reference kernels.py:700-928);
* ``ReplayRecordBuffers`` / ``record_nbytes`` / ``record_geometry_bytes`` -- the
  typed-SoA record layout and its byte accounting (kernels.py:166-294);
* ``GDNRecoverSSMCommitContext`` -- per-layer address tables and the commit
  (kernels.py:1399-2052): the plan and the fold in one launch
  (``gdn_recoverssm_plan_fold``), then the conv compaction that reads the
  stored plan; ``commit_deferred`` plans now and leaves the fold to the next
  verify (``gdn_recoverssm_verify_deferred``).

Every launch goes to the hand-written HIP kernels of ``libgdn_recoverssm_hip.so``
through its C ABI (``_native``). Validation happens before any launch and raises
``ValueError("GDN RecoverSSM: ...")``; a failed launch raises ``RuntimeError``
and is never retried.
"""

from __future__ import annotations

import ctypes
from collections import Counter
from collections.abc import Sequence
from dataclasses import dataclass, field, replace
from typing import Any

import torch

from . import _native as N

# vLLM's physical null page (vllm.v1.attention.backends.utils.NULL_BLOCK_ID).
NULL_BLOCK_ID = 0

# Speculative-window capacity of the kernels (reference kernels.py:101).
MAX_SPEC_QUERY_LEN = 8

# Largest key dimension the verify / fold kernels are instantiated for.
MAX_KEY_DIM = 256

_COUNTS: Counter = Counter()


def counts() -> dict:
    """Launch counters per entry point (``verify``, ``plan``, ``conv``, ``fold``, ``plan_fold``, ``publish``);
    ``prepared_<name>`` counts compile-only preparations."""
    return dict(_COUNTS)


# ---------------------------------------------------------------------------
# Validation helpers (reference kernels.py:143-163)
# ---------------------------------------------------------------------------


def _require(cond: bool, msg: str) -> None:
    """Argument validation that raises ``ValueError`` before any kernel launch."""
    if not cond:
        raise ValueError(f"GDN RecoverSSM: {msg}")


def _ptr_table(tensors: Sequence[torch.Tensor], device, offsets: Sequence[int] | None = None) -> torch.Tensor:
    """int64 device table of data pointers (plus optional byte offsets).

    Pointers with the top bit set are stored with their uint64 bit pattern.
    """
    ptrs = [t.data_ptr() + (offsets[i] if offsets else 0) for i, t in enumerate(tensors)]
    ptrs = [p if p < (1 << 63) else p - (1 << 64) for p in ptrs]
    return torch.tensor(ptrs, dtype=torch.int64, device=device)


# ---------------------------------------------------------------------------
# Record buffers (reference kernels.py:166-294)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class ReplayRecordBuffers:
    """Step-owned typed records; keys are shared by grouped value heads.

    ``correction [rows, HV, Q, V]`` FP32, ``key [rows, H, Q, K]`` in the key
    dtype (an already-normalised BF16/FP16 key keeps its exact input bits),
    ``decay [rows, HV, Q]`` FP32.
    """

    correction: torch.Tensor
    key: torch.Tensor
    decay: torch.Tensor

    @property
    def shape(self) -> tuple[int, int, int, int]:
        rows, heads, window, value_dim = self.correction.shape
        return (rows, heads, window, value_dim + self.key.shape[-1] + 1)

    @property
    def dtype(self):
        return torch.float32

    @property
    def device(self):
        return self.correction.device

    @property
    def num_key_heads(self) -> int:
        return int(self.key.shape[1])

    @property
    def key_dtype(self):
        return self.key.dtype

    @property
    def record_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.correction, self.key, self.decay))

    @classmethod
    def allocate(
        cls,
        rows: int,
        num_value_heads: int,
        num_key_heads: int,
        window: int,
        value_dim: int,
        key_dim: int,
        *,
        device,
        key_dtype=torch.float32,
    ):
        _require(
            rows > 0
            and num_key_heads > 0
            and 0 < window <= MAX_SPEC_QUERY_LEN
            and value_dim > 0
            and key_dim > 0
            and num_value_heads > 0
            and num_value_heads % num_key_heads == 0,
            "record head/row geometry is invalid",
        )
        _require(
            key_dtype in (torch.float16, torch.bfloat16, torch.float32),
            "record keys require FP16, BF16 or FP32",
        )
        return cls(
            torch.zeros((rows, num_value_heads, window, value_dim), dtype=torch.float32, device=device),
            torch.zeros((rows, num_key_heads, window, key_dim), dtype=key_dtype, device=device),
            torch.zeros((rows, num_value_heads, window), dtype=torch.float32, device=device),
        )


def record_nbytes(record: torch.Tensor | ReplayRecordBuffers) -> int:
    return record.record_bytes if isinstance(record, ReplayRecordBuffers) else record.numel() * record.element_size()


def record_geometry_bytes(
    rows: int,
    num_layers: int,
    num_value_heads: int,
    num_key_heads: int,
    window: int,
    key_dim: int,
    value_dim: int,
    key_dtype=torch.float32,
) -> int:
    """Physical bytes of one step's records, with deduplicated keys in their dtype."""
    _require(
        min(rows, num_layers, num_value_heads, num_key_heads, window, key_dim, value_dim) > 0,
        "record geometry must be positive",
    )
    _require(num_value_heads % num_key_heads == 0, "value heads must be a multiple of key heads")
    _require(
        key_dtype in (torch.float16, torch.bfloat16, torch.float32),
        "record keys require FP16, BF16 or FP32",
    )
    key_bytes = 4 if key_dtype == torch.float32 else 2
    return rows * num_layers * window * (num_value_heads * value_dim * 4 + num_key_heads * key_dim * key_bytes + num_value_heads * 4)


# ---------------------------------------------------------------------------
# Launch specs
# ---------------------------------------------------------------------------


@dataclass
class _LaunchSpec:
    """One HIP launch, built once and launched on the current stream.

    ``launch()`` submits it; ``compile_only()`` checks that the AOT library is
    loaded and the entry point exists without touching device memory (the
    kernels are compiled ahead of time). ``name`` is the entry point
    (``verify`` / ``plan`` / ``conv`` / ``fold`` / ``plan_fold`` / ``publish``).
    """

    name: str
    fn: Any
    args: tuple
    device: torch.device
    keepalive: tuple = field(default_factory=tuple)

    def launch(self) -> None:
        stream = N.stream_handle(self.device)
        status = self.fn(*self.args, stream)
        N.check(status, self.name)
        _COUNTS[self.name] += 1

    def compile_only(self) -> "_LaunchSpec":
        N.load()
        _COUNTS["prepared_" + self.name] += 1
        return self


def _lib():
    return N.load()


# ---------------------------------------------------------------------------
# Verify (reference kernels.py:700-928)
# ---------------------------------------------------------------------------


def _aligned16(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0


def gdn_recoverssm_verify(
    g: torch.Tensor,
    beta: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    checkpoint_state: torch.Tensor,
    replay_cache: torch.Tensor | ReplayRecordBuffers,
    query_start_loc: torch.Tensor,
    state_indices: torch.Tensor,
    spec_query_len: int,
    scale: float | None = None,
    qk_already_normalized: bool = True,
    out: torch.Tensor | None = None,
    _collect: list | None = None,
) -> torch.Tensor:
    """Verify a GDN speculative window against its checkpoint without modifying it.

    ``g`` (log-space decay) and ``beta`` in shape [1, T, HV] or [T, HV]; q, k:
    [1, T, H, K]; v: [1, T, HV, V]; checkpoint_state: [blocks, HV, V, K];
    replay_cache: typed ``ReplayRecordBuffers`` or a packed FP32
    [rows, HV, spec_query_len, V + K + 1] tensor. Returns out [1, T, HV, V].
    Reference: kernels.py:700-928.
    """
    return _verify(g, beta, q, k, v, checkpoint_state=checkpoint_state, replay_cache=replay_cache,
                   query_start_loc=query_start_loc, state_indices=state_indices, spec_query_len=spec_query_len,
                   scale=scale, qk_already_normalized=qk_already_normalized, out=out, gating=None, _collect=_collect)


def gdn_recoverssm_verify_gated(
    a: torch.Tensor,
    b: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    A_log: torch.Tensor,
    dt_bias: torch.Tensor,
    checkpoint_state: torch.Tensor,
    replay_cache: torch.Tensor | ReplayRecordBuffers,
    query_start_loc: torch.Tensor,
    state_indices: torch.Tensor,
    spec_query_len: int,
    scale: float | None = None,
    qk_already_normalized: bool = False,
    softplus_beta: float = 1.0,
    softplus_threshold: float = 20.0,
    out: torch.Tensor | None = None,
    _collect: list | None = None,
) -> torch.Tensor:
    """Verify with the gating producer (and, by default, the q/k L2 norm)
    fused in, as the gated verify of docs/reference/recoverssm_gdn_upstream.py:83-151.

    ``a`` and ``b`` are the raw gate projections ([1, T, HV] or [T, HV]);
    ``A_log`` and ``dt_bias`` are [HV]. Inside the kernel, in FP32:
    g = -exp(A_log) * softplus(a + dt_bias) (softplus with ``softplus_beta``
    and ``softplus_threshold``, as vLLM's fused_gdn_gating) and
    beta = sigmoid(b). q and k are raw unless ``qk_already_normalized``. It
    replaces the producers the layer runs before verify
    (spec_forward.py:91-96) and their round trip through memory.
    """
    _require(A_log.ndim == 1 and dt_bias.ndim == 1, "A_log and dt_bias must be one-dimensional")
    _require(A_log.stride(0) == 1 and dt_bias.stride(0) == 1, "A_log and dt_bias must be contiguous")
    _require(float(softplus_beta) > 0.0, "softplus beta must be positive")
    return _verify(a, b, q, k, v, checkpoint_state=checkpoint_state, replay_cache=replay_cache,
                   query_start_loc=query_start_loc, state_indices=state_indices, spec_query_len=spec_query_len,
                   scale=scale, qk_already_normalized=qk_already_normalized, out=out,
                   gating=(A_log, dt_bias, float(softplus_beta), float(softplus_threshold)), _collect=_collect)


@dataclass
class PendingCommit:
    """One layer's commit left for the next verify (``gdn_recoverssm_verify_deferred``).

    ``rows`` (int32, one entry per row of the next batch) names the pending
    row each next row continues, -1 for none. The plan arrays (source page,
    accepted length, final page, boundary page, boundary length; int32) and
    the records are those of the pending step, indexed by pending row, and
    cover ``num_rows`` rows. A next row applies its pending commit only when
    its own state index is that commit's final page; ``records`` are the typed
    records the pending step's verify wrote, and the next verify must write a
    different record buffer.

    ``commit_deferred`` returns commits whose ``rows`` continue every row in
    place (row i of the next batch continues row i); ``continue_pending`` maps
    a next batch given by request ids instead.
    """

    rows: torch.Tensor
    source: torch.Tensor
    lengths: torch.Tensor
    final: torch.Tensor
    boundary: torch.Tensor
    boundary_len: torch.Tensor
    records: "ReplayRecordBuffers"
    num_rows: int = 0


def continue_pending(pending: Sequence[PendingCommit], previous_requests: Sequence, next_requests: Sequence):
    """Re-key one step's pending commits (one per layer) for the next batch.

    ``previous_requests[r]`` identifies the request in row r of the pending
    step and ``next_requests[b]`` the request in row b of the next batch (any
    hashable ids, host-side, as the scheduler holds them). Returns the pending
    commits with a shared row map (next row -> pending row of the same
    request, -1 for a new request) and the sorted pending rows whose request
    is not in the next batch: their commits are applied by no verify, so
    ``flush_deferred(rows=...)`` must fold them before their pages are reused.
    """
    _require(len(pending) > 0, "no pending commits to continue")
    num_rows = int(pending[0].num_rows)
    _require(all(int(p.num_rows) == num_rows for p in pending), "pending commits of one step disagree on their rows")
    _require(len(previous_requests) >= num_rows, "previous request ids do not cover the pending rows")
    where = {}
    for r, req in enumerate(previous_requests[:num_rows]):
        _require(req not in where, f"request {req!r} appears twice in the pending step")
        where[req] = r
    seen = set()
    mapping = []
    for req in next_requests:
        _require(req not in seen, f"request {req!r} appears twice in the next batch")
        seen.add(req)
        mapping.append(where.get(req, -1))
    left = sorted(r for req, r in where.items() if req not in seen)
    rows = torch.tensor(mapping if mapping else [-1], dtype=torch.int32, device=pending[0].rows.device)
    return tuple(replace(p, rows=rows) for p in pending), left


def gdn_recoverssm_verify_deferred(
    g: torch.Tensor,
    beta: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    checkpoint_state: torch.Tensor,
    replay_cache: "ReplayRecordBuffers",
    pending: PendingCommit,
    query_start_loc: torch.Tensor,
    state_indices: torch.Tensor,
    spec_query_len: int,
    scale: float | None = None,
    qk_already_normalized: bool = True,
    out: torch.Tensor | None = None,
    _collect: list | None = None,
) -> torch.Tensor:
    """Verify with the previous step's commit folded in (the deferred commit of
    docs/GDN-RecoverSSM-实现方案.md:515-527; typed records).

    For each row that continues a pending commit (``pending.rows``) and whose
    state index is that commit's final page, the kernel reads the pending
    source page, replays its accepted prefix exactly as the fold does
    (kernels.py:1222-1324), stores the result to the final page (and the
    boundary snapshot), and verifies this step's window from the folded state,
    so every page is read once per step. Other rows verify from
    ``state_indices`` as ``gdn_recoverssm_verify`` does. Pending commits no row
    applies stay pending (see ``continue_pending`` and ``flush_deferred``).
    With no token in the batch the launch still applies the pending commits.
    """
    rec = pending.records
    _require(isinstance(rec, ReplayRecordBuffers), "the deferred commit needs typed record buffers")
    _require(isinstance(replay_cache, ReplayRecordBuffers), "the deferred commit needs typed record buffers")
    _require(
        rec.correction.data_ptr() != replay_cache.correction.data_ptr(),
        "the pending commit's records must not be the records this verify writes",
    )
    batch = state_indices.shape[0]
    num_rows = int(pending.num_rows)
    if num_rows <= 0:
        # Nothing is pending: the ordinary verify.
        return gdn_recoverssm_verify(g, beta, q, k, v, checkpoint_state=checkpoint_state, replay_cache=replay_cache,
                                     query_start_loc=query_start_loc, state_indices=state_indices,
                                     spec_query_len=spec_query_len, scale=scale,
                                     qk_already_normalized=qk_already_normalized, out=out, _collect=_collect)
    plan = (pending.source, pending.lengths, pending.final, pending.boundary, pending.boundary_len)
    _require(
        all(t_.dtype == torch.int32 and t_.ndim == 1 and t_.stride(0) == 1 for t_ in (pending.rows,) + plan),
        "pending arrays must be contiguous one-dimensional int32",
    )
    _require(pending.rows.shape[0] >= batch, "the pending row map does not cover the batch")
    _require(all(t_.shape[0] >= num_rows for t_ in plan), "pending plan arrays do not cover their rows")
    _require(num_rows <= rec.correction.shape[0], "the pending plan has more rows than its records")
    _require(
        rec.correction.shape[1:] == replay_cache.correction.shape[1:] and rec.key.shape[1:] == replay_cache.key.shape[1:],
        "pending records do not match this layer's record geometry",
    )
    arrays = (pending.rows,) + plan
    pc = N.PendingCommit(
        rows=arrays[0].data_ptr(), source=arrays[1].data_ptr(), lengths=arrays[2].data_ptr(),
        final_indices=arrays[3].data_ptr(), boundary_indices=arrays[4].data_ptr(),
        boundary_lengths=arrays[5].data_ptr(), correction=rec.correction.data_ptr(), key=rec.key.data_ptr(),
        decay=rec.decay.data_ptr(), record_rows=rec.correction.shape[0],
        key_dtype=N.dtype_code(rec.key.dtype), key_per_value_head=0, num_rows=num_rows,
    )
    for i in range(3):
        pc.corr_strides[i] = rec.correction.stride(i)
        pc.key_strides[i] = rec.key.stride(i)
        pc.decay_strides[i] = rec.decay.stride(i)
    return _verify(g, beta, q, k, v, checkpoint_state=checkpoint_state, replay_cache=replay_cache,
                   query_start_loc=query_start_loc, state_indices=state_indices, spec_query_len=spec_query_len,
                   scale=scale, qk_already_normalized=qk_already_normalized, out=out, gating=None,
                   pending=(pc, arrays, rec), _collect=_collect)


def _verify(g, beta, q, k, v, *, checkpoint_state, replay_cache, query_start_loc, state_indices, spec_query_len,
            scale, qk_already_normalized, out, gating, _collect, pending=None):
    _require(q.ndim == 4 and q.shape[0] == 1, "q must have shape [1, tokens, heads, dim]")
    _, total, H, K = q.shape
    _require(k.shape == q.shape, "q and k shapes differ")
    _require(v.ndim == 4 and tuple(v.shape[:2]) == (1, total), "v must have shape [1, tokens, value heads, dim]")
    HV, V = v.shape[-2], v.shape[-1]
    _require(H > 0 and HV >= H and HV % H == 0, "value heads must be a positive multiple of the q/k heads")
    if gating is not None:
        _require(gating[0].shape[0] == HV and gating[1].shape[0] == HV, "A_log and dt_bias need one entry per value head")
    _require(g.numel() == total * HV and beta.numel() == total * HV, "gate or beta shape is incompatible")
    g2 = g.reshape(total, HV)
    beta2 = beta.reshape(total, HV)
    _require(g2.stride(1) == 1 and beta2.stride(1) == 1, "gate and beta heads must be contiguous")
    _require(0 < spec_query_len <= MAX_SPEC_QUERY_LEN, f"spec_query_len must be in [1, {MAX_SPEC_QUERY_LEN}]")
    _require(all(t_.stride(-1) == 1 and t_.stride(-2) == K for t_ in (q, k)), "q and k heads must be contiguous")
    _require(v.stride(-1) == 1 and v.stride(-2) == V, "v heads must be contiguous")
    _require(checkpoint_state.ndim == 4, "checkpoint must be four-dimensional")
    nb = checkpoint_state.shape[0]
    _require(tuple(checkpoint_state.shape[1:]) == (HV, V, K), "checkpoint shape is incompatible")
    soa = isinstance(replay_cache, ReplayRecordBuffers)
    if soa:
        corr, key_record, decay_record = replay_cache.correction, replay_cache.key, replay_cache.decay
        _require(
            corr.ndim == 4
            and tuple(corr.shape[1:]) == (HV, spec_query_len, V)
            and tuple(key_record.shape) == (corr.shape[0], H, spec_query_len, K)
            and tuple(decay_record.shape) == (corr.shape[0], HV, spec_query_len),
            "typed record geometry is incompatible",
        )
        _require(corr.dtype == decay_record.dtype == torch.float32, "correction and decay records must remain FP32")
        _require(
            key_record.dtype in (torch.float16, torch.bfloat16, torch.float32)
            and (key_record.dtype == torch.float32 or (qk_already_normalized and key_record.dtype == k.dtype)),
            "low-precision key records require already-normalized input dtype",
        )
        _require(
            all(t.stride(-1) == 1 for t in (corr, key_record, decay_record)),
            "typed record innermost dimensions must be contiguous",
        )
    else:
        corr = key_record = decay_record = replay_cache
        _require(
            corr.ndim == 4 and tuple(corr.shape[1:]) == (HV, spec_query_len, V + K + 1),
            "packed replay record shape is incompatible",
        )
        _require(corr.dtype == torch.float32, "packed records must remain FP32")
        _require(corr.stride(-1) == 1, "packed record elements must be contiguous")
    _require(corr.shape[0] >= 1, "replay buffer has no rows")
    _require(state_indices.ndim == 1, "state indices must be one-dimensional")
    _require(
        query_start_loc.ndim == 1 and query_start_loc.shape[0] == state_indices.shape[0] + 1,
        "query metadata is incompatible",
    )
    _require(total <= state_indices.shape[0] * spec_query_len, "speculative decode input exceeds its activation capacity")
    _dev = q.device
    _require(
        all(
            t_.device == _dev
            for t_ in (k, v, g, beta, checkpoint_state, corr, key_record, decay_record, query_start_loc, state_indices)
            if t_ is not None
        )
        and (out is None or out.device == _dev),
        "inputs must be on the same device",
    )
    if scale is None:
        scale = K**-0.5
    if out is None:
        out = torch.empty(1, total, HV, V, dtype=v.dtype, device=v.device)
    _require(tuple(out.shape) == (1, total, HV, V) and out.stride()[2:] == (V, 1), "output shape or layout is incompatible")
    batch = state_indices.shape[0]
    if batch == 0 or (total == 0 and pending is None):
        return out
    # What the gfx950 kernels are built for (checked before any launch).
    _require(q.dtype == k.dtype == v.dtype, "q, k and v must share one activation dtype")
    for name, t_ in (("activation", q), ("output", out), ("gate", g2), ("beta", beta2), ("checkpoint", checkpoint_state)):
        _require(t_.dtype in (torch.float32, torch.bfloat16, torch.float16), f"{name} dtype {t_.dtype} is not supported")
    _require(
        query_start_loc.dtype in (torch.int32, torch.int64) and state_indices.dtype in (torch.int32, torch.int64),
        "query offsets and state indices must be int32 or int64",
    )
    _require(_dev.type == "cuda", "verify runs on a HIP device")
    es = checkpoint_state.element_size()
    chunk = 16 // es
    _require(
        K <= MAX_KEY_DIM
        and K % chunk == 0
        and checkpoint_state.stride(3) == 1
        and all(s_ % chunk == 0 for s_ in checkpoint_state.stride()[:3])
        and _aligned16(checkpoint_state),
        f"checkpoint rows must be contiguous, 16-byte aligned and K <= {MAX_KEY_DIM} a multiple of {chunk}",
    )
    f32 = 4
    if soa:
        key_ptr, decay_ptr = key_record.data_ptr(), decay_record.data_ptr()
        key_strides = key_record.stride()[:3]
        decay_strides = decay_record.stride()
        key_dtype = key_record.dtype
        key_per_value_head = 0
    else:
        # Packed [corr(V) | key(K) | decay(1)] FP32 rows: the key and decay
        # planes are views into the same record at offsets V and V + K.
        key_ptr = corr.data_ptr() + V * f32
        decay_ptr = corr.data_ptr() + (V + K) * f32
        key_strides = corr.stride()[:3]
        decay_strides = corr.stride()[:3]
        key_dtype = torch.float32
        key_per_value_head = 1
    config = (
        batch,
        total,
        H,
        HV,
        spec_query_len,
        nb,
        corr.shape[0],
        NULL_BLOCK_ID,
        q.stride(1),
        k.stride(1),
        v.stride(1),
        g2.stride(0),
        beta2.stride(0),
        checkpoint_state.stride(0),
        checkpoint_state.stride(1),
        checkpoint_state.stride(2),
        corr.stride(0),
        corr.stride(1),
        corr.stride(2),
        *key_strides,
        *decay_strides,
        out.stride(1),
        query_start_loc.stride(0),
        state_indices.stride(0),
    )
    ext = N.VerifyExt(
        key_dim=K,
        value_dim=V,
        act_dtype=N.dtype_code(q.dtype),
        beta_dtype=N.dtype_code(beta2.dtype),
        g_dtype=N.dtype_code(g2.dtype),
        state_dtype=N.dtype_code(checkpoint_state.dtype),
        key_record_dtype=N.dtype_code(key_dtype),
        qsl_dtype=N.dtype_code(query_start_loc.dtype),
        index_dtype=N.dtype_code(state_indices.dtype),
        qk_l2norm=0 if qk_already_normalized else 1,
        key_per_value_head=key_per_value_head,
        out_dtype=N.dtype_code(out.dtype),
    )
    cfg = N.i64_array(config)
    lib = _lib()
    tail = (
        checkpoint_state.data_ptr(),
        corr.data_ptr(),
        key_ptr,
        decay_ptr,
        out.data_ptr(),
        query_start_loc.data_ptr(),
        state_indices.data_ptr(),
        cfg,
        N.VERIFY_CONFIG_FIELDS,
        float(scale),
        ctypes.byref(ext),
    )
    keep = (q, k, v, g2, beta2, checkpoint_state, corr, key_record, decay_record, out, query_start_loc, state_indices,
            cfg, ext)
    if pending is not None:
        pc, arrays, rec = pending
        fn = lib.gdn_recoverssm_verify_deferred
        args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), g2.data_ptr(), beta2.data_ptr()) + tail + (ctypes.byref(pc),)
        keep = keep + (pc, arrays, rec)
    elif gating is None:
        fn, args = lib.gdn_recoverssm_verify, (q.data_ptr(), k.data_ptr(), v.data_ptr(), g2.data_ptr(),
                                                beta2.data_ptr()) + tail
    else:
        a_log, dt_bias, sp_beta, sp_threshold = gating
        _require(all(t_.device == _dev for t_ in (a_log, dt_bias)), "inputs must be on the same device")
        gext = N.GatingExt(a_log_dtype=N.dtype_code(a_log.dtype), dt_bias_dtype=N.dtype_code(dt_bias.dtype),
                           softplus_beta=sp_beta, softplus_threshold=sp_threshold)
        fn = lib.gdn_recoverssm_verify_gated
        args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), g2.data_ptr(), beta2.data_ptr(), a_log.data_ptr(),
                dt_bias.data_ptr()) + tail + (ctypes.byref(gext),)
        keep = keep + (a_log, dt_bias, gext)
    spec = _LaunchSpec("verify", fn, args, _dev, keepalive=keep)
    spec.config = tuple(int(x) for x in config)
    spec.scale = float(scale)
    if _collect is None:
        spec.launch()
    else:
        _collect.append(spec)
    return out


# ---------------------------------------------------------------------------
# Single-context commit (reference kernels.py:1399-2052)
# ---------------------------------------------------------------------------


def _record_planes(record, V: int, K: int):
    """(correction, key, decay) tensors plus the byte offsets of key / decay.

    Typed records expose three planes. A packed FP32 record [rows, HV, Q, V+K+1]
    is addressed as three strided planes of the same storage: the key at
    element offset V and the decay at V + K of every (row, head, token) record.
    """
    if isinstance(record, ReplayRecordBuffers):
        return record.correction, record.key, record.decay, 0, 0
    return record, record, record, V * 4, (V + K) * 4


@dataclass
class GDNRecoverSSMCommitContext:
    conv_states: tuple
    conv_state_base_addrs: torch.Tensor
    conv_state_block_strides: torch.Tensor
    conv_state_dim_strides: torch.Tensor
    conv_state_token_strides: torch.Tensor
    conv_history_len: int
    checkpoints: tuple
    state_base_addrs: torch.Tensor
    state_block_strides: torch.Tensor
    replays: tuple
    replay_base_addrs: torch.Tensor
    replay_block_strides: torch.Tensor
    commit_lens: torch.Tensor
    final_state_indices: torch.Tensor
    boundary_state_indices: torch.Tensor
    boundary_recovery_lens: torch.Tensor
    spec_query_len: int
    num_blocks: int

    @classmethod
    def from_tensors(
        cls,
        conv_states: Sequence[torch.Tensor],
        checkpoints: Sequence[torch.Tensor],
        replays: Sequence[torch.Tensor | ReplayRecordBuffers],
        *,
        spec_query_len: int,
        max_num_reqs: int,
        conv_dim_first: bool = True,
    ) -> "GDNRecoverSSMCommitContext":
        """Bind layer-owned page views and allocate reusable commit-plan buffers."""
        _require(len(checkpoints) > 0, "commit requires at least one layer")
        _require(len(conv_states) == len(checkpoints) == len(replays), "conv, state and replay lists differ")
        _require(0 < spec_query_len <= MAX_SPEC_QUERY_LEN, f"spec_query_len must be in [1, {MAX_SPEC_QUERY_LEN}]")
        if not conv_dim_first:
            conv_states = [s.transpose(-1, -2) for s in conv_states]
        ref = checkpoints[0]
        _require(ref.ndim == 4, "checkpoint must be four-dimensional")
        nb, HV, V, K = ref.shape
        _dev = ref.device
        for s in checkpoints:
            _require(
                s.shape == ref.shape and s.dtype == ref.dtype and s.stride()[1:] == ref.stride()[1:] and s.device == _dev,
                "layers need matching checkpoints",
            )
        soa = isinstance(replays[0], ReplayRecordBuffers)
        _require(
            all(isinstance(r, ReplayRecordBuffers) == soa for r in replays),
            "packed and typed records cannot share a commit context",
        )
        if soa:
            corrs = [r.correction for r in replays]
            keys = [r.key for r in replays]
            decays = [r.decay for r in replays]
            H = keys[0].shape[1]
            _require(H > 0 and HV % H == 0, "record key heads are incompatible")
            for c, k, d in zip(corrs, keys, decays):
                _require(
                    c.shape == corrs[0].shape
                    and tuple(c.shape[1:]) == (HV, spec_query_len, V)
                    and tuple(k.shape) == (c.shape[0], H, spec_query_len, K)
                    and tuple(d.shape) == (c.shape[0], HV, spec_query_len)
                    and c.dtype == d.dtype == torch.float32
                    and k.dtype in (torch.float16, torch.bfloat16, torch.float32)
                    and k.dtype == keys[0].dtype
                    and all(t.device == _dev for t in (c, k, d))
                    and c.stride()[1:] == corrs[0].stride()[1:]
                    and k.stride()[1:] == keys[0].stride()[1:]
                    and d.stride()[1:] == decays[0].stride()[1:],
                    "layers need matching typed replay geometry/dtypes/strides",
                )
        else:
            corrs = keys = decays = list(replays)
            H = HV
            for r in replays:
                _require(
                    r.ndim == 4
                    and tuple(r.shape[1:]) == (HV, spec_query_len, V + K + 1)
                    and r.shape == replays[0].shape
                    and r.dtype == torch.float32
                    and r.stride()[1:] == replays[0].stride()[1:]
                    and r.device == _dev,
                    "layers need matching packed FP32 replay buffers",
                )
        conv_ref = conv_states[0]
        _require(
            conv_ref.ndim == 3 and conv_ref.shape[0] == nb,
            "conv state must be [blocks, dim, window] with the checkpoint's block count",
        )
        for c in conv_states:
            _require(
                c.shape == conv_ref.shape and c.dtype == conv_ref.dtype and c.stride()[1:] == conv_ref.stride()[1:] and c.device == _dev,
                "layers need matching conv states",
            )
        conv_dim, conv_len = conv_ref.shape[1:]
        hist = conv_len - spec_query_len + 1
        _require(hist > 0, "conv state is shorter than its window")
        dev = ref.device
        key_off = 0 if soa else V * 4
        decay_off = 0 if soa else (V + K) * 4

        def addr(ts, off=0):
            return _ptr_table(ts, dev, [off] * len(ts) if off else None)

        def bstr(ts):
            return torch.tensor([t.stride(0) for t in ts], dtype=torch.int64, device=dev)

        def z():
            return torch.zeros(max_num_reqs, dtype=torch.int32, device=dev)

        context = cls(
            tuple(conv_states),
            addr(conv_states),
            bstr(conv_states),
            torch.tensor([s.stride(1) for s in conv_states], dtype=torch.int64, device=dev),
            torch.tensor([s.stride(2) for s in conv_states], dtype=torch.int64, device=dev),
            hist,
            tuple(checkpoints),
            addr(checkpoints),
            bstr(checkpoints),
            tuple(replays),
            addr(corrs),
            bstr(corrs),
            z(),
            z(),
            z(),
            z(),
            spec_query_len,
            nb,
        )
        context.records = list(replays)
        context.record_rows = int(corrs[0].shape[0])
        context.record_layout = "soa" if soa else "packed"
        context.num_key_heads = int(H)
        context.key_dtype = keys[0].dtype if soa else torch.float32
        context.correction_base_addrs = context.replay_base_addrs
        context.correction_block_strides = context.replay_block_strides
        context.key_base_addrs = addr(keys, key_off)
        context.key_block_strides = bstr(keys)
        context.decay_base_addrs = addr(decays, decay_off)
        context.decay_block_strides = bstr(decays)
        context.record_bytes = sum(record_nbytes(r) for r in replays)
        context.align_valid = z()
        context.align_col = z()
        context.plan_source = z()  # canonical source page of each planned row (NULL when invalid)
        context.pending_rows = torch.arange(max_num_reqs, dtype=torch.int32, device=dev)
        return context

    @classmethod
    def create(
        cls,
        layers: Sequence[Any],
        *,
        spec_query_len: int,
        max_num_reqs: int,
        record_rows: int | None = None,
        num_key_heads: int | None = None,
        key_dtype: torch.dtype | None = None,
        conv_dim_first: bool | None = None,
    ) -> "GDNRecoverSSMCommitContext":
        """Build the context from live layers' ``kv_cache`` pages (conv, checkpoint).

        Records are allocated here as row-indexed scratch and handed to each
        layer as ``layer._gdn_recoverssm_records``.
        """
        if conv_dim_first is None:
            try:  # vLLM decides the conv layout when it is installed
                from vllm.model_executor.layers.mamba.mamba_utils import is_conv_state_dim_first

                conv_dim_first = bool(is_conv_state_dim_first())
            except ImportError:
                conv_dim_first = True
        if any(len(layer.kv_cache) != 2 for layer in layers):
            raise ValueError("GDN RecoverSSM expects conv and checkpoint pages; the replay records live outside the cache")
        state0 = layers[0].kv_cache[1]
        num_heads, head_v, head_k = state0.shape[1], state0.shape[2], state0.shape[3]
        rows = int(record_rows or max_num_reqs)
        key_heads = num_heads if num_key_heads is None else int(num_key_heads)
        record_key_dtype = torch.float32 if key_dtype is None else key_dtype
        records = [
            ReplayRecordBuffers.allocate(
                rows, num_heads, key_heads, spec_query_len, head_v, head_k, device=state0.device, key_dtype=record_key_dtype
            )
            for _ in layers
        ]
        context = cls.from_tensors(
            [layer.kv_cache[0] for layer in layers],
            [layer.kv_cache[1] for layer in layers],
            records,
            spec_query_len=spec_query_len,
            max_num_reqs=max_num_reqs,
            conv_dim_first=conv_dim_first,
        )
        context.records = records
        for layer, record in zip(layers, records):
            layer._gdn_recoverssm_records = record
        return context

    def make_commit_specs(
        self,
        num_accepted_tokens,
        state_indices,
        query_start_loc,
        request_indices=None,
        block_table=None,
        num_computed_tokens=None,
        mamba_block_size=None,
        commit_conv: bool = True,
    ) -> tuple:
        """Build the launch specs for one step, without launching them."""
        specs: list = []
        self.commit(
            num_accepted_tokens,
            state_indices,
            query_start_loc,
            request_indices=request_indices,
            block_table=block_table,
            num_computed_tokens=num_computed_tokens,
            mamba_block_size=mamba_block_size,
            commit_conv=commit_conv,
            _collect=specs,
        )
        return tuple(specs)

    def prepare_verify(self, *, activation_dtype, state_table_width: int | None = None, device=None) -> list:
        """Validate the serving verify signatures (contiguous and combined-QKV
        value views, activation-typed and FP32 beta) without touching state."""
        device = self.checkpoints[0].device if device is None else device
        record = self.records[0]
        _, hv, value_dim, key_dim = self.checkpoints[0].shape
        key_heads = self.num_key_heads
        window = self.spec_query_len
        width = int(state_table_width or window)
        _require(width > 0, "verify preparation requires a positive table stride")
        q = torch.empty((1, window, key_heads, key_dim), dtype=activation_dtype, device=device)
        k = torch.empty_like(q)
        g = torch.empty((1, window, hv), dtype=torch.float32, device=device)
        output = torch.empty((1, window, hv, value_dim), dtype=activation_dtype, device=device)
        state_table = torch.empty((1, width), dtype=torch.int32, device=device)
        offsets = torch.empty(2, dtype=torch.int32, device=device)
        report = []
        for packed_value in (False, True):
            if packed_value:
                features = 2 * key_heads * key_dim + hv * value_dim
                combined = torch.empty((1, window, features), dtype=activation_dtype, device=device)
                value = combined[:, :, 2 * key_heads * key_dim :].view(1, window, hv, value_dim)
            else:
                value = torch.empty_like(output)
            for beta_dtype in tuple(dict.fromkeys((torch.float32, activation_dtype))):
                beta = torch.empty((1, window, hv), dtype=beta_dtype, device=device)
                specs: list = []
                gdn_recoverssm_verify(
                    g, beta, q, k, value, checkpoint_state=self.checkpoints[0], replay_cache=record,
                    query_start_loc=offsets, state_indices=state_table[:, 0], spec_query_len=window,
                    qk_already_normalized=True, out=output, _collect=specs,
                )
                for spec in specs:
                    spec.compile_only()
                report.append(
                    dict(
                        activation_dtype=str(activation_dtype), beta_dtype=str(beta_dtype),
                        value_token_stride=value.stride(1), state_index_stride=width, state_blocks=self.num_blocks,
                        record_rows=self.record_rows, num_value_heads=hv, num_key_heads=key_heads, window=window,
                    )
                )
        self.verify_prepare_report = tuple(report)
        return report

    def prepare(
        self,
        *,
        capacity: int,
        state_table_width: int,
        request_mapping: bool,
        device,
        align_mode: bool = False,
        mamba_block_size: int | None = None,
        block_table_width: int | None = None,
        request_index_dtype=torch.int64,
        accepted_dtype=torch.int32,
        state_index_dtype=torch.int32,
        query_index_dtype=torch.int32,
        computed_dtype=torch.int32,
    ) -> list[int]:
        """Validate the none/align commit signatures for every row count."""
        _require(
            not align_mode or (mamba_block_size is not None and mamba_block_size >= self.spec_query_len),
            "align preparation requires the runtime block size",
        )
        compiled_rows = []
        for rows in range(1, min(capacity, self.record_rows) + 1):
            table = torch.empty((rows, state_table_width), dtype=state_index_dtype, device=device)
            qsl = torch.empty(rows + 1, dtype=query_index_dtype, device=device)
            accepted = torch.empty(rows, dtype=accepted_dtype, device=device)
            mapping = torch.empty(rows, dtype=request_index_dtype, device=device) if request_mapping else None
            bt = computed = None
            if align_mode:
                width = int(block_table_width or state_table_width)
                bt = torch.empty((rows, width), dtype=state_index_dtype, device=device)
                computed = torch.empty(rows, dtype=computed_dtype, device=device)
            for spec in self.make_commit_specs(
                accepted, table[:, 0], qsl, request_indices=mapping, block_table=bt, num_computed_tokens=computed,
                mamba_block_size=mamba_block_size if align_mode else None,
            ):
                spec.compile_only()
            compiled_rows.append(rows)
        return compiled_rows

    def commit(
        self,
        num_accepted_tokens: torch.Tensor,
        state_indices: torch.Tensor,
        query_start_loc: torch.Tensor,
        request_indices: torch.Tensor | None = None,
        block_table: torch.Tensor | None = None,
        num_computed_tokens: torch.Tensor | None = None,
        mamba_block_size: int | None = None,
        commit_conv: bool = True,
        _collect: list | None = None,
        _fold_source: torch.Tensor | None = None,
    ) -> None:
        """Fold accepted GDN and convolution inputs into every layer's checkpoint."""
        batch = state_indices.shape[0]
        if batch == 0:
            return
        _require(state_indices.ndim == 1, "state indices must be one-dimensional")
        _require(batch <= self.commit_lens.shape[0], "commit batch exceeds its plan capacity")
        _require(query_start_loc.ndim == 1 and query_start_loc.shape[0] == batch + 1, "commit metadata is incompatible")
        _require(request_indices is None or request_indices.shape[0] >= batch, "request mapping is too short")
        _require(
            num_accepted_tokens.ndim == 1 and (request_indices is not None or num_accepted_tokens.shape[0] >= batch),
            "accepted-token counts are too short",
        )
        _align = (block_table, num_computed_tokens, mamba_block_size)
        _require(all(x is None for x in _align) or all(x is not None for x in _align), "align metadata is incomplete")
        _require(
            mamba_block_size is None or mamba_block_size >= self.spec_query_len,
            "align block size must cover one speculative window",
        )
        _require(
            block_table is None or (block_table.ndim == 2 and block_table.shape[1] > 0),
            "block table must be two-dimensional with a positive width",
        )
        _dev = self.checkpoints[0].device
        _require(
            all(
                t_ is None or t_.device == _dev
                for t_ in (num_accepted_tokens, state_indices, query_start_loc, request_indices, block_table, num_computed_tokens)
            ),
            "commit inputs must be on the same device",
        )
        _require(_dev.type == "cuda", "the commit runs on a HIP device")
        align = block_table is not None
        lib = _lib()
        grp = N.PlanGroups()
        gr = grp[0]
        gr.state_indices = state_indices.data_ptr()
        gr.si_stride = state_indices.stride(0)
        gr.si_dtype = N.dtype_code(state_indices.dtype)
        gr.query_start_loc = query_start_loc.data_ptr()
        gr.qsl_stride = query_start_loc.stride(0)
        gr.qsl_dtype = N.dtype_code(query_start_loc.dtype)
        if request_indices is not None:
            gr.request_indices = request_indices.data_ptr()
            gr.map_stride = request_indices.stride(0)
            gr.map_dtype = N.dtype_code(request_indices.dtype)
        if align:
            gr.block_table = block_table.data_ptr()
            gr.table_row_stride = block_table.stride(0)
            gr.table_col_stride = block_table.stride(1)
            gr.table_width = block_table.shape[1]
            gr.table_rows = block_table.shape[0]
            gr.table_dtype = N.dtype_code(block_table.dtype)
            gr.num_computed = num_computed_tokens.data_ptr()
            gr.computed_stride = num_computed_tokens.stride(0)
            gr.computed_len = num_computed_tokens.shape[0]
            gr.computed_dtype = N.dtype_code(num_computed_tokens.dtype)
            gr.block_size = int(mamba_block_size)
        else:
            gr.block_size = 1
            gr.table_width = 1
        gr.num_blocks = self.num_blocks
        plan_args = (
            num_accepted_tokens.data_ptr(),
            N.dtype_code(num_accepted_tokens.dtype),
            num_accepted_tokens.stride(0),
            num_accepted_tokens.shape[0],
            grp,
            1,
            self.plan_source.data_ptr(),
            self.commit_lens.data_ptr(),
            self.final_state_indices.data_ptr(),
            self.boundary_state_indices.data_ptr(),
            self.boundary_recovery_lens.data_ptr(),
            self.align_valid.data_ptr(),
            self.align_col.data_ptr(),
            None,
            N.DT_I32,
            0,
            None,
            None,
            0,
            batch,
            self.commit_lens.shape[0],
            NULL_BLOCK_ID,
            self.spec_query_len,
            N.PLAN_ALIGN if align else 0,
        )
        keep = (num_accepted_tokens, state_indices, query_start_loc, request_indices, block_table, num_computed_tokens)
        plan_spec = _LaunchSpec("plan", lib.gdn_recoverssm_plan, plan_args, _dev, keepalive=(grp,) + keep)
        specs = [plan_spec]
        num_layers = len(self.checkpoints)
        if commit_conv:
            conv_ref = self.conv_states[0]
            conv_args = (
                self.conv_state_base_addrs.data_ptr(),
                self.conv_state_block_strides.data_ptr(),
                self.conv_state_dim_strides.data_ptr(),
                self.conv_state_token_strides.data_ptr(),
                state_indices.data_ptr(),
                N.dtype_code(state_indices.dtype),
                state_indices.stride(0),
                self.commit_lens.data_ptr(),
                self.final_state_indices.data_ptr(),
                self.boundary_state_indices.data_ptr(),
                self.boundary_recovery_lens.data_ptr(),
                None,
                self.commit_lens.shape[0],
                NULL_BLOCK_ID,
                batch,
                num_layers,
                conv_ref.shape[1],
                self.conv_history_len,
                conv_ref.shape[2],
                self.num_blocks,
                conv_ref.element_size(),
                1 if align else 0,
            )
            _require(conv_ref.element_size() in (2, 4), "conv state elements must be 2 or 4 bytes")
            specs.append(_LaunchSpec("conv", lib.gdn_recoverssm_conv_compact, conv_args, _dev, keepalive=keep))
        ref = self.checkpoints[0]
        _, HV, V, K = ref.shape
        record = self.replays[0]
        rr, kr, dr, _, _ = _record_planes(record, V, K)
        soa = self.record_layout == "soa"
        key_strides = kr.stride()[1:3] if soa else rr.stride()[1:3]
        decay_strides = dr.stride()[1:3] if soa else rr.stride()[1:3]
        fold_spec = _make_fold_spec(
            ref=ref,
            record_rows=rr.shape[0],
            corr_strides=rr.stride()[1:3],
            key_strides=key_strides,
            decay_strides=decay_strides,
            key_heads=self.num_key_heads,
            key_dtype=self.key_dtype,
            num_layers=num_layers,
            rows=batch,
            plan_capacity=self.commit_lens.shape[0],
            num_blocks=self.num_blocks,
            spec_query_len=self.spec_query_len,
            tables=(
                self.state_base_addrs, self.state_block_strides, self.correction_base_addrs, self.correction_block_strides,
                self.key_base_addrs, self.key_block_strides, self.decay_base_addrs, self.decay_block_strides,
            ),
            layer_groups=None,
            source=state_indices if _fold_source is None else _fold_source,
            plan=(self.commit_lens, self.final_state_indices, self.boundary_state_indices, self.boundary_recovery_lens),
            refs=(rr, kr, dr),
        )
        specs.append(fold_spec)
        if _fold_source is None:
            # One launch plans and folds; the conv compaction, which reads the
            # stored plan, follows it.
            specs = [_fuse_plan_fold(plan_spec, fold_spec)] + specs[1:-1]
        if _collect is not None:
            _collect.extend(specs)
        else:
            for spec in specs:
                spec.launch()
        self._last_specs = tuple(specs)

    def commit_deferred(
        self,
        num_accepted_tokens: torch.Tensor,
        state_indices: torch.Tensor,
        query_start_loc: torch.Tensor,
        request_indices: torch.Tensor | None = None,
        block_table: torch.Tensor | None = None,
        num_computed_tokens: torch.Tensor | None = None,
        mamba_block_size: int | None = None,
        commit_conv: bool = True,
        _collect: list | None = None,
    ) -> tuple:
        """Plan the commit (and compact the conv states) but leave the fold to
        the next step's ``gdn_recoverssm_verify_deferred``; returns one
        ``PendingCommit`` per layer. ``flush_deferred`` applies the pending
        fold directly instead (for a step that runs no verify)."""
        _require(self.record_layout == "soa", "the deferred commit needs typed record buffers")
        specs: list = []
        self.commit(num_accepted_tokens, state_indices, query_start_loc, request_indices=request_indices,
                    block_table=block_table, num_computed_tokens=num_computed_tokens,
                    mamba_block_size=mamba_block_size, commit_conv=commit_conv, _collect=specs,
                    _fold_source=self.plan_source)
        self._deferred_fold = next(sp for sp in specs if sp.name == "fold")
        self._deferred_rows = int(state_indices.shape[0])
        now = [sp for sp in specs if sp.name != "fold"]
        if _collect is not None:
            _collect.extend(now)
        else:
            for sp in now:
                sp.launch()
        return tuple(
            PendingCommit(self.pending_rows, self.plan_source, self.commit_lens, self.final_state_indices,
                          self.boundary_state_indices, self.boundary_recovery_lens, rec,
                          num_rows=self._deferred_rows)
            for rec in self.records
        )

    def flush_deferred(self, rows: Sequence[int] | torch.Tensor | None = None, _collect: list | None = None) -> None:
        """Apply the last ``commit_deferred`` plan with the ordinary fold.

        ``rows=None`` folds every planned row (a step that runs no verify
        after it, e.g. the end of a batch); a list of pending rows folds only
        those (rows whose request left the batch, see ``continue_pending``),
        leaving the rest to the next verify. A row must be folded once: by a
        flush or by the verify that continues it, never both.
        """
        spec = getattr(self, "_deferred_fold", None)
        _require(spec is not None, "no deferred commit to flush")
        if rows is not None:
            pick = torch.as_tensor(rows, dtype=torch.int64).reshape(-1).cpu()
            _require(
                bool(((pick >= 0) & (pick < self._deferred_rows)).all()),
                "flushed rows must be rows of the pending plan",
            )
            if pick.numel() == 0:
                return
            # The same fold over a length array that keeps only the picked rows.
            lengths = torch.zeros_like(self.commit_lens)
            idx = pick.to(lengths.device)
            lengths[idx] = self.commit_lens[idx]
            args = list(spec.args)
            args[14] = lengths.data_ptr()  # fold arguments: ..., source, lengths, finals, ...
            spec = _LaunchSpec(spec.name, spec.fn, tuple(args), spec.device, keepalive=spec.keepalive + (lengths,))
        if _collect is not None:
            _collect.append(spec)
        else:
            spec.launch()


def _fuse_plan_fold(plan: _LaunchSpec, fold: _LaunchSpec) -> _LaunchSpec:
    """``gdn_recoverssm_plan_fold``: the plan launch and the fold launch that
    reads its arrays, as one launch with identical results (every fold
    workgroup plans its own row; extra workgroups store the plan arrays)."""
    launch = N.plan_launch(plan.args)
    # fold arguments: 4 reference tensors, 8 tables, layer_groups, source,
    # 4 plan arrays, config, config length, extension
    args = (ctypes.byref(launch),) + tuple(fold.args[:13]) + tuple(fold.args[18:])
    spec = _LaunchSpec(
        "plan_fold", _lib().gdn_recoverssm_plan_fold, args, fold.device, keepalive=(plan.keepalive, fold.keepalive, launch)
    )
    spec.config = fold.config
    return spec


def _make_fold_spec(
    *,
    ref,
    record_rows,
    corr_strides,
    key_strides,
    decay_strides,
    key_heads,
    key_dtype,
    num_layers,
    rows,
    plan_capacity,
    num_blocks,
    spec_query_len,
    tables,
    layer_groups,
    source,
    plan,
    refs,
) -> _LaunchSpec:
    """Fold launch shared by the single-context and grouped commits."""
    _, HV, V, K = ref.shape
    es = ref.element_size()
    chunk = 16 // es
    _require(ref.dtype in (torch.float32, torch.bfloat16, torch.float16), "checkpoint dtype is not supported")
    _require(key_dtype in (torch.float32, torch.bfloat16, torch.float16), "record key dtype is not supported")
    _require(
        K <= MAX_KEY_DIM and K % chunk == 0 and ref.stride(3) == 1 and all(s_ % chunk == 0 for s_ in ref.stride()[:3]) and V <= 1024,
        f"checkpoint rows must be contiguous, 16-byte aligned, K <= {MAX_KEY_DIM} a multiple of {chunk}, V <= 1024",
    )
    config = (
        rows,
        num_layers,
        HV,
        key_heads,
        spec_query_len,
        num_blocks,
        record_rows,
        plan_capacity,
        NULL_BLOCK_ID,
        ref.stride(1),
        ref.stride(2),
        corr_strides[0],
        corr_strides[1],
        key_strides[0],
        key_strides[1],
        decay_strides[0],
        decay_strides[1],
    )
    ext = N.FoldExt(
        key_dim=K,
        value_dim=V,
        state_dtype=N.dtype_code(ref.dtype),
        key_dtype=N.dtype_code(key_dtype),
        source_dtype=N.dtype_code(source.dtype),
        reserved=0,
        source_stride=source.stride(0),
        state_k_stride=ref.stride(3),
    )
    cfg = N.i64_array(config)
    lengths, finals, boundaries, boundary_lens = plan
    rr, kr, dr = refs
    args = (
        ref.data_ptr(),
        rr.data_ptr(),
        kr.data_ptr(),
        dr.data_ptr(),
        *(t.data_ptr() for t in tables),
        None if layer_groups is None else layer_groups.data_ptr(),
        source.data_ptr(),
        lengths.data_ptr(),
        finals.data_ptr(),
        boundaries.data_ptr(),
        boundary_lens.data_ptr(),
        cfg,
        N.FOLD_CONFIG_FIELDS,
        ctypes.byref(ext),
    )
    spec = _LaunchSpec(
        "fold",
        _lib().gdn_recoverssm_fold,
        args,
        ref.device,
        keepalive=(ref, rr, kr, dr, *tables, layer_groups, source, *plan, cfg, ext),
    )
    spec.config = tuple(int(x) for x in config)
    return spec


__all__ = [
    "GDNRecoverSSMCommitContext",
    "ReplayRecordBuffers",
    "gdn_recoverssm_verify",
    "record_geometry_bytes",
    "record_nbytes",
]

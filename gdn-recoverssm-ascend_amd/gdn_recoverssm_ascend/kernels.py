"""Verify and single-context commit: the host side, on AMD Instinct MI355X.

The public names, argument meaning and error behaviour are the reference
plugin's ``gdn_recoverssm_ascend/kernels.py`` (its callers, ``layer_patch._verify``
and the commit proxy, run unchanged); everything below them is this module's:

* ``gdn_recoverssm_verify`` (reference kernels.py:700-928), with the gated
  variant (gating and the q/k L2 norm fused in) and the deferred variant (the
  previous step's fold applied by this verify);
* ``ReplayRecordBuffers``, ``record_nbytes``, ``record_geometry_bytes``: the
  typed record planes and their byte counts (kernels.py:166-294);
* ``GDNRecoverSSMCommitContext`` (kernels.py:1399-2052): one commit context
  per cache epoch. Its commit is the plan and the fold in one launch
  (``gdn_recoverssm_plan_fold``), then the conv compaction that reads the
  stored plan; ``commit_deferred`` plans now and leaves the fold to the next
  verify.

Arguments are checked by rule tables (``_rules``) before anything is launched
and a violation raises ``ValueError("GDN RecoverSSM: ...")``; every launch is a
``_LaunchSpec`` of a C entry point of ``libgdn_recoverssm_hip.so`` (``_native``)
on the current stream, and a failed launch raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import math
from collections import Counter
from collections.abc import Sequence
from dataclasses import dataclass, field, replace
from functools import cached_property
from typing import Any

import torch

from . import _native as N
from ._rules import enforce, fail, require
from ._tables import LayerPages, check_layers, record_planes

# vLLM's physical null page (vllm.v1.attention.backends.utils.NULL_BLOCK_ID).
NULL_BLOCK_ID = 0

# Speculative-window capacity of the kernels (reference kernels.py:101).
MAX_SPEC_QUERY_LEN = 8

# Largest key dimension the verify / fold kernels are instantiated for.
MAX_KEY_DIM = 256

_FLOAT_TYPES = (torch.float32, torch.bfloat16, torch.float16)
_INDEX_TYPES = (torch.int32, torch.int64)

_COUNTS: Counter = Counter()


def counts() -> dict:
    """Launches per entry point (``verify``, ``plan``, ``conv``, ``fold``,
    ``plan_fold``, ``publish``); ``prepared_<name>`` counts compile-only
    preparations."""
    return dict(_COUNTS)


# Kept for the grouped module and older callers: one rule, checked on the spot.
_require = require


# ---------------------------------------------------------------------------
# Records (reference kernels.py:166-294)
# ---------------------------------------------------------------------------


def _key_dtype_ok(dtype) -> bool:
    return dtype in _FLOAT_TYPES


@dataclass(frozen=True)
class ReplayRecordBuffers:
    """What one verify leaves for the commit, as three row-indexed planes:
    ``correction [rows, HV, Q, V]`` and ``decay [rows, HV, Q]`` in FP32, and
    ``key [rows, H, Q, K]`` in the key dtype, one key per key head (the value
    heads of a GQA group share it). A BF16/FP16 key record holds the input
    key's own bits, so it is only allowed for already-normalised keys."""

    correction: torch.Tensor
    key: torch.Tensor
    decay: torch.Tensor

    # Views derived from the three planes (the attribute names the callers use).
    planes = property(lambda self: (self.correction, self.key, self.decay))
    device = property(lambda self: self.correction.device)
    key_dtype = property(lambda self: self.key.dtype)
    num_key_heads = property(lambda self: int(self.key.shape[1]))
    dtype = property(lambda self: torch.float32, doc="Arithmetic type of the records (FP32 whatever the key dtype).")
    record_bytes = property(lambda self: sum(p.numel() * p.element_size() for p in self.planes))

    @property
    def shape(self) -> tuple[int, int, int, int]:
        """The packed layout this record set stands for: one [V | K | 1] row per
        (record row, value head, token)."""
        *lead, v = self.correction.shape
        return (*lead, v + self.key.shape[-1] + 1)

    @classmethod
    def allocate(cls, rows: int, num_value_heads: int, num_key_heads: int, window: int, value_dim: int,
                 key_dim: int, *, device, key_dtype=torch.float32):
        enforce((
            ("record head/row geometry is invalid",
             lambda: min(rows, num_value_heads, num_key_heads, value_dim, key_dim) > 0
             and 0 < window <= MAX_SPEC_QUERY_LEN and num_value_heads % num_key_heads == 0),
            ("record keys require FP16, BF16 or FP32", lambda: _key_dtype_ok(key_dtype)),
        ))
        planes = {
            "correction": ((rows, num_value_heads, window, value_dim), torch.float32),
            "key": ((rows, num_key_heads, window, key_dim), key_dtype),
            "decay": ((rows, num_value_heads, window), torch.float32),
        }
        return cls(**{name: torch.zeros(shape, dtype=dt, device=device) for name, (shape, dt) in planes.items()})


def record_nbytes(record: torch.Tensor | ReplayRecordBuffers) -> int:
    if isinstance(record, ReplayRecordBuffers):
        return record.record_bytes
    return record.numel() * record.element_size()


def record_geometry_bytes(rows: int, num_layers: int, num_value_heads: int, num_key_heads: int, window: int,
                          key_dim: int, value_dim: int, key_dtype=torch.float32) -> int:
    """Bytes of one step's typed records over all layers: per (row, layer,
    token) an FP32 correction and decay per value head and one key per key
    head in its dtype."""
    enforce((
        ("record geometry must be positive",
         lambda: min(rows, num_layers, num_value_heads, num_key_heads, window, key_dim, value_dim) > 0),
        ("value heads must be a multiple of key heads", lambda: num_value_heads % num_key_heads == 0),
        ("record keys require FP16, BF16 or FP32", lambda: _key_dtype_ok(key_dtype)),
    ))
    key_bytes = torch.empty((), dtype=key_dtype).element_size()
    per_token = num_value_heads * (value_dim + 1) * 4 + num_key_heads * key_dim * key_bytes
    return rows * num_layers * window * per_token


# ---------------------------------------------------------------------------
# Launch specs
# ---------------------------------------------------------------------------


@dataclass
class _LaunchSpec:
    """One launch of a C entry point, built once and launched on the current
    stream. ``launch()`` submits it; ``compile_only()`` only checks that the
    ahead-of-time library and its entry point are there (nothing is compiled
    at run time and no device memory is touched). ``name`` is the entry point
    (``verify`` / ``plan`` / ``conv`` / ``fold`` / ``plan_fold`` / ``publish``)."""

    name: str
    fn: Any
    args: tuple
    device: torch.device
    keepalive: tuple = field(default_factory=tuple)

    def launch(self) -> None:
        status = self.fn(*self.args, N.stream_handle(self.device))
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


class _VerifyCall:
    """The tensors of one verify call and the sizes that follow from them.
    Sizes are read lazily, so each rule only touches what the rules before it
    have established."""

    def __init__(self, g, beta, q, k, v, checkpoint, records, qsl, indices, window, normalized, out, gating,
                 retain=None):
        self.g, self.beta, self.q, self.k, self.v = g, beta, q, k, v
        self.checkpoint, self.records, self.qsl, self.indices = checkpoint, records, qsl, indices
        self.window, self.normalized, self.out, self.gating = int(window), normalized, out, gating
        self.typed = isinstance(records, ReplayRecordBuffers)
        self.retain = retain

    @property
    def retain_field(self) -> int:
        """The ABI's per-call cache hint: 0 for the process-wide setting, the
        byte count when positive, -1 for none."""
        if self.retain is None:
            return 0
        return int(self.retain) if int(self.retain) > 0 else -1

    tokens = cached_property(lambda c: c.q.shape[1])
    H = cached_property(lambda c: c.q.shape[2])
    K = cached_property(lambda c: c.q.shape[3])
    HV = cached_property(lambda c: c.v.shape[2])
    V = cached_property(lambda c: c.v.shape[3])
    rows = cached_property(lambda c: c.indices.shape[0])
    g2 = cached_property(lambda c: c.g.reshape(c.tokens, c.HV))
    beta2 = cached_property(lambda c: c.beta.reshape(c.tokens, c.HV))
    planes = cached_property(lambda c: record_planes(c.records, c.V, c.K))

    def tensors(self):
        p = self.planes
        return (self.k, self.v, self.g, self.beta, self.checkpoint, p.correction, p.key, p.decay, self.qsl,
                self.indices)


_ACTIVATION_RULES = (
    ("q must have shape [1, tokens, heads, dim]", lambda c: c.q.ndim == 4 and c.q.shape[0] == 1),
    ("q and k shapes differ", lambda c: c.k.shape == c.q.shape),
    ("v must have shape [1, tokens, value heads, dim]",
     lambda c: c.v.ndim == 4 and tuple(c.v.shape[:2]) == (1, c.tokens)),
    ("value heads must be a positive multiple of the q/k heads", lambda c: 0 < c.H <= c.HV and c.HV % c.H == 0),
    ("A_log and dt_bias need one entry per value head",
     lambda c: c.gating is None or c.gating[0].shape[0] == c.gating[1].shape[0] == c.HV),
    ("gate or beta shape is incompatible", lambda c: c.g.numel() == c.beta.numel() == c.tokens * c.HV),
    ("gate and beta heads must be contiguous", lambda c: c.g2.stride(1) == 1 and c.beta2.stride(1) == 1),
    (f"spec_query_len must be in [1, {MAX_SPEC_QUERY_LEN}]", lambda c: 0 < c.window <= MAX_SPEC_QUERY_LEN),
    ("q and k heads must be contiguous", lambda c: all(t.stride(-1) == 1 and t.stride(-2) == c.K for t in (c.q, c.k))),
    ("v heads must be contiguous", lambda c: c.v.stride(-1) == 1 and c.v.stride(-2) == c.V),
    ("checkpoint must be four-dimensional", lambda c: c.checkpoint.ndim == 4),
    ("checkpoint shape is incompatible", lambda c: tuple(c.checkpoint.shape[1:]) == (c.HV, c.V, c.K)),
)

_TYPED_RECORD_RULES = (
    ("typed record geometry is incompatible",
     lambda c: c.planes.correction.ndim == 4
     and tuple(c.planes.correction.shape[1:]) == (c.HV, c.window, c.V)
     and tuple(c.planes.key.shape) == (c.planes.correction.shape[0], c.H, c.window, c.K)
     and tuple(c.planes.decay.shape) == (c.planes.correction.shape[0], c.HV, c.window)),
    ("correction and decay records must remain FP32",
     lambda c: c.planes.correction.dtype == c.planes.decay.dtype == torch.float32),
    ("low-precision key records require already-normalized input dtype",
     lambda c: _key_dtype_ok(c.planes.key.dtype)
     and (c.planes.key.dtype == torch.float32 or (c.normalized and c.planes.key.dtype == c.k.dtype))),
    ("typed record innermost dimensions must be contiguous",
     lambda c: all(t.stride(-1) == 1 for t in (c.planes.correction, c.planes.key, c.planes.decay))),
)

_PACKED_RECORD_RULES = (
    ("packed replay record shape is incompatible",
     lambda c: c.records.ndim == 4 and tuple(c.records.shape[1:]) == (c.HV, c.window, c.V + c.K + 1)),
    ("packed records must remain FP32", lambda c: c.records.dtype == torch.float32),
    ("packed record elements must be contiguous", lambda c: c.records.stride(-1) == 1),
)

_BATCH_RULES = (
    ("replay buffer has no rows", lambda c: c.planes.correction.shape[0] >= 1),
    ("state indices must be one-dimensional", lambda c: c.indices.ndim == 1),
    ("query metadata is incompatible", lambda c: c.qsl.ndim == 1 and c.qsl.shape[0] == c.rows + 1),
    ("speculative decode input exceeds its activation capacity", lambda c: c.tokens <= c.rows * c.window),
    ("inputs must be on the same device",
     lambda c: all(t.device == c.q.device for t in c.tensors()) and (c.out is None or c.out.device == c.q.device)),
)


def _kernel_rules(c: _VerifyCall) -> tuple:
    """What the gfx950 kernels are built for (checked when there is work)."""
    named = (("activation", c.q), ("output", c.out), ("gate", c.g2), ("beta", c.beta2), ("checkpoint", c.checkpoint))
    chunk = 16 // c.checkpoint.element_size()
    return (
        ("q, k and v must share one activation dtype", lambda: c.q.dtype == c.k.dtype == c.v.dtype),
        *((f"{name} dtype {t.dtype} is not supported", lambda t=t: t.dtype in _FLOAT_TYPES) for name, t in named),
        ("query offsets and state indices must be int32 or int64",
         lambda: c.qsl.dtype in _INDEX_TYPES and c.indices.dtype in _INDEX_TYPES),
        ("verify runs on a HIP device", lambda: c.q.device.type == "cuda"),
        (f"checkpoint rows must be contiguous, 16-byte aligned and K <= {MAX_KEY_DIM} a multiple of {chunk}",
         lambda: c.K <= MAX_KEY_DIM and c.K % chunk == 0 and c.checkpoint.stride(3) == 1
         and all(s % chunk == 0 for s in c.checkpoint.stride()[:3]) and c.checkpoint.data_ptr() % 16 == 0),
    )


def _check_verify(c: _VerifyCall) -> None:
    enforce(_ACTIVATION_RULES, c)
    enforce(_TYPED_RECORD_RULES if c.typed else _PACKED_RECORD_RULES, c)
    enforce(_BATCH_RULES, c)


def _verify_config(c: _VerifyCall, out: torch.Tensor) -> tuple:
    """The 28 integer fields of the reference's GDN_VERIFY_FIELDS
    (csrc/common.h:8-36), in their order."""
    p = c.planes
    # Packed records: the key and decay planes share the correction's strides.
    key_strides = p.key.stride()[:3]
    decay_strides = p.decay.stride()[:3]
    return (c.rows, c.tokens, c.H, c.HV, c.window, c.checkpoint.shape[0], p.correction.shape[0], NULL_BLOCK_ID,
            c.q.stride(1), c.k.stride(1), c.v.stride(1), c.g2.stride(0), c.beta2.stride(0),
            *c.checkpoint.stride()[:3], *p.correction.stride()[:3], *key_strides, *decay_strides,
            out.stride(1), c.qsl.stride(0), c.indices.stride(0))


def _verify_spec(c: _VerifyCall, out, scale, *, pending=None) -> _LaunchSpec:
    p = c.planes
    config = _verify_config(c, out)
    ext = N.VerifyExt(
        key_dim=c.K, value_dim=c.V, act_dtype=N.dtype_code(c.q.dtype), beta_dtype=N.dtype_code(c.beta2.dtype),
        g_dtype=N.dtype_code(c.g2.dtype), state_dtype=N.dtype_code(c.checkpoint.dtype),
        key_record_dtype=N.dtype_code(torch.float32 if p.packed else p.key.dtype),
        qsl_dtype=N.dtype_code(c.qsl.dtype), index_dtype=N.dtype_code(c.indices.dtype),
        qk_l2norm=0 if c.normalized else 1, key_per_value_head=1 if p.packed else 0,
        out_dtype=N.dtype_code(out.dtype), state_cache_retain=c.retain_field,
    )
    cfg = N.i64_array(config)
    lib = _lib()
    inputs = (c.q.data_ptr(), c.k.data_ptr(), c.v.data_ptr(), c.g2.data_ptr(), c.beta2.data_ptr())
    common = (c.checkpoint.data_ptr(), p.correction.data_ptr(), p.key.data_ptr() + p.key_offset,
              p.decay.data_ptr() + p.decay_offset, out.data_ptr(), c.qsl.data_ptr(), c.indices.data_ptr(), cfg,
              N.VERIFY_CONFIG_FIELDS, float(scale), ctypes.byref(ext))
    keep = (c.q, c.k, c.v, c.g2, c.beta2, c.checkpoint, p.correction, p.key, p.decay, out, c.qsl, c.indices, cfg, ext)
    if pending is not None:
        struct, held = pending
        fn, args = lib.gdn_recoverssm_verify_deferred, inputs + common + (ctypes.byref(struct),)
        keep += (struct, held)
    elif c.gating is None:
        fn, args = lib.gdn_recoverssm_verify, inputs + common
    else:
        a_log, dt_bias, sp_beta, sp_threshold = c.gating
        require(a_log.device == dt_bias.device == c.q.device, "inputs must be on the same device")
        gext = N.GatingExt(a_log_dtype=N.dtype_code(a_log.dtype), dt_bias_dtype=N.dtype_code(dt_bias.dtype),
                           softplus_beta=sp_beta, softplus_threshold=sp_threshold)
        fn = lib.gdn_recoverssm_verify_gated
        args = inputs + (a_log.data_ptr(), dt_bias.data_ptr()) + common + (ctypes.byref(gext),)
        keep += (a_log, dt_bias, gext)
    spec = _LaunchSpec("verify", fn, args, c.q.device, keepalive=keep)
    spec.config = tuple(int(x) for x in config)
    spec.scale = float(scale)
    return spec


def _run_verify(c: _VerifyCall, scale, out, _collect, *, pending=None) -> torch.Tensor:
    """Checks, output allocation, the early return on an empty batch, the
    kernel checks, then the launch (or its spec into ``_collect``)."""
    _check_verify(c)
    want = (1, c.tokens, c.HV, c.V)
    out = torch.empty(want, dtype=c.v.dtype, device=c.v.device) if out is None else out
    require(tuple(out.shape) == want and out.stride()[2:] == (c.V, 1), "output shape or layout is incompatible")
    # Nothing to verify: done, unless pending commits still have to be applied.
    idle = c.rows == 0 or (c.tokens == 0 and pending is None)
    if not idle:
        c.out = out
        enforce(_kernel_rules(c))
        # The default scale is the reference's 1 / sqrt(K).
        _submit(_verify_spec(c, out, math.pow(c.K, -0.5) if scale is None else scale, pending=pending), _collect)
    return out


def _submit(spec: "_LaunchSpec", collect: list | None) -> None:
    """Launch now, or hand the spec to a caller that collects them."""
    if collect is not None:
        collect.append(spec)
        return
    spec.launch()


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
    state_cache_retain: int | None = None,
    _collect: list | None = None,
) -> torch.Tensor:
    """Verify a speculative window from each row's checkpoint page, which is
    only read (reference kernels.py:700-928).

    ``g`` (log decay) and ``beta``: [1, T, HV] or [T, HV]; ``q``, ``k``:
    [1, T, H, K]; ``v``: [1, T, HV, V]; ``checkpoint_state``: [pages, HV, V, K];
    ``replay_cache``: ``ReplayRecordBuffers`` or a packed FP32
    [rows, HV, spec_query_len, V + K + 1] tensor; ``query_start_loc`` [B + 1];
    ``state_indices`` [B] (a page <= 0 or past the pool is the null page: zero
    outputs, no records). ``scale`` defaults to K^-0.5. With
    ``qk_already_normalized=False`` q and k are L2-normalised in the kernel
    (eps 1e-6). Returns ``out`` [1, T, HV, V], allocated when not given.
    ``state_cache_retain`` (no counterpart in the reference) is this call's
    cache hint in bytes (see ``set_state_cache_retain``; None: the
    process-wide setting); results do not depend on it.
    """
    c = _VerifyCall(g, beta, q, k, v, checkpoint_state, replay_cache, query_start_loc, state_indices, spec_query_len,
                    qk_already_normalized, out, None, _retain_arg(state_cache_retain))
    return _run_verify(c, scale, out, _collect)


def _retain_arg(nbytes):
    if nbytes is not None and int(nbytes) < 0:
        fail("the retained state bytes must be >= 0")
    return None if nbytes is None else int(nbytes)


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
    state_cache_retain: int | None = None,
    _collect: list | None = None,
) -> torch.Tensor:
    """Verify with the layer's gating producer (and by default the q/k L2
    norm) computed in the kernel, as the gated verify of
    docs/reference/recoverssm_gdn_upstream.py:83-151.

    ``a``, ``b``: the raw gate projections ([1, T, HV] or [T, HV]); ``A_log``,
    ``dt_bias``: [HV]. Per token and value head, in FP32:
    g = -exp(A_log) * softplus(a + dt_bias) with vLLM's fused_gdn_gating
    softplus (``softplus_beta``, ``softplus_threshold``), and beta = sigmoid(b).
    It replaces the producers the layer runs before verify
    (spec_forward.py:91-96) and their round trip through memory.
    """
    enforce((
        ("A_log and dt_bias must be one-dimensional", lambda: A_log.ndim == 1 and dt_bias.ndim == 1),
        ("A_log and dt_bias must be contiguous", lambda: A_log.stride(0) == 1 and dt_bias.stride(0) == 1),
        ("softplus beta must be positive", lambda: float(softplus_beta) > 0.0),
    ))
    gating = (A_log, dt_bias, float(softplus_beta), float(softplus_threshold))
    c = _VerifyCall(a, b, q, k, v, checkpoint_state, replay_cache, query_start_loc, state_indices, spec_query_len,
                    qk_already_normalized, out, gating, _retain_arg(state_cache_retain))
    return _run_verify(c, scale, out, _collect)


# ---------------------------------------------------------------------------
# Deferred commit
# ---------------------------------------------------------------------------


@dataclass
class PendingCommit:
    """One layer's commit left for the next verify (``gdn_recoverssm_verify_deferred``).

    ``rows`` (int32, one entry per row of the next batch) names the pending
    row each next row continues, -1 for none; no two next rows may continue
    the same pending row (``continue_pending`` refuses a request id given
    twice). The plan arrays (source page,
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

    @property
    def plan(self) -> tuple:
        return (self.source, self.lengths, self.final, self.boundary, self.boundary_len)


def continue_pending(pending: Sequence[PendingCommit], previous_requests: Sequence, next_requests: Sequence):
    """Re-key one step's pending commits (one per layer) for the next batch.

    ``previous_requests[r]`` identifies the request in row r of the pending
    step and ``next_requests[b]`` the request in row b of the next batch (any
    hashable ids, host-side, as the scheduler holds them). Returns the pending
    commits with a shared row map (next row -> pending row of the same
    request, -1 for a new request) and the sorted pending rows whose request
    is not in the next batch: their commits are applied by no verify, so
    ``flush_deferred(rows=...)`` must fold them before their pages are reused.
    ``settle_deferred(next_state_indices, rows)`` folds those rows and also
    the continued ones whose next state index is not the pending final page
    (which the verify does not apply either), deciding on the device.
    """
    require(len(pending) > 0, "no pending commits to continue")
    num_rows = int(pending[0].num_rows)
    require(all(int(p.num_rows) == num_rows for p in pending), "pending commits of one step disagree on their rows")
    rows, left = _request_row_map(num_rows, previous_requests, next_requests, pending[0].rows.device)
    return tuple(replace(p, rows=rows) for p in pending), left


def _request_row_map(num_rows: int, previous_requests: Sequence, next_requests: Sequence, device):
    """The row map of a deferred step's next batch, keyed by request:
    ``previous_requests[r]`` is the request of pending row r (r < num_rows),
    ``next_requests[b]`` that of next row b. Returns (int32 tensor on
    ``device``: next row -> pending row of the same request, -1 for a new
    request; a single -1 for an empty batch, which the kernels never index)
    and the sorted pending rows whose request is not in the next batch."""
    require(len(previous_requests) >= num_rows, "previous request ids do not cover the pending rows")
    where = {}
    for r, req in enumerate(previous_requests[:num_rows]):
        require(req not in where, f"request {req!r} appears twice in the pending step")
        where[req] = r
    seen = set()
    mapping = []
    for req in next_requests:
        require(req not in seen, f"request {req!r} appears twice in the next batch")
        seen.add(req)
        mapping.append(where.get(req, -1))
    left = sorted(r for req, r in where.items() if req not in seen)
    return _to_device_rows(mapping if mapping else [-1], device), left


_PENDING_RULES = (
    ("the deferred commit needs typed record buffers",
     lambda p, recs: isinstance(p.records, ReplayRecordBuffers) and isinstance(recs, ReplayRecordBuffers)),
    ("the pending commit's records must not be the records this verify writes",
     lambda p, recs: p.records.correction.data_ptr() != recs.correction.data_ptr()),
    ("pending arrays must be contiguous one-dimensional int32",
     lambda p, recs: all(t.dtype == torch.int32 and t.ndim == 1 and t.stride(0) == 1 for t in (p.rows,) + p.plan)),
    ("pending plan arrays do not cover their rows",
     lambda p, recs: all(t.shape[0] >= int(p.num_rows) for t in p.plan)),
    ("the pending plan has more rows than its records", lambda p, recs: int(p.num_rows) <= p.records.correction.shape[0]),
    ("pending records do not match this layer's record geometry",
     lambda p, recs: p.records.correction.shape[1:] == recs.correction.shape[1:]
     and p.records.key.shape[1:] == recs.key.shape[1:]),
)


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
    enforce(_PENDING_RULES, pending, replay_cache)
    if int(pending.num_rows) <= 0:
        # Nothing is pending: the ordinary verify.
        return gdn_recoverssm_verify(g, beta, q, k, v, checkpoint_state=checkpoint_state, replay_cache=replay_cache,
                                     query_start_loc=query_start_loc, state_indices=state_indices,
                                     spec_query_len=spec_query_len, scale=scale,
                                     qk_already_normalized=qk_already_normalized, out=out, _collect=_collect)
    require(pending.rows.shape[0] >= state_indices.shape[0], "the pending row map does not cover the batch")
    rec = pending.records
    struct = N.PendingCommit(
        rows=pending.rows.data_ptr(), source=pending.source.data_ptr(), lengths=pending.lengths.data_ptr(),
        final_indices=pending.final.data_ptr(), boundary_indices=pending.boundary.data_ptr(),
        boundary_lengths=pending.boundary_len.data_ptr(), correction=rec.correction.data_ptr(),
        key=rec.key.data_ptr(), decay=rec.decay.data_ptr(), record_rows=rec.correction.shape[0],
        key_dtype=N.dtype_code(rec.key.dtype), key_per_value_head=0, num_rows=int(pending.num_rows),
    )
    for i in range(3):
        struct.corr_strides[i] = rec.correction.stride(i)
        struct.key_strides[i] = rec.key.stride(i)
        struct.decay_strides[i] = rec.decay.stride(i)
    c = _VerifyCall(g, beta, q, k, v, checkpoint_state, replay_cache, query_start_loc, state_indices, spec_query_len,
                    qk_already_normalized, out, None)
    return _run_verify(c, scale, out, _collect, pending=(struct, (pending, rec)))


def _settle_spec(lengths: torch.Tensor, finals: torch.Tensor, capacity: int, num_rows: int, rows: torch.Tensor,
                 nexts: Sequence, out: torch.Tensor, row_list: torch.Tensor, row_count: torch.Tensor) -> _LaunchSpec:
    """The launch (gdn_recoverssm_settle) that decides on the device what a
    settle of a deferred commit folds, for the plan groups of one plan:
    ``lengths`` / ``finals`` hold ``len(nexts)`` groups of ``capacity`` plan
    rows, ``nexts[g]`` is group g's next state indices (None: a group outside
    the next step). Group g's pending row r < ``num_rows`` is applied by the
    next verify when some next row b has rows[b] == r and nexts[g][b] is r's
    final page (the deferred verify's own test); ``out`` gets the plan's
    lengths with 0 for the applied rows, ``row_list`` / ``row_count`` the
    ascending rows left with a length in some group and their number, for a
    fold over them (``_fold_rows_spec``); the plan's length of every entry
    handed on that way becomes 0, so a later settle or flush does not fold it
    again. Nothing is synchronised with the host."""
    groups = len(nexts)
    require(1 <= groups <= N.SETTLE_MAX_GROUPS, f"a settle covers 1..{N.SETTLE_MAX_GROUPS} plan groups")
    require(0 <= num_rows <= min(capacity, N.SETTLE_MAX_ROWS),
            f"a settle covers at most {N.SETTLE_MAX_ROWS} pending rows")
    dev = out.device
    require(rows.dtype == torch.int32 and rows.is_contiguous() and rows.device == dev,
            "the pending row map must be a contiguous int32 tensor on the plan's device")
    table = (N.SettleNext * groups)()
    held = [lengths, finals, rows, out, row_list, row_count, table]
    for g, nxt in enumerate(nexts):
        if nxt is None:
            continue
        require(nxt.ndim == 1 and nxt.device == dev and nxt.dtype in (torch.int32, torch.int64),
                "next state indices must be a 1-D int32 or int64 tensor on the plan's device")
        require(rows.shape[0] >= nxt.shape[0], "the pending row map does not cover the next batch")
        table[g].state_indices = nxt.data_ptr()
        table[g].stride = nxt.stride(0) if nxt.shape[0] > 1 else 1
        table[g].rows = nxt.shape[0]
        table[g].dtype = N.dtype_code(nxt.dtype)
        held.append(nxt)
    args = (lengths.data_ptr(), finals.data_ptr(), groups, int(capacity), int(num_rows), rows.data_ptr(),
            rows.shape[0], table, out.data_ptr(), row_list.data_ptr(), row_count.data_ptr())
    return _LaunchSpec("settle", _lib().gdn_recoverssm_settle, args, dev, keepalive=tuple(held))


class _MarkFolded:
    """After an explicit fold of pending rows (a flush), their accepted
    lengths in the plan become 0, so a later flush or settle of the same plan
    folds them no more; launched in stream order, like a ``_LaunchSpec``.
    ``lengths`` holds ``groups`` plan groups of ``capacity`` rows; ``rows``
    (a device int32 tensor) names the folded rows of every group, None the
    first ``num_rows`` of each."""

    name = "mark_folded"

    def __init__(self, lengths: torch.Tensor, capacity: int, rows: torch.Tensor | None = None, num_rows: int = 0):
        self.view = lengths.view(-1, int(capacity))
        self.rows = None if rows is None else rows.long()
        self.num_rows = int(num_rows)

    def launch(self) -> None:
        if self.rows is None:
            self.view[:, :self.num_rows].zero_()
        else:
            self.view.index_fill_(1, self.rows, 0)


def _to_device_rows(values: list, device) -> torch.Tensor:
    """An int32 tensor of the host list ``values`` on ``device``, copied on
    the current stream from pinned memory without waiting for the device (the
    pinned staging block is not reused before the copy has run)."""
    if torch.device(device).type == "cpu":
        return torch.tensor(values, dtype=torch.int32)
    return torch.tensor(values, dtype=torch.int32, pin_memory=True).to(device, non_blocking=True)


# ---------------------------------------------------------------------------
# Commit launches shared by the single context and the grouped buckets
# ---------------------------------------------------------------------------


def _fill_plan_group(group, *, state_indices, query_start_loc, request_indices, block_table, num_computed_tokens,
                     block_size, num_blocks) -> None:
    """One gdn_plan_group: the step metadata of one cache group (grouped_commit.py:113-146)."""
    def bind(t, ptr, stride, dtype):
        setattr(group, ptr, t.data_ptr())
        setattr(group, stride, t.stride(0))
        setattr(group, dtype, N.dtype_code(t.dtype))

    bind(state_indices, "state_indices", "si_stride", "si_dtype")
    bind(query_start_loc, "query_start_loc", "qsl_stride", "qsl_dtype")
    if request_indices is not None:
        bind(request_indices, "request_indices", "map_stride", "map_dtype")
    if block_table is not None:
        group.block_table = block_table.data_ptr()
        group.table_row_stride, group.table_col_stride = block_table.stride()
        group.table_rows, group.table_width = block_table.shape
        group.table_dtype = N.dtype_code(block_table.dtype)
        bind(num_computed_tokens, "num_computed", "computed_stride", "computed_dtype")
        group.computed_len = num_computed_tokens.shape[0]
        group.block_size = int(block_size)
    else:
        group.block_size = 1
        group.table_width = 1
    group.num_blocks = int(num_blocks)


def _conv_spec(pages: LayerPages, *, source, source_dtype, source_stride, plan, layer_groups, capacity, rows,
               history, max_blocks, align, device, keep=()) -> _LaunchSpec:
    conv = pages.conv_states[0]
    require(conv.element_size() in (2, 4), "conv state elements must be 2 or 4 bytes")
    lengths, finals, boundaries, boundary_lens = plan
    args = (pages.conv_addrs.data_ptr(), pages.conv_block_strides.data_ptr(), pages.conv_dim_strides.data_ptr(),
            pages.conv_token_strides.data_ptr(), source.data_ptr(), source_dtype, source_stride, lengths.data_ptr(),
            finals.data_ptr(), boundaries.data_ptr(), boundary_lens.data_ptr(),
            None if layer_groups is None else layer_groups.data_ptr(), capacity, NULL_BLOCK_ID, rows,
            len(pages.conv_states), conv.shape[1], history, conv.shape[2], max_blocks, conv.element_size(),
            1 if align else 0)
    return _LaunchSpec("conv", _lib().gdn_recoverssm_conv_compact, args, device, keepalive=keep)


def _make_fold_spec(*, pages: LayerPages, record_rows, key_heads, key_dtype, rows, plan_capacity, num_blocks,
                    spec_query_len, layer_groups, source, plan) -> _LaunchSpec:
    """The fold launch (config = the 17 GDN_FOLD_FIELDS of csrc/common.h:37-54)."""
    ref = pages.checkpoints[0]
    _, HV, V, K = ref.shape
    chunk = 16 // ref.element_size()
    planes = pages.first_planes
    enforce((
        ("checkpoint dtype is not supported", lambda: ref.dtype in _FLOAT_TYPES),
        ("record key dtype is not supported", lambda: key_dtype in _FLOAT_TYPES),
        (f"checkpoint rows must be contiguous, 16-byte aligned, K <= {MAX_KEY_DIM} a multiple of {chunk}, V <= 1024",
         lambda: K <= MAX_KEY_DIM and K % chunk == 0 and ref.stride(3) == 1
         and all(s % chunk == 0 for s in ref.stride()[:3]) and V <= 1024),
    ))
    config = (rows, len(pages.checkpoints), HV, key_heads, spec_query_len, num_blocks, record_rows, plan_capacity,
              NULL_BLOCK_ID, ref.stride(1), ref.stride(2), *planes.correction.stride()[1:3], *planes.key.stride()[1:3],
              *planes.decay.stride()[1:3])
    ext = N.FoldExt(key_dim=K, value_dim=V, state_dtype=N.dtype_code(ref.dtype), key_dtype=N.dtype_code(key_dtype),
                    source_dtype=N.dtype_code(source.dtype), reserved=0, source_stride=source.stride(0),
                    state_k_stride=ref.stride(3))
    cfg = N.i64_array(config)
    tables = pages.device_tables
    args = (ref.data_ptr(), planes.correction.data_ptr(), planes.key.data_ptr(), planes.decay.data_ptr(),
            *(t.data_ptr() for t in tables), None if layer_groups is None else layer_groups.data_ptr(),
            source.data_ptr(), *(t.data_ptr() for t in plan), cfg, N.FOLD_CONFIG_FIELDS, ctypes.byref(ext))
    spec = _LaunchSpec("fold", _lib().gdn_recoverssm_fold, args, ref.device,
                       keepalive=(pages, layer_groups, source, *plan, cfg, ext))
    spec.config = tuple(int(x) for x in config)
    spec.ext = ext
    return spec


def _fold_rows_spec(spec: _LaunchSpec, rows: torch.Tensor, count: torch.Tensor | None = None, *,
                    lengths: torch.Tensor | None = None, listed: int | None = None) -> _LaunchSpec:
    """The same fold over the listed plan rows only: ``rows`` is a strictly
    increasing int32 tensor on the fold's device (the extension block's row
    list), so the launch has a workgroup per (layer, listed row, head)
    instead of one per row of the plan. With ``count`` (a device int32 the
    device wrote) only the first ``count`` of ``listed`` entries (all of
    ``rows`` by default) are folded, by a fixed grid that loops over their
    tiles. ``lengths`` replaces the plan's accepted lengths."""
    ext = N.FoldExt.from_buffer_copy(spec.ext)
    ext.row_list = rows.data_ptr()
    ext.row_list_len = rows.numel() if listed is None else int(listed)
    held = (rows, ext)
    if count is not None:
        ext.row_count = count.data_ptr()
        held += (count,)
    args = list(spec.args[:-1]) + [ctypes.byref(ext)]
    if lengths is not None:
        args[_FOLD_LENGTHS_ARG] = lengths.data_ptr()
        held += (lengths,)
    out = _LaunchSpec(spec.name, spec.fn, tuple(args), spec.device, keepalive=spec.keepalive + held)
    out.config, out.ext = spec.config, ext
    return out


def _picked_rows(rows, num_rows: int, device) -> torch.Tensor | None:
    """Pending rows named by a flush, checked against the plan's rows, as a
    sorted int32 tensor of distinct rows on ``device`` (None when empty)."""
    # Host rows (a list, or a tensor read back once); checked and sorted here.
    pick = rows.reshape(-1).tolist() if isinstance(rows, torch.Tensor) else [int(r) for r in rows]
    require(all(0 <= r < num_rows for r in pick), "flushed rows must be rows of the pending plan")
    if not pick:
        return None
    return _to_device_rows(sorted(set(pick)), device)


# Positions in the fold's argument tuple: 4 reference tensors, 8 tables,
# layer groups, source, 4 plan arrays, config, config length, extension.
_FOLD_LENGTHS_ARG = 14
_FOLD_PLAN_ARGS = slice(13, 18)


def _fuse_plan_fold(plan: _LaunchSpec, fold: _LaunchSpec) -> _LaunchSpec:
    """``gdn_recoverssm_plan_fold``: a plan launch and the fold launch that
    reads its arrays as one launch with identical results (each fold
    workgroup plans its own row; extra workgroups store the plan arrays)."""
    launch = N.plan_launch(plan.args)
    args = ((ctypes.byref(launch),) + tuple(fold.args[:_FOLD_PLAN_ARGS.start])
            + tuple(fold.args[_FOLD_PLAN_ARGS.stop:]))
    spec = _LaunchSpec("plan_fold", _lib().gdn_recoverssm_plan_fold, args, fold.device,
                       keepalive=(plan.keepalive, fold.keepalive, launch))
    spec.config = fold.config
    return spec


# ---------------------------------------------------------------------------
# Single-context commit (reference kernels.py:1399-2052)
# ---------------------------------------------------------------------------


def _commit_rules(ctx, accepted, state_indices, qsl, request_indices, block_table, num_computed, block_size):
    align_parts = (block_table, num_computed, block_size)
    batch = state_indices.shape[0]
    device = ctx.checkpoints[0].device
    tensors = (accepted, state_indices, qsl, request_indices, block_table, num_computed)
    return (
        ("state indices must be one-dimensional", lambda: state_indices.ndim == 1),
        ("commit batch exceeds its plan capacity", lambda: batch <= ctx.commit_lens.shape[0]),
        ("commit metadata is incompatible", lambda: qsl.ndim == 1 and qsl.shape[0] == batch + 1),
        ("request mapping is too short", lambda: request_indices is None or request_indices.shape[0] >= batch),
        ("accepted-token counts are too short",
         lambda: accepted.ndim == 1 and (request_indices is not None or accepted.shape[0] >= batch)),
        ("align metadata is incomplete",
         lambda: all(x is None for x in align_parts) or all(x is not None for x in align_parts)),
        ("align block size must cover one speculative window",
         lambda: block_size is None or block_size >= ctx.spec_query_len),
        ("block table must be two-dimensional with a positive width",
         lambda: block_table is None or (block_table.dim() == 2 and block_table.size(-1) >= 1)),
        ("commit inputs must be on the same device",
         lambda: all(t is None or t.device == device for t in tensors)),
        ("the commit runs on a HIP device", lambda: device.type == "cuda"),
    )


def _conv_dim_first_default() -> bool:
    """Conv pages are channel-major unless an installed vLLM says otherwise."""
    try:
        from vllm.model_executor.layers.mamba.mamba_utils import is_conv_state_dim_first
    except ImportError:
        return True
    return bool(is_conv_state_dim_first())


class GDNRecoverSSMCommitContext:
    """The commit of one cache epoch: every layer's checkpoint pages, conv
    states and record planes bound once (their device address tables built
    once), and the plan arrays of up to ``max_num_reqs`` rows, reused by every
    step. ``commit`` folds each row's accepted prefix into its final page (and
    the align-mode boundary snapshot) and compacts the conv states."""

    def __init__(self, pages: LayerPages, *, spec_query_len: int, max_num_reqs: int, conv_history_len: int,
                 record_layout: str, num_key_heads: int, key_dtype):
        self.pages = pages
        self.spec_query_len = int(spec_query_len)
        self.num_blocks = int(pages.checkpoints[0].shape[0])
        self.conv_history_len = int(conv_history_len)
        self.record_layout = record_layout
        self.num_key_heads = int(num_key_heads)
        self.key_dtype = key_dtype
        self.records = list(pages.records)
        self.record_rows = int(pages.first_planes.correction.shape[0])
        self.record_bytes = sum(record_nbytes(r) for r in pages.records)
        dev = pages.checkpoints[0].device
        plan = {name: torch.zeros(max_num_reqs, dtype=torch.int32, device=dev) for name in (
            "commit_lens", "final_state_indices", "boundary_state_indices", "boundary_recovery_lens", "align_valid",
            "align_col", "plan_source")}
        self.__dict__.update(plan)
        # Rows of the next batch continue the same rows of a pending commit.
        self.pending_rows = torch.arange(max_num_reqs, dtype=torch.int32, device=dev)
        # What a settle folds (settle_deferred): lengths, listed rows, count.
        self.settle_lens = torch.zeros(max_num_reqs, dtype=torch.int32, device=dev)
        self.settle_rows = torch.zeros(max(1, max_num_reqs), dtype=torch.int32, device=dev)
        self.settle_count = torch.zeros(1, dtype=torch.int32, device=dev)

    # The reference context's table attributes, served from the bound pages.
    conv_states = property(lambda self: self.pages.conv_states)
    checkpoints = property(lambda self: self.pages.checkpoints)
    replays = property(lambda self: self.pages.records)
    conv_state_base_addrs = property(lambda self: self.pages.conv_addrs)
    conv_state_block_strides = property(lambda self: self.pages.conv_block_strides)
    conv_state_dim_strides = property(lambda self: self.pages.conv_dim_strides)
    conv_state_token_strides = property(lambda self: self.pages.conv_token_strides)
    state_base_addrs = property(lambda self: self.pages.state_addrs)
    state_block_strides = property(lambda self: self.pages.state_block_strides)
    correction_base_addrs = property(lambda self: self.pages.correction_addrs)
    correction_block_strides = property(lambda self: self.pages.correction_block_strides)
    replay_base_addrs = correction_base_addrs
    replay_block_strides = correction_block_strides
    key_base_addrs = property(lambda self: self.pages.key_addrs)
    key_block_strides = property(lambda self: self.pages.key_block_strides)
    decay_base_addrs = property(lambda self: self.pages.decay_addrs)
    decay_block_strides = property(lambda self: self.pages.decay_block_strides)

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
        """Bind the layers' pages and records (conv states token-major when
        ``conv_dim_first`` is false) and allocate the plan arrays."""
        # Token-major conv pages are viewed channel-major: the kernels take strides.
        conv_states = list(conv_states) if conv_dim_first else [c.mT for c in conv_states]
        typed = [isinstance(r, ReplayRecordBuffers) for r in replays]
        require(all(typed) or not any(typed), "packed and typed records cannot share a commit context")
        check_layers(conv_states, checkpoints, replays, window=spec_query_len, typed=bool(typed and typed[0]),
                     max_window=MAX_SPEC_QUERY_LEN)
        pages = LayerPages(conv_states, checkpoints, replays, checkpoints[0].device)
        first = pages.first_planes
        return cls(pages, spec_query_len=spec_query_len, max_num_reqs=max_num_reqs,
                   conv_history_len=conv_states[0].shape[2] - spec_query_len + 1,
                   record_layout="packed" if first.packed else "soa",
                   num_key_heads=checkpoints[0].shape[1] if first.packed else first.key.shape[1],
                   key_dtype=torch.float32 if first.packed else first.key.dtype)

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
        """The context of live layers whose ``kv_cache`` is (conv state,
        checkpoint). Records are row-indexed step scratch, not cache pages:
        they are allocated here, ``record_rows`` (default ``max_num_reqs``)
        rows per layer, and handed to each layer as
        ``layer._gdn_recoverssm_records`` for its verify to write."""
        caches = [tuple(layer.kv_cache) for layer in layers]
        if {len(c) for c in caches} != {2}:
            raise ValueError("GDN RecoverSSM expects conv and checkpoint pages; the replay records live outside the cache")
        conv_pages, state_pages = (list(pages) for pages in zip(*caches))
        _, HV, V, K = state_pages[0].shape
        rows = int(record_rows or max_num_reqs)
        key_heads = HV if num_key_heads is None else int(num_key_heads)
        records = [ReplayRecordBuffers.allocate(rows, HV, key_heads, spec_query_len, V, K, device=state_pages[0].device,
                                                key_dtype=key_dtype or torch.float32) for _ in caches]
        layout = _conv_dim_first_default() if conv_dim_first is None else conv_dim_first
        context = cls.from_tensors(conv_pages, state_pages, records, spec_query_len=spec_query_len,
                                   max_num_reqs=max_num_reqs, conv_dim_first=layout)
        for layer, record in zip(layers, records):
            layer._gdn_recoverssm_records = record
        return context

    # -- preparation (nothing is compiled at run time: these only check that
    # -- every serving signature is accepted and its entry point is there) --

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
        """The launch specs of one step's commit, not launched."""
        specs: list = []
        self.commit(num_accepted_tokens, state_indices, query_start_loc, request_indices, block_table,
                    num_computed_tokens, mamba_block_size, commit_conv, specs)
        return tuple(specs)

    def prepare_verify(self, *, activation_dtype, state_table_width: int | None = None, device=None) -> list:
        """Check the serving verify signatures of this epoch without touching
        a page: a contiguous and a combined-QKV value view (the fused
        projection's token stride), each with an FP32 and an activation-typed
        beta; one report dict per signature."""
        device = device or self.checkpoints[0].device
        _, HV, V, K = self.checkpoints[0].shape
        H, Q = self.num_key_heads, self.spec_query_len
        width = int(state_table_width or Q)
        require(width > 0, "verify preparation requires a positive table stride")

        def blank(*shape, dtype=activation_dtype):
            return torch.empty(shape, dtype=dtype, device=device)

        q, k = blank(1, Q, H, K), blank(1, Q, H, K)
        g, out = blank(1, Q, HV, dtype=torch.float32), blank(1, Q, HV, V)
        table, offsets = blank(1, width, dtype=torch.int32), blank(2, dtype=torch.int32)
        fused = blank(1, Q, 2 * H * K + HV * V)
        value_views = {False: blank(1, Q, HV, V), True: fused[:, :, 2 * H * K:].view(1, Q, HV, V)}
        # What every signature of this epoch shares, then one entry per signature.
        epoch = {"activation_dtype": str(activation_dtype), "state_index_stride": width,
                 "state_blocks": self.num_blocks, "record_rows": self.record_rows, "num_value_heads": HV,
                 "num_key_heads": H, "window": Q}
        signatures = [(value, beta_dtype) for value in value_views.values()
                      for beta_dtype in dict.fromkeys((torch.float32, activation_dtype))]
        report = []
        for value, beta_dtype in signatures:
            specs: list = []
            gdn_recoverssm_verify(g, blank(1, Q, HV, dtype=beta_dtype), q, k, value,
                                  checkpoint_state=self.checkpoints[0], replay_cache=self.records[0],
                                  query_start_loc=offsets, state_indices=table[:, 0], spec_query_len=Q,
                                  qk_already_normalized=True, out=out, _collect=specs)
            _ = [spec.compile_only() for spec in specs]
            report.append({**epoch, "beta_dtype": str(beta_dtype), "value_token_stride": value.stride(1)})
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
        """Check the none / align commit signature for every batch size up to
        ``capacity`` (and the record rows); returns the row counts checked."""
        require(not align_mode or (mamba_block_size or 0) >= self.spec_query_len,
                "align preparation requires the runtime block size")
        width = int(block_table_width or state_table_width)

        def blank(shape, dtype):
            return torch.empty(shape, dtype=dtype, device=device)

        def signature(n: int) -> tuple:
            """Placeholder commit inputs of n rows with the serving dtypes and strides."""
            return (blank(n, accepted_dtype), blank((n, state_table_width), state_index_dtype)[:, 0],
                    blank(n + 1, query_index_dtype), blank(n, request_index_dtype) if request_mapping else None,
                    blank((n, width), state_index_dtype) if align_mode else None,
                    blank(n, computed_dtype) if align_mode else None, mamba_block_size if align_mode else None)

        batch_sizes = list(range(1, min(capacity, self.record_rows) + 1))
        for n in batch_sizes:
            _ = [spec.compile_only() for spec in self.make_commit_specs(*signature(n))]
        return batch_sizes

    # -- the commit --

    def _plan_spec(self, accepted, state_indices, qsl, request_indices, block_table, num_computed, block_size,
                   rows) -> _LaunchSpec:
        groups = N.PlanGroups()
        _fill_plan_group(groups[0], state_indices=state_indices, query_start_loc=qsl, request_indices=request_indices,
                         block_table=block_table, num_computed_tokens=num_computed, block_size=block_size,
                         num_blocks=self.num_blocks)
        align = block_table is not None
        args = (accepted.data_ptr(), N.dtype_code(accepted.dtype), accepted.stride(0), accepted.shape[0], groups, 1,
                self.plan_source.data_ptr(), self.commit_lens.data_ptr(), self.final_state_indices.data_ptr(),
                self.boundary_state_indices.data_ptr(), self.boundary_recovery_lens.data_ptr(),
                self.align_valid.data_ptr(), self.align_col.data_ptr(), None, N.DT_I32, 0, None, None, 0, rows,
                self.commit_lens.shape[0], NULL_BLOCK_ID, self.spec_query_len, N.PLAN_ALIGN if align else 0)
        keep = (groups, accepted, state_indices, qsl, request_indices, block_table, num_computed)
        return _LaunchSpec("plan", _lib().gdn_recoverssm_plan, args, state_indices.device, keepalive=keep)

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
        """Fold every committed row's accepted prefix into its final page (and
        its boundary snapshot in align mode) in every layer, then compact the
        conv states. ``_fold_source`` (internal) keeps the plan and the fold
        apart, the fold reading its source pages from that array."""
        rows = state_indices.shape[0]
        if rows == 0:
            return
        enforce(_commit_rules(self, num_accepted_tokens, state_indices, query_start_loc, request_indices,
                              block_table, num_computed_tokens, mamba_block_size))
        align = block_table is not None
        device = self.checkpoints[0].device
        plan = self._plan_spec(num_accepted_tokens, state_indices, query_start_loc, request_indices, block_table,
                               num_computed_tokens, mamba_block_size, rows)
        arrays = (self.commit_lens, self.final_state_indices, self.boundary_state_indices, self.boundary_recovery_lens)
        conv = None
        if commit_conv:
            conv = _conv_spec(self.pages, source=state_indices, source_dtype=N.dtype_code(state_indices.dtype),
                              source_stride=state_indices.stride(0), plan=arrays, layer_groups=None,
                              capacity=self.commit_lens.shape[0], rows=rows, history=self.conv_history_len,
                              max_blocks=self.num_blocks, align=align, device=device,
                              keep=(state_indices, query_start_loc))
        fold = _make_fold_spec(pages=self.pages, record_rows=self.record_rows, key_heads=self.num_key_heads,
                               key_dtype=self.key_dtype, rows=rows, plan_capacity=self.commit_lens.shape[0],
                               num_blocks=self.num_blocks, spec_query_len=self.spec_query_len, layer_groups=None,
                               source=state_indices if _fold_source is None else _fold_source, plan=arrays)
        if _fold_source is None:
            # One launch plans and folds; the conv compaction reads the plan it stores.
            specs = [_fuse_plan_fold(plan, fold)] + ([conv] if conv else [])
        else:
            specs = [plan] + ([conv] if conv else []) + [fold]
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
        """Plan the commit and compact the conv states now, and leave the fold
        to the next step's ``gdn_recoverssm_verify_deferred``: returns one
        ``PendingCommit`` per layer. ``flush_deferred`` folds instead (the
        last step, or rows whose requests left)."""
        require(self.record_layout == "soa", "the deferred commit needs typed record buffers")
        specs: list = []
        self.commit(num_accepted_tokens, state_indices, query_start_loc, request_indices, block_table,
                    num_computed_tokens, mamba_block_size, commit_conv, specs, _fold_source=self.plan_source)
        self._deferred_fold = next(sp for sp in specs if sp.name == "fold")
        self._deferred_rows = int(state_indices.shape[0])
        now = [sp for sp in specs if sp.name != "fold"]
        if _collect is not None:
            _collect.extend(now)
        else:
            for sp in now:
                sp.launch()
        plan = (self.plan_source, self.commit_lens, self.final_state_indices, self.boundary_state_indices,
                self.boundary_recovery_lens)
        return tuple(PendingCommit(self.pending_rows, *plan, rec, num_rows=self._deferred_rows)
                     for rec in self.records)

    def settle_deferred(self, next_state_indices: torch.Tensor, rows: torch.Tensor | None = None,
                        _collect: list | None = None) -> None:
        """Fold now, with the ordinary fold, every row of the last
        ``commit_deferred`` plan that the next deferred verify will not apply:
        the next verify applies pending row ``r`` only through a next row
        ``b`` with ``rows[b] == r`` whose state index ``next_state_indices[b]``
        is that commit's final page. Rows whose request left, and continued
        requests whose next state index names another page, are folded here,
        so no commit is lost. Decided on the device (no host synchronisation);
        call it before the next verify. ``rows`` is the row map of the
        pending commits (``continue_pending``), the in-place map by default.
        """
        spec = getattr(self, "_deferred_fold", None)
        require(spec is not None, "no deferred commit to flush")
        rows = self.pending_rows if rows is None else rows
        require(next_state_indices.ndim == 1 and rows.shape[0] >= next_state_indices.shape[0],
                "the pending row map does not cover the next batch")
        # The device decides which rows to fold, lists them in the context's
        # own arrays and marks them folded in the plan (the rows the verifies
        # apply keep their lengths); the fold then covers the listed rows only.
        num = self._deferred_rows
        if num == 0:
            return  # nothing is pending
        _submit(_settle_spec(self.commit_lens, self.final_state_indices, self.commit_lens.shape[0], num, rows,
                             [next_state_indices], self.settle_lens, self.settle_rows, self.settle_count), _collect)
        _submit(_fold_rows_spec(spec, self.settle_rows, self.settle_count, lengths=self.settle_lens, listed=num),
                _collect)

    def flush_deferred(self, rows: Sequence[int] | torch.Tensor | None = None, _collect: list | None = None) -> None:
        """Apply the last ``commit_deferred`` plan with the ordinary fold.

        ``rows=None`` folds every planned row (a step that runs no verify
        after it, e.g. the end of a batch); a list of pending rows folds only
        those (rows whose request left the batch, see ``continue_pending``),
        leaving the rest to the next verify. The folded rows are then marked
        in the plan (accepted length 0), so a later flush, settle or verify
        does not apply them again (a verify then reads the folded final
        page); a row the next verify has applied is not marked (every layer's
        verify reads the plan), so it must not be flushed afterwards.
        """
        spec = getattr(self, "_deferred_fold", None)
        require(spec is not None, "no deferred commit to flush")
        if rows is not None:
            # The same fold over the picked rows only (a launch sized to them).
            picked = _picked_rows(rows, self._deferred_rows, self.commit_lens.device)
            if picked is None:
                return
            spec = _fold_rows_spec(spec, picked)
            mark = _MarkFolded(self.commit_lens, self.commit_lens.shape[0], picked)
        else:
            mark = _MarkFolded(self.commit_lens, self.commit_lens.shape[0], num_rows=self._deferred_rows)
        _submit(spec, _collect)
        _submit(mark, _collect)


__all__ = [
    "GDNRecoverSSMCommitContext",
    "PendingCommit",
    "ReplayRecordBuffers",
    "continue_pending",
    "gdn_recoverssm_verify",
    "gdn_recoverssm_verify_deferred",
    "gdn_recoverssm_verify_gated",
    "record_geometry_bytes",
    "record_nbytes",
]

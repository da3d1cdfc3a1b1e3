"""The reference's native operator ABI as torch operators.

The reference registers ``gdn_recoverssm_ac::abi_version``, ``verify`` and
``fold`` (csrc/ops.cpp:243-257) and its backend hook calls them through
``torch.ops.gdn_recoverssm_ac`` with the 28-field verify and 17-field fold
configs (ascendc_backend.py:98-212). This module registers the same three
operators, with the same schemas and mutation annotations, under
``torch.ops.gdn_recoverssm_hip``: a backend written against the reference's
namespace switches by name.

Before anything is launched each operator checks the config against its
tensors, as the reference's operators do (csrc/ops.cpp:91-141 for verify,
:171-228 for fold), for the wider set this library implements (any head dims
the kernels take, FP16 as well, int64 metadata, column views): the config
length and reserved null page, devices, dtypes, shapes, row capacities,
record geometry, contiguity, and every stride the config carries against the
tensor's own. A violation raises ``ValueError("GDN RecoverSSM: ...")`` naming
the check (``validate_verify`` / ``validate_fold`` are the checks alone); a
failed launch raises ``RuntimeError``. The element types and head dims the C
ABI takes beside the config come from the tensors. The Meta kernels do
nothing, as the reference's do.

Importing the module registers the operators (once per process).
"""

from __future__ import annotations

import ctypes

import torch

from . import _native as N

NAMESPACE = "gdn_recoverssm_hip"

# The reference's schemas (csrc/ops.cpp:244-246), unchanged.
ABI_SCHEMA = "abi_version() -> int"
VERIFY_SCHEMA = (
    "verify(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, Tensor state, Tensor(a!) correction, "
    "Tensor(b!) key, Tensor(c!) decay, Tensor(d!) out, Tensor qsl, Tensor indices, int[] config, float scale) -> ()"
)
FOLD_SCHEMA = (
    "fold(Tensor(a!) state, Tensor correction, Tensor key, Tensor decay, Tensor state_addrs, "
    "Tensor state_block_strides, Tensor corr_addrs, Tensor corr_block_strides, Tensor key_addrs, "
    "Tensor key_block_strides, Tensor decay_addrs, Tensor decay_block_strides, Tensor layer_groups, "
    "Tensor source, Tensor lengths, Tensor final_indices, Tensor boundary_indices, Tensor boundary_lengths, "
    "int[] config) -> ()"
)


def _abi_version() -> int:
    return int(N.load().gdn_recoverssm_abi_version())


_FLOAT = (torch.float32, torch.bfloat16, torch.float16)
_INDEX = (torch.int32, torch.int64)


def _checks(op: str, table) -> None:
    """Raise ``ValueError`` for the first failed (check class, condition) row.

    Conditions are callables, evaluated in order, so a later row may rely on
    the shapes an earlier one established."""
    for what, cond in table:
        if not cond():
            raise ValueError(f"GDN RecoverSSM: {op} operator: {what}")


def validate_verify(q, k, v, g, beta, state, correction, key, decay, out, qsl, indices, config) -> None:
    """The verify operator's checks (csrc/ops.cpp:91-141), in its order."""
    c = list(config)
    n = dict(zip(("rows", "tokens", "heads", "value_heads", "Q", "blocks", "record_rows", "null_block"), c[:8]))
    tensors = (k, v, g, beta, state, correction, key, decay, out, qsl, indices)
    act = q.dtype
    _checks("verify", (
        ("config must have 28 fields", lambda: len(c) == 28),
        ("physical page zero is the null page (config null_block must be 0)", lambda: c[7] == 0),
        ("all tensors must be on the same device", lambda: all(t.device == q.device for t in tensors)),
        ("dtype: q, k and v share one FP32/BF16/FP16 activation dtype", lambda: act in _FLOAT and k.dtype == act
         and v.dtype == act),
        ("dtype: out, key records, beta and g are FP32 or the activation dtype",
         lambda: all(t.dtype in (act, torch.float32) for t in (out, key, beta, g))),
        ("dtype: checkpoint FP32/BF16/FP16, correction and decay FP32",
         lambda: state.dtype in _FLOAT and correction.dtype == torch.float32 and decay.dtype == torch.float32),
        ("dtype: query_start_loc and state indices int32 or int64",
         lambda: qsl.dtype in _INDEX and indices.dtype in _INDEX),
        ("activation shape: q [1, T, H, K], k like q, v [1, T, HV, V], out like v",
         lambda: q.dim() == 4 and q.size(0) == 1 and k.shape == q.shape and v.dim() == 4 and v.size(0) == 1
         and v.size(1) == q.size(1) and out.shape == v.shape),
        ("verify geometry: config tokens/heads/value heads/window disagree with the tensors",
         lambda: n["rows"] > 0 and n["tokens"] == q.size(1) and n["heads"] == q.size(2) > 0
         and n["value_heads"] == v.size(2) and n["value_heads"] % n["heads"] == 0 and 0 < n["Q"] <= 8
         and n["tokens"] <= n["rows"] * n["Q"]),
        ("state geometry: checkpoint must be [blocks, HV, V, K] with K contiguous",
         lambda: state.dim() == 4 and tuple(state.shape) == (n["blocks"], n["value_heads"], v.size(3), q.size(3))
         and state.stride(3) == 1 and state.stride(2) >= q.size(3)),
        ("row capacity: query_start_loc needs rows + 1 entries and state indices rows",
         lambda: qsl.dim() == 1 and qsl.numel() >= n["rows"] + 1 and indices.dim() == 1
         and indices.numel() >= n["rows"]),
        ("record geometry: correction [R, HV, Q, V], key [R, H, Q, K], decay [R, HV, Q] with R = config "
         "record rows",
         lambda: correction.dim() == 4 and key.dim() == 4 and decay.dim() == 3
         and tuple(correction.shape) == (n["record_rows"], n["value_heads"], n["Q"], v.size(3))
         and tuple(key.shape) == (n["record_rows"], n["heads"], n["Q"], q.size(3))
         and tuple(decay.shape) == (n["record_rows"], n["value_heads"], n["Q"])),
        ("record elements must be contiguous",
         lambda: correction.stride(3) == 1 and key.stride(3) == 1 and decay.stride(2) == 1),
        ("gate geometry: g and beta [T, HV] with contiguous heads",
         lambda: g.dim() == 2 and beta.dim() == 2 and tuple(g.shape) == (n["tokens"], n["value_heads"])
         and tuple(beta.shape) == (n["tokens"], n["value_heads"]) and g.stride(1) == 1 and beta.stride(1) == 1),
        ("activation elements: q, k, v and out heads must be contiguous",
         lambda: q.stride(3) == 1 and q.stride(2) == q.size(3) and k.stride(3) == 1 and k.stride(2) == k.size(3)
         and v.stride(3) == 1 and v.stride(2) == v.size(3) and out.stride(3) == 1 and out.stride(2) == out.size(3)),
        ("config strides do not match the tensors' strides",
         lambda: tuple(c[8:28]) == (q.stride(1), k.stride(1), v.stride(1), g.stride(0), beta.stride(0),
                                    *state.stride()[:3], *correction.stride()[:3], *key.stride()[:3],
                                    *decay.stride()[:3], out.stride(1), qsl.stride(0), indices.stride(0))),
    ))


def validate_fold(state, correction, key, decay, state_addrs, state_block_strides, corr_addrs, corr_block_strides,
                  key_addrs, key_block_strides, decay_addrs, decay_block_strides, layer_groups, source, lengths,
                  final_indices, boundary_indices, boundary_lengths, config) -> None:
    """The fold operator's checks (csrc/ops.cpp:171-228), in its order. An
    empty ``layer_groups`` maps every layer to the plan's first group, and
    ``source`` may be a strided int32/int64 view (the single-context commit
    folds from the state indices of its one group)."""
    c = list(config)
    n = dict(zip(("rows", "layers", "heads", "key_heads", "Q", "blocks", "record_rows", "cap", "null_block"), c[:9]))
    tables = (state_addrs, state_block_strides, corr_addrs, corr_block_strides, key_addrs, key_block_strides,
              decay_addrs, decay_block_strides)
    plan = (lengths, final_indices, boundary_indices, boundary_lengths)
    everything = (correction, key, decay, *tables, layer_groups, source, *plan)
    P = lengths.numel()
    _checks("fold", (
        ("config must have 17 fields", lambda: len(c) == 17),
        ("physical page zero is the null page (config null_block must be 0)", lambda: c[8] == 0),
        ("all tensors must be on the same device", lambda: all(t.device == state.device for t in everything)),
        ("dtype: checkpoint and key records FP32/BF16/FP16, correction and decay FP32",
         lambda: state.dtype in _FLOAT and key.dtype in _FLOAT and correction.dtype == torch.float32
         and decay.dtype == torch.float32),
        ("layer table: address and stride tables must be contiguous int64 [layers]",
         lambda: n["layers"] > 0 and all(t.dtype == torch.int64 and t.dim() == 1 and t.is_contiguous()
                                         and t.numel() == n["layers"] for t in tables)),
        ("layer group table: contiguous int32 [layers] (or empty: every layer in group 0)",
         lambda: layer_groups.dtype == torch.int32 and layer_groups.dim() == 1 and layer_groups.is_contiguous()
         and layer_groups.numel() in (0, n["layers"])),
        ("plan tensors: lengths, final, boundary and boundary lengths contiguous int32 of one length, a "
         "multiple of the plan capacity",
         lambda: all(t.dtype == torch.int32 and t.dim() == 1 and t.is_contiguous() and t.numel() == P for t in plan)
         and n["cap"] > 0 and P >= n["cap"] and P % n["cap"] == 0),
        ("plan source: int32 or int64 [groups * capacity] (one group: at least rows entries)",
         lambda: source.dtype in _INDEX and source.dim() == 1
         and source.numel() >= (P // n["cap"] - 1) * n["cap"] + n["rows"]),
        ("fold geometry: config rows/heads/window disagree",
         lambda: 0 < n["rows"] <= min(n["record_rows"], n["cap"]) and n["heads"] > 0 and n["key_heads"] > 0
         and n["heads"] % n["key_heads"] == 0 and 0 < n["Q"] <= 8),
        ("fold state geometry: checkpoint must be [blocks, HV, V, K] with K contiguous",
         lambda: state.dim() == 4 and state.size(1) == n["heads"] and state.stride(3) == 1
         and state.stride(2) >= state.size(3)),
        ("fold record geometry: correction [>= R, HV, Q, V], key [>= R, H, Q, K], decay [>= R, HV, Q] with "
         "contiguous elements",
         lambda: correction.dim() == 4 and key.dim() == 4 and decay.dim() == 3
         and correction.size(0) >= n["record_rows"] and key.size(0) >= n["record_rows"]
         and decay.size(0) >= n["record_rows"]
         and tuple(correction.shape[1:]) == (n["heads"], n["Q"], state.size(2))
         and tuple(key.shape[1:]) == (n["key_heads"], n["Q"], state.size(3))
         and tuple(decay.shape[1:]) == (n["heads"], n["Q"])
         and correction.stride(3) == 1 and key.stride(3) == 1 and decay.stride(2) == 1),
        ("fold config strides do not match the tensors' strides",
         lambda: tuple(c[9:17]) == (state.stride(1), state.stride(2), correction.stride(1), correction.stride(2),
                                    key.stride(1), key.stride(2), decay.stride(1), decay.stride(2))),
    ))


def _verify(q, k, v, g, beta, state, correction, key, decay, out, qsl, indices, config, scale):
    """csrc/ops.cpp:87-154: pre-normalised q/k, typed-SoA records."""
    validate_verify(q, k, v, g, beta, state, correction, key, decay, out, qsl, indices, config)
    lib = N.load()
    ext = N.VerifyExt(
        key_dim=q.shape[-1], value_dim=v.shape[-1], act_dtype=N.dtype_code(q.dtype),
        beta_dtype=N.dtype_code(beta.dtype), g_dtype=N.dtype_code(g.dtype), state_dtype=N.dtype_code(state.dtype),
        key_record_dtype=N.dtype_code(key.dtype), qsl_dtype=N.dtype_code(qsl.dtype),
        index_dtype=N.dtype_code(indices.dtype), qk_l2norm=0, key_per_value_head=0, out_dtype=N.dtype_code(out.dtype),
    )
    cfg = N.i64_array(config)
    status = lib.gdn_recoverssm_verify(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), state.data_ptr(),
        correction.data_ptr(), key.data_ptr(), decay.data_ptr(), out.data_ptr(), qsl.data_ptr(), indices.data_ptr(),
        cfg, len(config), float(scale), ctypes.byref(ext), N.stream_handle(q.device),
    )
    N.check(status, "verify")


def _fold(state, correction, key, decay, state_addrs, state_block_strides, corr_addrs, corr_block_strides, key_addrs,
          key_block_strides, decay_addrs, decay_block_strides, layer_groups, source, lengths, final_indices,
          boundary_indices, boundary_lengths, config):
    """csrc/ops.cpp:170-239: state, correction, key and decay are layer 0's
    tensors (element types and head dims); the pages of every layer are reached
    through the address and stride tables."""
    validate_fold(state, correction, key, decay, state_addrs, state_block_strides, corr_addrs, corr_block_strides,
                  key_addrs, key_block_strides, decay_addrs, decay_block_strides, layer_groups, source, lengths,
                  final_indices, boundary_indices, boundary_lengths, config)
    lib = N.load()
    ext = N.FoldExt(
        key_dim=key.shape[-1], value_dim=correction.shape[-1], state_dtype=N.dtype_code(state.dtype),
        key_dtype=N.dtype_code(key.dtype), source_dtype=N.dtype_code(source.dtype), source_stride=source.stride(0),
        state_k_stride=state.stride(-1),
    )
    cfg = N.i64_array(config)
    status = lib.gdn_recoverssm_fold(
        state.data_ptr(), correction.data_ptr(), key.data_ptr(), decay.data_ptr(), state_addrs.data_ptr(),
        state_block_strides.data_ptr(), corr_addrs.data_ptr(), corr_block_strides.data_ptr(), key_addrs.data_ptr(),
        key_block_strides.data_ptr(), decay_addrs.data_ptr(), decay_block_strides.data_ptr(),
        layer_groups.data_ptr() if layer_groups.numel() else None, source.data_ptr(), lengths.data_ptr(),
        final_indices.data_ptr(), boundary_indices.data_ptr(), boundary_lengths.data_ptr(), cfg, len(config),
        ctypes.byref(ext), N.stream_handle(state.device),
    )
    N.check(status, "fold")


def _meta_noop(*args):
    return None


_LIBRARY = None


def register() -> None:
    """Define and implement the operators (idempotent)."""
    global _LIBRARY
    if _LIBRARY is not None:
        return
    library = torch.library.Library(NAMESPACE, "DEF")
    library.define(ABI_SCHEMA)
    library.define(VERIFY_SCHEMA)
    library.define(FOLD_SCHEMA)
    library.impl("abi_version", _abi_version, "CompositeExplicitAutograd")
    library.impl("verify", _verify, "CUDA")
    library.impl("fold", _fold, "CUDA")
    library.impl("verify", _meta_noop, "Meta")
    library.impl("fold", _meta_noop, "Meta")
    _LIBRARY = library


register()

__all__ = ["NAMESPACE", "ABI_SCHEMA", "VERIFY_SCHEMA", "FOLD_SCHEMA", "register", "validate_fold", "validate_verify"]

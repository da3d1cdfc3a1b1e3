"""The reference's native operator ABI as torch operators.

The reference registers ``gdn_recoverssm_ac::abi_version``, ``verify`` and
``fold`` (csrc/ops.cpp:243-257) and its backend hook calls them through
``torch.ops.gdn_recoverssm_ac`` with the 28-field verify and 17-field fold
configs (ascendc_backend.py:98-212). This module registers the same three
operators, with the same schemas and mutation annotations, under
``torch.ops.gdn_recoverssm_hip``: a backend written against the reference's
namespace switches by name. Each operator validates nothing itself and calls
the C ABI of ``libgdn_recoverssm_hip.so`` on the tensors' current stream; the
element types and head dims the C ABI takes beside the config come from the
tensors. A rejected configuration raises ``ValueError`` and a failed launch
``RuntimeError``, before or instead of any device work. The Meta kernels do
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


def _verify(q, k, v, g, beta, state, correction, key, decay, out, qsl, indices, config, scale):
    """csrc/ops.cpp:87-154: pre-normalised q/k, typed-SoA records."""
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
    through the address and stride tables. An empty ``layer_groups`` maps every
    layer to the plan's first group."""
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

__all__ = ["NAMESPACE", "ABI_SCHEMA", "VERIFY_SCHEMA", "FOLD_SCHEMA", "register"]

"""ctypes binding of the C ABI in ``include/gdn_recoverssm_hip.h``.

The shared library is built ahead of time into ``_lib/libgdn_recoverssm_hip.so``
(see ``_build.py``). There is no fallback: if the library is missing or its ABI
version differs, every launch raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

from ._build import CSRC_DIR, LIB_PATH, built_digest, source_digest

ABI_VERSION = 1
VERIFY_CONFIG_FIELDS = 28
FOLD_CONFIG_FIELDS = 17
PLAN_MAX_GROUPS = 8

GDN_OK, GDN_ERR_INVALID, GDN_ERR_UNSUPPORTED, GDN_ERR_LAUNCH = 0, 1, 2, 3
DT_F32, DT_BF16, DT_F16, DT_I32, DT_I64 = 0, 1, 2, 3, 4
PLAN_ALIGN, PLAN_PUBLISH, PLAN_GROUPED = 1, 2, 4

_DTYPE_CODES = {
    torch.float32: DT_F32,
    torch.bfloat16: DT_BF16,
    torch.float16: DT_F16,
    torch.int32: DT_I32,
    torch.int64: DT_I64,
}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"GDN RecoverSSM: dtype {dtype} has no HIP kernel") from None


c_i64 = ctypes.c_int64
c_i32 = ctypes.c_int32
c_vp = ctypes.c_void_p
P_i64 = ctypes.POINTER(ctypes.c_int64)


class VerifyExt(ctypes.Structure):
    _fields_ = [
        ("key_dim", c_i64),
        ("value_dim", c_i64),
        ("act_dtype", c_i32),
        ("beta_dtype", c_i32),
        ("g_dtype", c_i32),
        ("state_dtype", c_i32),
        ("key_record_dtype", c_i32),
        ("qsl_dtype", c_i32),
        ("index_dtype", c_i32),
        ("qk_l2norm", c_i32),
        ("key_per_value_head", c_i32),
        ("out_dtype", c_i32),
        ("state_cache_retain", c_i64),
    ]


class FoldExt(ctypes.Structure):
    _fields_ = [
        ("key_dim", c_i64),
        ("value_dim", c_i64),
        ("state_dtype", c_i32),
        ("key_dtype", c_i32),
        ("source_dtype", c_i32),
        ("reserved", c_i32),
        ("source_stride", c_i64),
        ("state_k_stride", c_i64),
        ("row_list", ctypes.c_void_p),
        ("row_list_len", c_i64),
        ("row_count", ctypes.c_void_p),
    ]


class SettleNext(ctypes.Structure):
    """gdn_settle_next: one plan group's next batch for gdn_recoverssm_settle."""
    _fields_ = [
        ("state_indices", ctypes.c_void_p),
        ("stride", c_i64),
        ("rows", c_i64),
        ("dtype", c_i32),
        ("reserved", c_i32),
    ]


SETTLE_MAX_GROUPS = 3
SETTLE_MAX_ROWS = 65536


class GatingExt(ctypes.Structure):
    _fields_ = [
        ("a_log_dtype", c_i32),
        ("dt_bias_dtype", c_i32),
        ("softplus_beta", ctypes.c_float),
        ("softplus_threshold", ctypes.c_float),
    ]


class PendingCommit(ctypes.Structure):
    _fields_ = [
        ("rows", c_vp), ("source", c_vp), ("lengths", c_vp), ("final_indices", c_vp),
        ("boundary_indices", c_vp), ("boundary_lengths", c_vp),
        ("correction", c_vp), ("key", c_vp), ("decay", c_vp),
        ("record_rows", c_i64),
        ("corr_strides", c_i64 * 3), ("key_strides", c_i64 * 3), ("decay_strides", c_i64 * 3),
        ("key_dtype", c_i32), ("key_per_value_head", c_i32),
        ("num_rows", c_i64),
    ]


class PlanGroup(ctypes.Structure):
    _fields_ = [
        ("state_indices", c_vp), ("si_stride", c_i64), ("si_dtype", c_i32), ("pad0", c_i32),
        ("query_start_loc", c_vp), ("qsl_stride", c_i64), ("qsl_dtype", c_i32), ("pad1", c_i32),
        ("request_indices", c_vp), ("map_stride", c_i64), ("map_dtype", c_i32), ("pad2", c_i32),
        ("block_table", c_vp), ("table_row_stride", c_i64), ("table_col_stride", c_i64), ("table_width", c_i64),
        ("table_rows", c_i64), ("table_dtype", c_i32), ("pad3", c_i32),
        ("num_computed", c_vp), ("computed_stride", c_i64), ("computed_len", c_i64), ("computed_dtype", c_i32),
        ("pad4", c_i32),
        ("num_blocks", c_i64), ("block_size", c_i64),
    ]


PlanGroups = PlanGroup * PLAN_MAX_GROUPS


class PlanLaunch(ctypes.Structure):  # gdn_plan_launch: gdn_recoverssm_plan's arguments as one block
    _fields_ = [
        ("sampled", c_vp), ("sampled_stride", c_i64), ("sampled_len", c_i64), ("sampled_dtype", c_i32),
        ("num_groups", c_i32), ("groups", ctypes.POINTER(PlanGroup)),
        ("source_plan", c_vp), ("lens_plan", c_vp), ("final_plan", c_vp), ("boundary_plan", c_vp),
        ("boundary_lens_plan", c_vp), ("valid_plan", c_vp), ("col_plan", c_vp),
        ("idx_mapping", c_vp), ("idx_mapping_len", c_i64), ("idx_mapping_dtype", c_i32), ("flags", ctypes.c_uint32),
        ("persistent_cols", c_vp), ("persistent_accepted", c_vp), ("persistent_len", c_i64),
        ("num_rows", c_i64), ("plan_capacity", c_i64), ("null_block", c_i64), ("spec_query_len", c_i64),
    ]


class ConvLaunch(ctypes.Structure):  # gdn_conv_launch: the conv tables of gdn_recoverssm_commit_noalloc
    _fields_ = [
        ("conv_addrs", c_vp), ("conv_block_strides", c_vp), ("conv_dim_strides", c_vp), ("conv_token_strides", c_vp),
        ("conv_dim", c_i64), ("history", c_i64), ("window", c_i64), ("element_bytes", c_i32), ("reserved", c_i32),
    ]


NOALLOC_PLAN_ENTRIES = 32768  # GDN_NOALLOC_PLAN_ENTRIES


def plan_launch(plan_args: tuple) -> PlanLaunch:
    """The gdn_recoverssm_plan argument tuple (without the stream) as a PlanLaunch."""
    (sampled, sampled_dtype, sampled_stride, sampled_len, groups, num_groups, source, lens, final, boundary,
     boundary_lens, valid, col, idx_mapping, idx_dtype, idx_len, pcols, pacc, plen, rows, cap, null_block, window,
     flags) = plan_args
    return PlanLaunch(
        sampled=sampled, sampled_stride=sampled_stride, sampled_len=sampled_len, sampled_dtype=sampled_dtype,
        num_groups=num_groups, groups=ctypes.cast(groups, ctypes.POINTER(PlanGroup)),
        source_plan=source, lens_plan=lens, final_plan=final, boundary_plan=boundary,
        boundary_lens_plan=boundary_lens, valid_plan=valid, col_plan=col, idx_mapping=idx_mapping,
        idx_mapping_len=idx_len, idx_mapping_dtype=idx_dtype, flags=flags, persistent_cols=pcols,
        persistent_accepted=pacc, persistent_len=plen, num_rows=rows, plan_capacity=cap, null_block=null_block,
        spec_query_len=window,
    )

_LIB = None
_LOCK = threading.Lock()


def library_path() -> str:
    return os.environ.get("GDN_RECOVERSSM_HIP_LIB", LIB_PATH)


def load() -> ctypes.CDLL:
    """Load the HIP library once (raises RuntimeError when it is missing)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        path = library_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"GDN RecoverSSM HIP library not found at {path}; build it with "
                "`python -m gdn_recoverssm_ascend._build` (there is no fallback path)"
            )
        _refuse_stale(path)
        lib = ctypes.CDLL(path)
        lib.gdn_recoverssm_abi_version.restype = ctypes.c_int
        lib.gdn_recoverssm_abi_version.argtypes = []
        lib.gdn_recoverssm_last_error.restype = ctypes.c_char_p
        lib.gdn_recoverssm_last_error.argtypes = []
        lib.gdn_recoverssm_verify.restype = ctypes.c_int
        lib.gdn_recoverssm_verify.argtypes = [c_vp] * 12 + [P_i64, c_i64, ctypes.c_float, ctypes.POINTER(VerifyExt), c_vp]
        lib.gdn_recoverssm_verify_gated.restype = ctypes.c_int
        lib.gdn_recoverssm_verify_gated.argtypes = [c_vp] * 14 + [
            P_i64, c_i64, ctypes.c_float, ctypes.POINTER(VerifyExt), ctypes.POINTER(GatingExt), c_vp,
        ]
        lib.gdn_recoverssm_verify_deferred.restype = ctypes.c_int
        lib.gdn_recoverssm_verify_deferred.argtypes = [c_vp] * 12 + [
            P_i64, c_i64, ctypes.c_float, ctypes.POINTER(VerifyExt), ctypes.POINTER(PendingCommit), c_vp,
        ]
        lib.gdn_recoverssm_fold.restype = ctypes.c_int
        lib.gdn_recoverssm_fold.argtypes = [c_vp] * 18 + [P_i64, c_i64, ctypes.POINTER(FoldExt), c_vp]
        lib.gdn_recoverssm_plan_fold.restype = ctypes.c_int
        lib.gdn_recoverssm_plan_fold.argtypes = [ctypes.POINTER(PlanLaunch)] + [c_vp] * 13 + [
            P_i64, c_i64, ctypes.POINTER(FoldExt), c_vp,
        ]
        lib.gdn_recoverssm_commit_noalloc.restype = ctypes.c_int
        lib.gdn_recoverssm_commit_noalloc.argtypes = [ctypes.POINTER(PlanLaunch)] + [c_vp] * 13 + [
            P_i64, c_i64, ctypes.POINTER(FoldExt), ctypes.POINTER(ConvLaunch), c_vp,
        ]
        lib.gdn_recoverssm_plan.restype = ctypes.c_int
        lib.gdn_recoverssm_plan.argtypes = [
            c_vp, c_i32, c_i64, c_i64,  # sampled
            ctypes.POINTER(PlanGroup), c_i32,  # groups
            c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,  # plan outputs
            c_vp, c_i32, c_i64,  # idx_mapping
            c_vp, c_vp, c_i64,  # persistent outputs
            c_i64, c_i64, c_i64, c_i64, ctypes.c_uint32, c_vp,
        ]
        lib.gdn_recoverssm_conv_compact.restype = ctypes.c_int
        lib.gdn_recoverssm_conv_compact.argtypes = [
            c_vp, c_vp, c_vp, c_vp,  # tables
            c_vp, c_i32, c_i64,  # source
            c_vp, c_vp, c_vp, c_vp, c_vp,  # lengths, final, boundary, boundary_len, layer_groups
            c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i32, c_i32, c_vp,
        ]
        lib.gdn_recoverssm_publish.restype = ctypes.c_int
        lib.gdn_recoverssm_publish.argtypes = [
            c_vp, c_i64, c_vp, c_i32, c_i64, c_i64, c_vp, c_i32, c_i64, c_vp, c_vp, c_i64, c_i64, c_vp,
        ]
        lib.gdn_recoverssm_set_state_cache_retain.restype = c_i64
        lib.gdn_recoverssm_set_state_cache_retain.argtypes = [c_i64]
        lib.gdn_recoverssm_settle.restype = ctypes.c_int
        lib.gdn_recoverssm_settle.argtypes = [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_i64,
                                              ctypes.POINTER(SettleNext), c_vp, c_vp, c_vp, c_vp]
        version = lib.gdn_recoverssm_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"GDN RecoverSSM HIP library ABI mismatch: {version} != {ABI_VERSION}")
        _LIB = lib
    return _LIB


def _refuse_stale(path: str) -> None:
    """Refuse a library built from other kernel sources than the ones beside
    the package. The in-tree library must carry the digest build() records;
    a library named by GDN_RECOVERSSM_HIP_LIB is checked when it carries one."""
    recorded = built_digest(path)
    if recorded is None and os.path.abspath(path) != os.path.abspath(LIB_PATH):
        return
    if not os.path.isdir(CSRC_DIR):
        return  # an installed library without its sources: nothing to compare against
    current = source_digest()
    if recorded != current:
        raise RuntimeError(
            f"GDN RecoverSSM HIP library at {path} was built from other kernel sources "
            f"(recorded digest {recorded or 'missing'}, sources {current}); rebuild it with "
            "`python -m gdn_recoverssm_ascend._build` (there is no fallback path)"
        )


def exported_symbols() -> tuple[str, ...]:
    return (
        "gdn_recoverssm_abi_version",
        "gdn_recoverssm_last_error",
        "gdn_recoverssm_verify",
        "gdn_recoverssm_verify_gated",
        "gdn_recoverssm_verify_deferred",
        "gdn_recoverssm_fold",
        "gdn_recoverssm_plan_fold",
        "gdn_recoverssm_commit_noalloc",
        "gdn_recoverssm_plan",
        "gdn_recoverssm_conv_compact",
        "gdn_recoverssm_publish",
        "gdn_recoverssm_set_state_cache_retain",
        "gdn_recoverssm_settle",
    )


def check(status: int, what: str) -> None:
    if status == GDN_OK:
        return
    msg = load().gdn_recoverssm_last_error().decode(errors="replace")
    if status in (GDN_ERR_INVALID, GDN_ERR_UNSUPPORTED):
        raise ValueError(f"GDN RecoverSSM: {what} rejected by the HIP library: {msg}")
    raise RuntimeError(f"GDN RecoverSSM: {what} failed: {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def i64_array(values) -> ctypes.Array:
    return (c_i64 * len(values))(*[int(v) for v in values])

"""The reference's native operator ABI as torch operators, on the CPU:
``torch.ops.gdn_recoverssm_hip.{abi_version, verify, fold}`` exist with the
reference's schemas (csrc/ops.cpp:244-246 of the reference plugin, mutation
annotations included), the Meta kernels accept the shapes without work, and
there is no CPU kernel to fall back to."""

import pytest
import torch

from gdn_recoverssm_ascend import torch_ops as T

OPS = torch.ops.gdn_recoverssm_hip

REFERENCE_VERIFY = (
    "verify(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, Tensor state, Tensor(a!) correction, "
    "Tensor(b!) key, Tensor(c!) decay, Tensor(d!) out, Tensor qsl, Tensor indices, int[] config, float scale) -> ()"
)
REFERENCE_FOLD = (
    "fold(Tensor(a!) state, Tensor correction, Tensor key, Tensor decay, Tensor state_addrs, "
    "Tensor state_block_strides, Tensor corr_addrs, Tensor corr_block_strides, Tensor key_addrs, "
    "Tensor key_block_strides, Tensor decay_addrs, Tensor decay_block_strides, Tensor layer_groups, "
    "Tensor source, Tensor lengths, Tensor final_indices, Tensor boundary_indices, Tensor boundary_lengths, "
    "int[] config) -> ()"
)


def test_abi_version_is_one():
    assert OPS.abi_version() == 1


def test_schemas_match_the_reference():
    assert str(OPS.verify.default._schema) == f"{T.NAMESPACE}::{REFERENCE_VERIFY}"
    assert str(OPS.fold.default._schema) == f"{T.NAMESPACE}::{REFERENCE_FOLD}"
    written = [a.name for a in OPS.verify.default._schema.arguments if a.alias_info and a.alias_info.is_write]
    assert written == ["correction", "key", "decay", "out"]  # the checkpoint is read-only
    written = [a.name for a in OPS.fold.default._schema.arguments if a.alias_info and a.alias_info.is_write]
    assert written == ["state"]


def _meta(*shape, dtype=torch.float32):
    return torch.empty(*shape, device="meta", dtype=dtype)


def test_meta_kernels_do_no_work():
    i32 = torch.int32
    OPS.verify(_meta(1, 8, 1, 128), _meta(1, 8, 1, 128), _meta(1, 8, 3, 128), _meta(8, 3), _meta(8, 3),
               _meta(4, 3, 128, 128), _meta(2, 3, 4, 128), _meta(2, 1, 4, 128), _meta(2, 3, 4), _meta(1, 8, 3, 128),
               _meta(3, dtype=i32), _meta(2, dtype=i32), [0] * 28, 1.0)
    tables = [_meta(2, dtype=torch.int64) for _ in range(8)]
    OPS.fold(_meta(4, 3, 128, 128), _meta(2, 3, 4, 128), _meta(2, 1, 4, 128), _meta(2, 3, 4), *tables,
             _meta(2, dtype=i32), _meta(2, dtype=i32), _meta(2, dtype=i32), _meta(2, dtype=i32), _meta(2, dtype=i32),
             _meta(2, dtype=i32), [0] * 17)


def test_no_cpu_kernel():
    q = torch.zeros(1, 8, 1, 128)
    with pytest.raises(NotImplementedError):
        OPS.verify(q, q, torch.zeros(1, 8, 3, 128), torch.zeros(8, 3), torch.zeros(8, 3),
                   torch.zeros(4, 3, 128, 128), torch.zeros(2, 3, 4, 128), torch.zeros(2, 1, 4, 128),
                   torch.zeros(2, 3, 4), torch.zeros(1, 8, 3, 128), torch.zeros(3, dtype=torch.int32),
                   torch.zeros(2, dtype=torch.int32), [0] * 28, 1.0)


# ---------------------------------------------------------------------------
# Config-vs-tensor checks (csrc/ops.cpp:91-141 and :171-228 of the reference):
# one case per check class, each on an otherwise valid CPU argument set.
# ---------------------------------------------------------------------------

def _verify_args(**over):
    B, T, H, HV, K, V, Q, NB, R = 2, 4, 1, 2, 8, 8, 2, 5, 3
    a = dict(q=torch.zeros(1, T, H, K, dtype=torch.bfloat16), k=torch.zeros(1, T, H, K, dtype=torch.bfloat16),
             v=torch.zeros(1, T, HV, V, dtype=torch.bfloat16), g=torch.zeros(T, HV), beta=torch.zeros(T, HV),
             state=torch.zeros(NB, HV, V, K), correction=torch.zeros(R, HV, Q, V),
             key=torch.zeros(R, H, Q, K, dtype=torch.bfloat16), decay=torch.zeros(R, HV, Q),
             out=torch.zeros(1, T, HV, V, dtype=torch.bfloat16), qsl=torch.zeros(B + 1, dtype=torch.int32),
             indices=torch.zeros(B, dtype=torch.int32))
    a.update(over)
    x = a
    cfg = [B, T, H, HV, Q, NB, R, 0, x["q"].stride(1), x["k"].stride(1), x["v"].stride(1), x["g"].stride(0),
           x["beta"].stride(0), *x["state"].stride()[:3], *x["correction"].stride()[:3], *x["key"].stride()[:3],
           *x["decay"].stride()[:3], x["out"].stride(1), x["qsl"].stride(0), x["indices"].stride(0)]
    return a, cfg


def _call_verify(a, cfg):
    T.validate_verify(a["q"], a["k"], a["v"], a["g"], a["beta"], a["state"], a["correction"], a["key"], a["decay"],
                      a["out"], a["qsl"], a["indices"], cfg)


def test_verify_checks_accept_a_valid_set():
    _call_verify(*_verify_args())
    # int64 metadata, a column view of a state table, FP32 beta / key records / output
    table = torch.zeros(2, 4, dtype=torch.int64)
    _call_verify(*_verify_args(indices=table[:, 0], qsl=torch.zeros(3, dtype=torch.int64),
                               key=torch.zeros(3, 1, 2, 8), out=torch.zeros(1, 4, 2, 8)))


@pytest.mark.parametrize("case,match", [
    ("config_len", "28 fields"),
    ("null_block", "null page"),
    ("device", "same device"),
    ("act_dtype", "activation dtype"),
    ("out_dtype", "FP32 or the activation dtype"),
    ("record_dtype", "correction and decay FP32"),
    ("index_dtype", "int32 or int64"),
    ("act_shape", "activation shape"),
    ("geometry", "verify geometry"),
    ("state", "state geometry"),
    ("capacity", "row capacity"),
    ("records", "record geometry"),
    ("record_elements", "record elements"),
    ("gates", "gate geometry"),
    ("act_elements", "activation elements"),
    ("strides", "config strides"),
])
def test_verify_checks_reject(case, match):
    a, cfg = _verify_args()
    if case == "config_len":
        cfg = cfg[:27]
    elif case == "null_block":
        cfg[7] = 1
    elif case == "device":
        a["decay"] = torch.zeros(3, 2, 2, device="meta")
    elif case == "act_dtype":
        a["k"] = a["k"].float()
    elif case == "out_dtype":
        a["out"] = a["out"].half()
    elif case == "record_dtype":
        a["correction"] = a["correction"].bfloat16()
    elif case == "index_dtype":
        a["qsl"] = a["qsl"].short()
    elif case == "act_shape":
        a["out"] = torch.zeros(1, 4, 2, 4, dtype=torch.bfloat16)
    elif case == "geometry":
        cfg[1] = 5  # tokens
    elif case == "state":
        cfg[5] = 6  # blocks
    elif case == "capacity":
        cfg[0], cfg[1] = 3, 4  # rows beyond query_start_loc / indices
    elif case == "records":
        cfg[6] = 2  # record rows
    elif case == "record_elements":
        a, cfg = _verify_args(correction=torch.zeros(3, 2, 8, 2).transpose(2, 3))
    elif case == "gates":
        a, cfg = _verify_args(g=torch.zeros(2, 4).t())
    elif case == "act_elements":
        a, cfg = _verify_args(v=torch.zeros(1, 4, 8, 2, dtype=torch.bfloat16).transpose(2, 3))
    elif case == "strides":
        cfg[13] += 8  # state block stride
    with pytest.raises(ValueError, match=match):
        _call_verify(a, cfg)


def _fold_args(**over):
    L, B, HV, H, K, V, Q, NB, R, cap = 2, 3, 2, 1, 8, 8, 2, 5, 4, 4
    a = dict(state=torch.zeros(NB, HV, V, K), correction=torch.zeros(R, HV, Q, V),
             key=torch.zeros(R, H, Q, K, dtype=torch.bfloat16), decay=torch.zeros(R, HV, Q),
             tables=[torch.zeros(L, dtype=torch.int64) for _ in range(8)],
             layer_groups=torch.zeros(L, dtype=torch.int32), source=torch.zeros(cap, dtype=torch.int32),
             plan=[torch.zeros(cap, dtype=torch.int32) for _ in range(4)])
    a.update(over)
    x = a
    cfg = [B, L, HV, H, Q, NB, R, cap, 0, x["state"].stride(1), x["state"].stride(2), x["correction"].stride(1),
           x["correction"].stride(2), x["key"].stride(1), x["key"].stride(2), x["decay"].stride(1),
           x["decay"].stride(2)]
    return a, cfg


def _call_fold(a, cfg):
    T.validate_fold(a["state"], a["correction"], a["key"], a["decay"], *a["tables"], a["layer_groups"], a["source"],
                    *a["plan"], cfg)


def test_fold_checks_accept_a_valid_set():
    _call_fold(*_fold_args())
    # every layer in group 0, the state indices of the one group as a strided int64 source
    table = torch.zeros(3, 4, dtype=torch.int64)
    _call_fold(*_fold_args(layer_groups=torch.zeros(0, dtype=torch.int32), source=table[:, 0]))


@pytest.mark.parametrize("case,match", [
    ("config_len", "17 fields"),
    ("null_block", "null page"),
    ("device", "same device"),
    ("dtype", "correction and decay FP32"),
    ("tables", "layer table"),
    ("groups", "layer group table"),
    ("plan", "plan tensors"),
    ("source", "plan source"),
    ("geometry", "fold geometry"),
    ("state", "fold state geometry"),
    ("records", "fold record geometry"),
    ("strides", "fold config strides"),
])
def test_fold_checks_reject(case, match):
    a, cfg = _fold_args()
    if case == "config_len":
        cfg = cfg + [0]
    elif case == "null_block":
        cfg[8] = 3
    elif case == "device":
        a["plan"][2] = torch.zeros(4, dtype=torch.int32, device="meta")
    elif case == "dtype":
        a["decay"] = a["decay"].half()
    elif case == "tables":
        a["tables"][5] = torch.zeros(3, dtype=torch.int64)  # not one entry per layer
    elif case == "groups":
        a["layer_groups"] = torch.zeros(2, dtype=torch.int64)
    elif case == "plan":
        a["plan"][1] = torch.zeros(6, dtype=torch.int32)
    elif case == "source":
        a["source"] = torch.zeros(2, dtype=torch.int32)  # fewer entries than rows
    elif case == "geometry":
        cfg[4] = 9  # a window beyond 8 tokens
    elif case == "state":
        cfg[2] = 3  # value heads
    elif case == "records":
        cfg[6] = 5  # record rows beyond the records
    elif case == "strides":
        cfg[12] += 1  # correction token stride
    with pytest.raises(ValueError, match=match):
        _call_fold(a, cfg)

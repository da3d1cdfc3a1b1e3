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

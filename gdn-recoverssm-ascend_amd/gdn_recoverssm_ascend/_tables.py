"""Per-layer device tables through which the commit kernels reach the pages.

The fold, the fused plan + fold and the conv compaction address every layer's
checkpoint pages, conv-state pages and record planes through int64 device
tables: one base address and one row (block) stride per layer, plus the conv
states' channel and token strides. ``LayerPages`` builds all of them once per
cache epoch for an ordered list of layers: the layers of one commit context, or
the layers of every context in a grouped bucket, in bucket order. It also
checks that the layers agree on everything the kernels take from the first
layer (shapes, dtypes, inner strides).
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch

from ._rules import enforce

_F32 = 4


def pointer_table(tensors: Sequence[torch.Tensor], device, byte_offset: int = 0) -> torch.Tensor:
    """int64 device table of the tensors' data pointers (plus a byte offset);
    an address with the top bit set keeps its bit pattern."""
    values = []
    for t in tensors:
        p = t.data_ptr() + byte_offset
        values.append(p - (1 << 64) if p >= (1 << 63) else p)
    return torch.tensor(values, dtype=torch.int64, device=device)


def stride_table(tensors: Sequence[torch.Tensor], dim: int, device) -> torch.Tensor:
    """int64 device table of each tensor's element stride along ``dim``."""
    strides = torch.as_tensor([t.stride()[dim] for t in tensors], dtype=torch.int64)
    return strides.to(device)


@dataclass(frozen=True)
class RecordPlanes:
    """One layer's records as three planes: correction [rows, HV, Q, V],
    key [rows, H(or HV), Q, K] and decay [rows, HV, Q]. Typed records are three
    tensors; a packed FP32 record [rows, HV, Q, V + K + 1] is one tensor whose
    key plane starts V floats and whose decay plane starts V + K floats into
    each (row, head, token) record."""

    correction: torch.Tensor
    key: torch.Tensor
    decay: torch.Tensor
    key_offset: int = 0  # bytes
    decay_offset: int = 0  # bytes

    @property
    def packed(self) -> bool:
        return self.key is self.correction


def record_planes(record, value_dim: int, key_dim: int) -> RecordPlanes:
    if hasattr(record, "correction"):
        return RecordPlanes(record.correction, record.key, record.decay)
    return RecordPlanes(record, record, record, value_dim * _F32, (value_dim + key_dim) * _F32)


class LayerPages:
    """Checkpoint pages, conv states and record planes of an ordered list of
    layers, with the device tables the commit kernels read. ``device_tables``
    lists the eight fold tables in the kernels' argument order."""

    def __init__(self, conv_states: Sequence[torch.Tensor], checkpoints: Sequence[torch.Tensor],
                 records: Sequence, device):
        self.conv_states = tuple(conv_states)
        self.checkpoints = tuple(checkpoints)
        self.records = tuple(records)
        _, _, V, K = self.checkpoints[0].shape
        self.planes = tuple(record_planes(r, V, K) for r in self.records)
        first = self.planes[0]
        dev = device
        self.state_addrs = pointer_table(self.checkpoints, dev)
        self.state_block_strides = stride_table(self.checkpoints, 0, dev)
        self.conv_addrs = pointer_table(self.conv_states, dev)
        self.conv_block_strides = stride_table(self.conv_states, 0, dev)
        self.conv_dim_strides = stride_table(self.conv_states, 1, dev)
        self.conv_token_strides = stride_table(self.conv_states, 2, dev)
        corr = [p.correction for p in self.planes]
        keys = [p.key for p in self.planes]
        decays = [p.decay for p in self.planes]
        self.correction_addrs = pointer_table(corr, dev)
        self.correction_block_strides = stride_table(corr, 0, dev)
        self.key_addrs = pointer_table(keys, dev, first.key_offset)
        self.key_block_strides = stride_table(keys, 0, dev)
        self.decay_addrs = pointer_table(decays, dev, first.decay_offset)
        self.decay_block_strides = stride_table(decays, 0, dev)

    @property
    def device_tables(self) -> tuple:
        return (self.state_addrs, self.state_block_strides, self.correction_addrs, self.correction_block_strides,
                self.key_addrs, self.key_block_strides, self.decay_addrs, self.decay_block_strides)

    @property
    def first_planes(self) -> RecordPlanes:
        return self.planes[0]


def _same_tail(tensors: Sequence[torch.Tensor], dims: int = 1) -> bool:
    """Equal shapes, dtypes, devices and strides past the first `dims` dims."""
    a = tensors[0]
    return all(t.shape[dims:] == a.shape[dims:] and t.dtype == a.dtype and t.device == a.device
               and t.stride()[dims:] == a.stride()[dims:] for t in tensors)


def check_layers(conv_states, checkpoints, records, *, window: int, typed: bool, max_window: int) -> None:
    """The commit context's layer checks (messages of kernels.py:1438-1517)."""
    ck = list(checkpoints)
    enforce((
        ("commit requires at least one layer", lambda: len(ck) > 0),
        ("conv, state and replay lists differ", lambda: len(conv_states) == len(ck) == len(records)),
        (f"spec_query_len must be in [1, {max_window}]", lambda: 0 < window <= max_window),
        ("checkpoint must be four-dimensional", lambda: ck[0].ndim == 4),
        ("layers need matching checkpoints",
         lambda: all(c.shape == ck[0].shape for c in ck) and _same_tail(ck)),
    ))
    _, HV, V, K = ck[0].shape
    dev = ck[0].device
    if typed:
        planes = [record_planes(r, V, K) for r in records]
        H = planes[0].key.shape[1]
        corr = [p.correction for p in planes]
        keys = [p.key for p in planes]
        decays = [p.decay for p in planes]
        enforce((
            ("record key heads are incompatible", lambda: H > 0 and HV % H == 0),
            ("layers need matching typed replay geometry/dtypes/strides",
             lambda: all(c.shape == corr[0].shape for c in corr) and _same_tail(corr) and _same_tail(keys)
             and _same_tail(decays)
             and tuple(corr[0].shape[1:]) == (HV, window, V)
             and all(tuple(k.shape) == (c.shape[0], H, window, K) for k, c in zip(keys, corr))
             and all(tuple(d.shape) == (c.shape[0], HV, window) for d, c in zip(decays, corr))
             and corr[0].dtype == torch.float32 and decays[0].dtype == torch.float32
             and keys[0].dtype in (torch.float16, torch.bfloat16, torch.float32)
             and all(t.device == dev for t in corr + keys + decays)),
        ))
    else:
        enforce((
            ("layers need matching packed FP32 replay buffers",
             lambda: all(isinstance(r, torch.Tensor) for r in records)
             and records[0].ndim == 4 and tuple(records[0].shape[1:]) == (HV, window, V + K + 1)
             and all(r.shape == records[0].shape for r in records) and _same_tail(list(records))
             and records[0].dtype == torch.float32 and records[0].device == dev),
        ))
    conv0 = conv_states[0]
    enforce((
        ("conv state must be [blocks, dim, window] with the checkpoint's block count",
         lambda: conv0.ndim == 3 and conv0.shape[0] == ck[0].shape[0]),
        ("layers need matching conv states",
         lambda: all(c.shape == conv0.shape for c in conv_states) and _same_tail(list(conv_states))
         and conv0.device == dev),
        ("conv state is shorter than its window", lambda: conv0.shape[2] - window + 1 > 0),
    ))

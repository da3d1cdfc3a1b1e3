"""Step-owned grouped recovery: one plan + SSM fold launch and one conv pass per bucket.

Host side of the post-sampling commit, keeping the reference plugin's API
(``gdn_recoverssm_ascend/grouped_commit.py``): ``CommitEntry``,
``GroupedCommitBucket``, ``GroupedCommitCoordinator`` and
``prepare_grouped_commit``. A bucket launches the gfx950 HIP entry points
``gdn_recoverssm_plan_fold`` (the reference's plan and fold kernels as one
launch) and ``gdn_recoverssm_conv_compact``; ``make_specs(...,
fuse_plan_fold=False)`` gives the reference's three launches
(``gdn_recoverssm_plan``, conv, ``gdn_recoverssm_fold``) instead. A
multi-bucket align step adds ``gdn_recoverssm_publish``.

A bucket holds up to three homogeneous cache groups (the reference's bucket
width, grouped_commit.py:947-954), so bucket boundaries match the reference
coordinator exactly.
"""

from __future__ import annotations

import logging
from dataclasses import dataclass
from typing import Any

import torch

from . import _native as N
from .kernels import (
    NULL_BLOCK_ID,
    _fuse_plan_fold,
    _LaunchSpec,
    _make_fold_spec,
    _ptr_table,
    _record_planes,
    _require,
)

logger = logging.getLogger("gdn_recoverssm_ascend.grouped_commit")

# Cache groups per physical bucket (reference grouped_commit.py:947-954).
GROUPS_PER_BUCKET = 3


@dataclass(frozen=True)
class CommitEntry:
    metadata: Any
    payload: Any
    context: Any


def _layout_key(context):
    state = context.checkpoints[0]
    conv = context.conv_states[0]
    record = context.records[0]
    soa = context.record_layout == "soa"
    rr = record.correction if soa else record
    kr = record.key if soa else record
    dr = record.decay if soa else record
    return (
        state.device,
        state.dtype,
        tuple(state.shape[1:]),
        tuple(state.stride()[1:]),
        conv.dtype,
        tuple(conv.shape[1:]),
        tuple(conv.stride()[1:]),
        context.conv_history_len,
        context.spec_query_len,
        context.record_layout,
        context.num_key_heads,
        rr.dtype,
        tuple(rr.stride()[1:]),
        kr.dtype,
        tuple(kr.stride()[1:]),
        dr.dtype,
        tuple(dr.stride()[1:]),
    )


def _logical_key(entry):
    p = entry.payload
    rows = int(p.state_indices.shape[0])
    host_rows = tuple(getattr(p, "request_rows", ()))
    host_lens = tuple(getattr(p, "query_lens", ()))
    if len(host_rows) != rows or len(host_lens) != rows:
        # Without host row evidence a group cannot share a physical launch.
        return (id(entry.metadata),)
    return (host_rows, host_lens, p.block_size, p.block_table is not None)


def _publisher_descriptors(buckets):
    """Persistent device table (valid ptr, col ptr, capacity, groups) per bucket."""
    owner = buckets[0]
    key = tuple((id(b.valid), id(b.col), b.capacity, len(b.contexts)) for b in buckets)
    if getattr(owner, "_publisher_key", None) != key:
        values = []
        for bucket in buckets:
            for value in (bucket.valid.data_ptr(), bucket.col.data_ptr(), bucket.capacity, len(bucket.contexts)):
                values.append(value if value < (1 << 63) else value - (1 << 64))
        owner._publisher_descriptors = torch.tensor(values, dtype=torch.int64, device=owner.device)
        owner._publisher_plan_owners = tuple((b.valid, b.col) for b in buckets)
        owner._publisher_key = key
    return owner._publisher_descriptors


def _publish_spec(buckets, request_indices, idx_mapping, persistent_cols, persistent_accepted, rows):
    descriptors = _publisher_descriptors(buckets)
    args = (
        descriptors.data_ptr(),
        len(buckets),
        request_indices.data_ptr(),
        N.dtype_code(request_indices.dtype),
        request_indices.stride(0),
        request_indices.shape[0],
        idx_mapping.data_ptr(),
        N.dtype_code(idx_mapping.dtype),
        idx_mapping.numel(),
        persistent_cols.data_ptr(),
        persistent_accepted.data_ptr(),
        min(persistent_cols.numel(), persistent_accepted.numel()),
        rows,
    )
    spec = _LaunchSpec(
        "publish",
        N.load().gdn_recoverssm_publish,
        args,
        buckets[0].device,
        keepalive=(descriptors, request_indices, idx_mapping, persistent_cols, persistent_accepted),
    )
    spec.descriptors = descriptors
    return spec


class GroupedCommitBucket:
    """Stable per-layer address tables and per-group plan storage for one epoch."""

    def __init__(self, contexts):
        self.contexts = tuple(contexts)
        if not 0 < len(contexts) <= GROUPS_PER_BUCKET:
            raise ValueError("one recovery bucket requires one to three contexts")
        key = _layout_key(contexts[0])
        if any(_layout_key(c) != key for c in contexts[1:]):
            raise ValueError("grouped recovery requires homogeneous layer layouts")
        self.capacity = min(int(c.record_rows) for c in contexts)
        if self.capacity <= 0:
            raise ValueError("grouped recovery has no record rows")
        self.device = contexts[0].checkpoints[0].device
        self.checkpoints = tuple(t for c in contexts for t in c.checkpoints)
        self.conv_states = tuple(t for c in contexts for t in c.conv_states)
        self.records = tuple(t for c in contexts for t in c.records)
        self.layer_groups = torch.tensor(
            [g for g, c in enumerate(contexts) for _ in c.checkpoints], dtype=torch.int32, device=self.device
        )
        self.max_blocks = max(int(c.num_blocks) for c in contexts)
        self.spec_query_len = int(contexts[0].spec_query_len)
        self.record_layout = contexts[0].record_layout
        self.num_key_heads = int(contexts[0].num_key_heads)
        self.key_dtype = contexts[0].key_dtype
        self.conv_history_len = int(contexts[0].conv_history_len)
        self.state_addrs = _ptr_table(self.checkpoints, self.device)
        self.conv_addrs = _ptr_table(self.conv_states, self.device)
        self.state_block_strides = self._strides(self.checkpoints, 0)
        self.conv_block_strides = self._strides(self.conv_states, 0)
        self.conv_dim_strides = self._strides(self.conv_states, 1)
        self.conv_token_strides = self._strides(self.conv_states, 2)
        _, _, V, K = self.checkpoints[0].shape
        planes = [_record_planes(r, V, K) for r in self.records]
        self.corrections = tuple(p[0] for p in planes)
        self.keys = tuple(p[1] for p in planes)
        self.decays = tuple(p[2] for p in planes)
        key_off, decay_off = planes[0][3], planes[0][4]
        self.correction_addrs = _ptr_table(self.corrections, self.device)
        self.key_addrs = _ptr_table(self.keys, self.device, [key_off] * len(self.keys) if key_off else None)
        self.decay_addrs = _ptr_table(self.decays, self.device, [decay_off] * len(self.decays) if decay_off else None)
        self.correction_block_strides = self._strides(self.corrections, 0)
        self.key_block_strides = self._strides(self.keys, 0)
        self.decay_block_strides = self._strides(self.decays, 0)
        size = self.capacity * len(contexts)
        self.source = torch.zeros(size, dtype=torch.int32, device=self.device)
        self.length = torch.zeros_like(self.source)
        self.final = torch.zeros_like(self.source)
        self.boundary = torch.zeros_like(self.source)
        self.boundary_len = torch.zeros_like(self.source)
        self.valid = torch.zeros_like(self.source)
        self.col = torch.zeros_like(self.source)

    def _strides(self, tensors, dim):
        return torch.tensor([t.stride(dim) for t in tensors], dtype=torch.int64, device=self.device)

    def make_specs(
        self, entries, sampled, idx_mapping, persistent_cols, persistent_accepted, *, publish_align=True,
        fuse_plan_fold=True,
    ):
        """Launch specs of one bucket's commit: the fused plan + fold, then the
        conv compaction (with ``fuse_plan_fold=False``: plan, conv, fold as
        three launches, the reference's order, identical results)."""
        contexts = tuple(e.context for e in entries)
        if len(contexts) != len(self.contexts) or any(a is not b for a, b in zip(contexts, self.contexts)):
            raise ValueError("grouped recovery bucket belongs to a different KV epoch")
        p = tuple(e.payload for e in entries)
        rows = int(p[0].state_indices.shape[0])
        if not 0 < rows <= self.capacity:
            raise ValueError(
                "grouped recovery rows out of range: "
                f"rows={rows}, record capacity={self.capacity}, groups={len(p)}, state_indices shapes="
                f"{[tuple(x.state_indices.shape) for x in p]}"
            )
        if any(int(x.state_indices.shape[0]) != rows for x in p):
            raise ValueError("grouped recovery row counts differ")
        align = p[0].block_table is not None
        if any((x.block_table is not None) != align for x in p):
            raise ValueError("grouped recovery cannot mix align and none plans")
        if any(x.request_indices is None for x in p):
            raise ValueError("grouped recovery requires an explicit native row mapping")
        required = [sampled, idx_mapping, persistent_accepted]
        for x in p:
            required.extend((x.state_indices, x.query_start_loc, x.request_indices))
            if align:
                required.extend((x.block_table, x.num_computed_tokens))
        if align:
            required.append(persistent_cols)
        if any(t is None or t.device != self.device for t in required):
            raise ValueError("grouped recovery inputs must share the checkpoint device")
        if sampled.data_ptr() == persistent_accepted.data_ptr():
            raise ValueError("sampled counts must not alias persistent acceptance output")
        for x in p:
            if x.query_start_loc.numel() < rows + 1:
                raise ValueError("grouped recovery offsets are shorter than their rows")
            if align and (x.block_size is None or x.block_size < self.spec_query_len):
                raise ValueError("align blocks must cover the speculative window")
            if align and x.block_table.shape[1] <= 0:
                raise ValueError("align block table has no columns")
            host_rows = tuple(getattr(x, "request_rows", ()))
            if len(host_rows) == rows and any(r < 0 or r >= sampled.numel() or r >= idx_mapping.numel() for r in host_rows):
                raise ValueError("native request mapping exceeds the sampled batch")
        if self.device.type != "cuda":
            raise ValueError("grouped recovery runs on a HIP device")
        lib = N.load()
        groups = N.PlanGroups()
        for gi, (x, c) in enumerate(zip(p, contexts)):
            gr = groups[gi]
            gr.state_indices = x.state_indices.data_ptr()
            gr.si_stride = x.state_indices.stride(0)
            gr.si_dtype = N.dtype_code(x.state_indices.dtype)
            gr.query_start_loc = x.query_start_loc.data_ptr()
            gr.qsl_stride = x.query_start_loc.stride(0)
            gr.qsl_dtype = N.dtype_code(x.query_start_loc.dtype)
            gr.request_indices = x.request_indices.data_ptr()
            gr.map_stride = x.request_indices.stride(0)
            gr.map_dtype = N.dtype_code(x.request_indices.dtype)
            if align:
                gr.block_table = x.block_table.data_ptr()
                gr.table_row_stride = x.block_table.stride(0)
                gr.table_col_stride = x.block_table.stride(1)
                gr.table_width = x.block_table.shape[1]
                gr.table_rows = x.block_table.shape[0]
                gr.table_dtype = N.dtype_code(x.block_table.dtype)
                gr.num_computed = x.num_computed_tokens.data_ptr()
                gr.computed_stride = x.num_computed_tokens.stride(0)
                gr.computed_len = x.num_computed_tokens.shape[0]
                gr.computed_dtype = N.dtype_code(x.num_computed_tokens.dtype)
                gr.block_size = int(x.block_size)
            else:
                gr.block_size = 1
                gr.table_width = 1
            gr.num_blocks = int(c.num_blocks)
        flags = N.PLAN_GROUPED | (N.PLAN_ALIGN if align else 0) | (N.PLAN_PUBLISH if (align and publish_align) else 0)
        plan_args = (
            sampled.data_ptr(),
            N.dtype_code(sampled.dtype),
            sampled.stride(0),
            sampled.numel(),
            groups,
            len(p),
            self.source.data_ptr(),
            self.length.data_ptr(),
            self.final.data_ptr(),
            self.boundary.data_ptr(),
            self.boundary_len.data_ptr(),
            self.valid.data_ptr(),
            self.col.data_ptr(),
            idx_mapping.data_ptr(),
            N.dtype_code(idx_mapping.dtype),
            idx_mapping.numel(),
            None if persistent_cols is None else persistent_cols.data_ptr(),
            persistent_accepted.data_ptr(),
            min(persistent_accepted.numel(), persistent_cols.numel() if persistent_cols is not None else 0),
            rows,
            self.capacity,
            NULL_BLOCK_ID,
            self.spec_query_len,
            flags,
        )
        keep = [sampled, idx_mapping, persistent_cols, persistent_accepted]
        for x in p:
            keep.extend((x.state_indices, x.query_start_loc, x.request_indices, x.block_table, x.num_computed_tokens))
        plan = _LaunchSpec("plan", lib.gdn_recoverssm_plan, plan_args, self.device, keepalive=(groups, *keep))
        plan.flags = flags
        plan.num_groups = len(p)
        conv = self.conv_states[0]
        _require(conv.element_size() in (2, 4), "conv state elements must be 2 or 4 bytes")
        compact_args = (
            self.conv_addrs.data_ptr(),
            self.conv_block_strides.data_ptr(),
            self.conv_dim_strides.data_ptr(),
            self.conv_token_strides.data_ptr(),
            self.source.data_ptr(),
            N.DT_I32,
            1,
            self.length.data_ptr(),
            self.final.data_ptr(),
            self.boundary.data_ptr(),
            self.boundary_len.data_ptr(),
            self.layer_groups.data_ptr(),
            self.capacity,
            NULL_BLOCK_ID,
            rows,
            len(self.conv_states),
            int(conv.shape[1]),
            self.conv_history_len,
            int(conv.shape[2]),
            self.max_blocks,
            conv.element_size(),
            1 if align else 0,
        )
        compact = _LaunchSpec("conv", lib.gdn_recoverssm_conv_compact, compact_args, self.device)
        state = self.checkpoints[0]
        _, hv, v, k = state.shape
        rr, kr, dr = self.corrections[0], self.keys[0], self.decays[0]
        soa = self.record_layout == "soa"
        fold = _make_fold_spec(
            ref=state,
            record_rows=self.capacity,
            corr_strides=rr.stride()[1:3],
            key_strides=kr.stride()[1:3] if soa else rr.stride()[1:3],
            decay_strides=dr.stride()[1:3] if soa else rr.stride()[1:3],
            key_heads=self.num_key_heads,
            key_dtype=self.key_dtype,
            num_layers=len(self.checkpoints),
            rows=rows,
            plan_capacity=self.capacity,
            num_blocks=self.max_blocks,
            spec_query_len=self.spec_query_len,
            tables=(
                self.state_addrs, self.state_block_strides, self.correction_addrs, self.correction_block_strides,
                self.key_addrs, self.key_block_strides, self.decay_addrs, self.decay_block_strides,
            ),
            layer_groups=self.layer_groups,
            source=self.source,
            plan=(self.length, self.final, self.boundary, self.boundary_len),
            refs=(rr, kr, dr),
        )
        if not fuse_plan_fold:
            return plan, compact, fold
        # One launch plans and folds; the conv compaction reads the stored plan after it.
        return _fuse_plan_fold(plan, fold), compact


class GroupedCommitCoordinator:
    """One coordinator belongs to one RecoverSSMState, never a module global."""

    def __init__(self):
        self._buckets = {}
        self._seen = set()
        self.steps = 0
        self.last_launch_count = 0
        self.last_group_count = 0
        self.last_rows = 0

    def commit(self, metadata, sampled, idx_mapping, persistent_cols, persistent_accepted):
        entries = []
        for m in metadata:
            p = getattr(m, "recoverssm_commit", None)
            builder = getattr(m, "recoverssm_builder", None)
            if p is None or builder is None:
                continue
            context = getattr(m, "recoverssm_context", None)
            if context is None:
                raise RuntimeError("a serving RecoverSSM commit has no producer binding epoch")
            entries.append(CommitEntry(m, p, context))
        if not entries:
            self.last_launch_count = self.last_group_count = self.last_rows = 0
            return
        aligned = [e for e in entries if e.payload.block_table is not None]
        if aligned:
            if len(aligned) != len(entries):
                raise ValueError("one recovery step cannot mix align and none ownership")
            logical = _logical_key(aligned[0])
            if len(logical) == 1 or any(_logical_key(e) != logical for e in aligned[1:]):
                raise ValueError("GDN groups must agree on logical rows, query lengths and align block size")
            if any(e.context.spec_query_len != entries[0].context.spec_query_len for e in entries):
                raise ValueError("GDN groups must agree on the speculative window")
        logical_groups = {}
        for entry in entries:
            key = (_layout_key(entry.context), _logical_key(entry))
            logical_groups.setdefault(key, []).append(entry)
        grouped = [
            items[start : start + GROUPS_PER_BUCKET]
            for items in logical_groups.values()
            for start in range(0, len(items), GROUPS_PER_BUCKET)
        ]
        live = {}
        launches = 0
        for subset in grouped:
            contexts = tuple(e.context for e in subset)
            epoch = tuple(id(c) for c in contexts)
            bucket = self._buckets.get(epoch)
            if bucket is None:
                prepared = getattr(subset[0].metadata.recoverssm_builder, "_prepared_group_bucket", None)
                if (
                    prepared is not None
                    and len(prepared.contexts) == len(contexts)
                    and all(a is b for a, b in zip(prepared.contexts, contexts))
                ):
                    bucket = prepared
                else:
                    bucket = GroupedCommitBucket(contexts)
            live[epoch] = bucket
            specs = bucket.make_specs(
                subset, sampled, idx_mapping, persistent_cols, persistent_accepted, publish_align=len(grouped) == 1
            )
            for spec in specs:
                spec.launch()
            launches += len(specs)
        if aligned and len(grouped) > 1:
            buckets = tuple(live.values())
            publish = _publish_spec(
                buckets,
                entries[0].payload.request_indices,
                idx_mapping,
                persistent_cols,
                persistent_accepted,
                int(entries[0].payload.state_indices.shape[0]),
            )
            publish.launch()
            launches += 1
        # Retain only the current epochs.
        self._buckets = live
        self.steps += 1
        self.last_launch_count = launches
        self.last_group_count = len(entries)
        self.last_rows = int(entries[0].payload.state_indices.shape[0])
        reason = (len(entries), len(grouped))
        if reason not in self._seen:
            self._seen.add(reason)
            logger.info("GDN recovery coordinator: groups=%d buckets=%d launches=%d", len(entries), len(grouped), launches)


def prepare_grouped_commit(builders, block_tables=None, *, num_computed_tokens=None):
    """Build and validate the serving-shaped grouped launches before requests arrive.

    Mirrors the reference's compile-only preparation: it binds the real
    contexts, uses one-row dummies for the per-step inputs and leaves the
    prepared bucket on each builder (``_prepared_group_bucket``) for the
    coordinator to adopt. Returns the number of prepared launches.
    """
    from types import SimpleNamespace

    groups = {}
    for builder in builders:
        context = builder._get_context()
        if context is not None:
            align = builder.vllm_config.cache_config.mamba_cache_mode == "align"
            key = (_layout_key(context), align, int(builder.kv_cache_spec.block_size))
            groups.setdefault(key, []).append((builder, context))
    total = 0
    prepared_buckets, prepared_entries = [], []
    chunks = [items[s : s + GROUPS_PER_BUCKET] for items in groups.values() for s in range(0, len(items), GROUPS_PER_BUCKET)]
    mapping = cols = accepted = None
    for items in chunks:
        bucket = GroupedCommitBucket(tuple(c for _, c in items))
        dev = bucket.device
        entries = []
        for builder, context in items:
            q = context.spec_query_len
            native_state_table = getattr(builder, "spec_state_indices_tensor", None)
            if native_state_table is not None and getattr(native_state_table, "shape", (0,))[0] >= 1:
                table = native_state_table[:1]
            else:
                table = torch.zeros((1, q), dtype=torch.int32, device=dev)
            align = builder.vllm_config.cache_config.mamba_cache_mode == "align"
            block_size = int(builder.kv_cache_spec.block_size)
            if align:
                group_id = getattr(builder, "_gdn_kv_cache_group_id", None)
                bound = getattr(block_tables, "input_block_tables", None)
                if bound is None or group_id is None or not 0 <= group_id < len(bound):
                    raise RuntimeError("grouped align preparation requires the bound native group table")
                bound_table = bound[group_id][:1]
            else:
                bound_table = None

            def _at_least(tensor, rows, *, dtype=torch.int32):
                if tensor is not None and getattr(tensor, "shape", (0,))[0] >= rows:
                    return tensor[:rows]
                return torch.zeros((rows,), dtype=dtype, device=dev)

            qsl_src = getattr(builder, "spec_query_start_loc", None)
            map_src = getattr(builder, "spec_sequence_indices", None)
            payload = SimpleNamespace(
                state_indices=table[:, 0],
                query_start_loc=_at_least(qsl_src, 2, dtype=getattr(qsl_src, "dtype", torch.int32)),
                request_indices=_at_least(map_src, 1, dtype=getattr(map_src, "dtype", torch.int32)),
                block_table=bound_table,
                num_computed_tokens=(
                    num_computed_tokens[:1] if num_computed_tokens is not None else torch.zeros(1, dtype=torch.int32, device=dev)
                )
                if align
                else None,
                block_size=block_size if align else None,
                request_rows=(0,),
                query_lens=(q,),
            )
            entries.append(CommitEntry(None, payload, context))
        sampled = torch.zeros(1, dtype=torch.int32, device=dev)
        mapping = torch.zeros(1, dtype=torch.int32, device=dev)
        cols = torch.zeros(1, dtype=torch.int32, device=dev)
        accepted = torch.zeros(1, dtype=torch.int32, device=dev)
        for spec in bucket.make_specs(entries, sampled, mapping, cols, accepted, publish_align=len(chunks) == 1):
            spec.compile_only()
            total += 1
        prepared_buckets.append(bucket)
        prepared_entries.extend(entries)
        for builder, _ in items:
            builder._prepared_group_bucket = bucket
    if len(prepared_buckets) > 1 and prepared_entries[0].payload.block_table is not None:
        if len({e.payload.block_size for e in prepared_entries}) != 1:
            raise ValueError("shared GDN align ownership requires one block size")
        _publish_spec(tuple(prepared_buckets), prepared_entries[0].payload.request_indices, mapping, cols, accepted, 1).compile_only()
        total += 1
    return total


__all__ = [
    "CommitEntry",
    "GroupedCommitBucket",
    "GroupedCommitCoordinator",
    "prepare_grouped_commit",
]

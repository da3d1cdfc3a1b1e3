"""Grouped commit: every GDN cache group of a step committed in shared launches.

The public names and their contract are the reference plugin's
``gdn_recoverssm_ascend/grouped_commit.py``: ``CommitEntry``,
``GroupedCommitBucket``, ``GroupedCommitCoordinator`` and
``prepare_grouped_commit``. A step's cache groups are partitioned into
buckets of at most three groups that share one page layout and one set of
logical rows; each bucket commits with ``gdn_recoverssm_plan_fold`` (plan and
fold in one launch) and ``gdn_recoverssm_conv_compact``, and an align-mode
step split over several buckets publishes the persistent running columns once
every bucket has committed (``gdn_recoverssm_publish``). ``make_specs(...,
fuse_plan_fold=False)`` gives plan, conv and fold as three launches instead,
with identical results.
"""

from __future__ import annotations

import logging
from dataclasses import dataclass
from types import SimpleNamespace
from typing import Any

import torch

from . import _native as N
from ._rules import enforce, fail, require
from ._tables import LayerPages
from .kernels import (_FOLD_LENGTHS_ARG, NULL_BLOCK_ID, PendingCommit, _conv_spec, _fill_plan_group,
                      _fold_rows_spec, _fuse_plan_fold, _LaunchSpec, _make_fold_spec, _MarkFolded, _picked_rows,
                      _request_row_map, _settle_spec)

logger = logging.getLogger("gdn_recoverssm_ascend.grouped_commit")

# Cache groups per physical bucket (reference grouped_commit.py:947-954).
GROUPS_PER_BUCKET = 3


@dataclass(frozen=True)
class CommitEntry:
    """One cache group's share of a step: its attention metadata, the commit
    payload the metadata carries, and the commit context of its layers."""

    metadata: Any
    payload: Any
    context: Any


# ---------------------------------------------------------------------------
# What may share a bucket
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class _PageLayout:
    """Everything the shared launches take from the first layer of a bucket:
    the members' pages, conv states and records must agree on all of it."""

    device: Any
    state: tuple
    conv: tuple
    conv_history: int
    window: int
    records: tuple

    @classmethod
    def of(cls, context) -> "_PageLayout":
        pages = context.pages
        state, conv = pages.checkpoints[0], pages.conv_states[0]
        planes = pages.first_planes

        def form(t):
            return (t.dtype, tuple(t.shape[1:]), tuple(t.stride()[1:]))

        return cls(state.device, form(state), form(conv), int(context.conv_history_len), int(context.spec_query_len),
                   (context.record_layout, int(context.num_key_heads), form(planes.correction), form(planes.key),
                    form(planes.decay)))


@dataclass(frozen=True)
class _LogicalRows:
    """The rows a group's payload commits, from the host-side evidence the
    metadata builder records (request row and query length of every row),
    with the align block size. Groups can share launches only when they
    agree on all of it."""

    request_rows: tuple
    query_lens: tuple
    block_size: Any
    align: bool


@dataclass(frozen=True)
class _Unshared:
    """A payload without host row evidence: it commits in a bucket of its own."""

    owner: int


def _rows_of(entry: CommitEntry):
    payload = entry.payload
    evidence = tuple(tuple(getattr(payload, name, ())) for name in ("request_rows", "query_lens"))
    if any(len(e) != len(payload.state_indices) for e in evidence):
        return _Unshared(id(entry.metadata))
    return _LogicalRows(*evidence, payload.block_size, payload.block_table is not None)


def _partition(entries: list) -> list:
    """Buckets of at most ``GROUPS_PER_BUCKET`` entries that agree on page
    layout and logical rows, in first-seen order."""
    classes: dict = {}
    for entry in entries:
        classes.setdefault((_PageLayout.of(entry.context), _rows_of(entry)), []).append(entry)
    return [members[i:i + GROUPS_PER_BUCKET] for members in classes.values()
            for i in range(0, len(members), GROUPS_PER_BUCKET)]


# ---------------------------------------------------------------------------
# Publication across buckets (grouped_commit.py:531-610)
# ---------------------------------------------------------------------------


def _publisher_descriptors(buckets) -> torch.Tensor:
    """(valid pointer, column pointer, capacity, groups) of every bucket, as
    one int64 device table, cached on the first bucket while the same plan
    arrays are in use; the cache keeps those arrays (only them) alive."""
    owner = buckets[0]
    # The table's own words identify it: the same plan arrays, capacities and
    # group counts give the same words.
    words = tuple(w for b in buckets for w in (b.valid.data_ptr(), b.col.data_ptr(), b.capacity, len(b.contexts)))
    cached = owner.__dict__.get("_publisher")
    if cached is None or cached[0] != words:
        signed = [w - (1 << 64) if w >= (1 << 63) else w for w in words]
        table = torch.tensor(signed, dtype=torch.int64, device=owner.device)
        owner._publisher = (words, table, tuple((b.valid, b.col) for b in buckets))
    return owner._publisher[1]


def _publish_spec(buckets, request_indices, idx_mapping, persistent_cols, persistent_accepted, rows) -> _LaunchSpec:
    table = _publisher_descriptors(buckets)
    args = (table.data_ptr(), len(buckets), request_indices.data_ptr(), N.dtype_code(request_indices.dtype),
            request_indices.stride(0), request_indices.shape[0], idx_mapping.data_ptr(),
            N.dtype_code(idx_mapping.dtype), idx_mapping.numel(), persistent_cols.data_ptr(),
            persistent_accepted.data_ptr(), min(persistent_cols.numel(), persistent_accepted.numel()), rows)
    spec = _LaunchSpec("publish", N.load().gdn_recoverssm_publish, args, buckets[0].device,
                       keepalive=(table, request_indices, idx_mapping, persistent_cols, persistent_accepted))
    spec.descriptors = table
    return spec


# ---------------------------------------------------------------------------
# Buckets
# ---------------------------------------------------------------------------


def _bucket_rules(bucket, entries, payloads, rows, sampled, idx_mapping, persistent_cols, persistent_accepted):
    align = payloads[0].block_table is not None
    needed = [sampled, idx_mapping, persistent_accepted] + ([persistent_cols] if align else [])
    for p in payloads:
        needed += [p.state_indices, p.query_start_loc, p.request_indices]
        needed += [p.block_table, p.num_computed_tokens] if align else []

    def host_rows_fit(p):
        host = tuple(getattr(p, "request_rows", ()))
        limit = min(sampled.numel(), idx_mapping.numel())
        return len(host) != rows or all(0 <= r < limit for r in host)

    return (
        ("grouped recovery row counts differ", lambda: all(int(p.state_indices.shape[0]) == rows for p in payloads)),
        ("grouped recovery cannot mix align and none plans",
         lambda: all((p.block_table is not None) == align for p in payloads)),
        ("grouped recovery requires an explicit native row mapping",
         lambda: all(p.request_indices is not None for p in payloads)),
        ("grouped recovery inputs must share the checkpoint device",
         lambda: all(t is not None and t.device == bucket.device for t in needed)),
        ("sampled counts must not alias persistent acceptance output",
         lambda: sampled.data_ptr() != persistent_accepted.data_ptr()),
        ("grouped recovery offsets are shorter than their rows",
         lambda: all(p.query_start_loc.numel() >= rows + 1 for p in payloads)),
        ("align blocks must cover the speculative window",
         lambda: not align or all(p.block_size is not None and p.block_size >= bucket.spec_query_len
                                  for p in payloads)),
        ("align block table has no columns", lambda: not align or all(p.block_table.shape[1] > 0 for p in payloads)),
        ("native request mapping exceeds the sampled batch", lambda: all(host_rows_fit(p) for p in payloads)),
        ("grouped recovery runs on a HIP device", lambda: bucket.device.type == "cuda"),
    )


class GroupedCommitBucket:
    """One to three cache groups of one epoch committed by shared launches:
    the address tables of all their layers (built once) and one plan slot of
    ``capacity`` rows per group."""

    def __init__(self, contexts):
        contexts = tuple(contexts)
        enforce((
            ("one recovery bucket requires one to three contexts", lambda: 0 < len(contexts) <= GROUPS_PER_BUCKET),
            ("grouped recovery requires homogeneous layer layouts",
             lambda: len({_PageLayout.of(c) for c in contexts}) == 1),
            ("grouped recovery has no record rows", lambda: min(int(c.record_rows) for c in contexts) > 0),
        ))
        first = contexts[0]
        self.contexts = contexts
        self.capacity = min(int(c.record_rows) for c in contexts)
        self.device = first.checkpoints[0].device
        self.spec_query_len = int(first.spec_query_len)
        self.record_layout = first.record_layout
        self.num_key_heads = int(first.num_key_heads)
        self.key_dtype = first.key_dtype
        self.conv_history_len = int(first.conv_history_len)
        self.max_blocks = int(max(c.num_blocks for c in contexts))
        self.pages = LayerPages([t for c in contexts for t in c.conv_states],
                                [t for c in contexts for t in c.checkpoints],
                                [t for c in contexts for t in c.records], self.device)
        # Each layer's group: context g's layers all map to plan group g.
        per_context = torch.tensor([len(c.checkpoints) for c in contexts])
        self.layer_groups = torch.repeat_interleave(torch.arange(len(contexts), dtype=torch.int32),
                                                    per_context).to(self.device)
        # Plan arrays: group g's row r at g * capacity + r.
        # settle_length / settle_rows / settle_count: what a deferred settle
        # folds (lengths, the rows it lists, their number).
        for name in ("source", "length", "final", "boundary", "boundary_len", "valid", "col", "settle_length"):
            setattr(self, name, torch.zeros(self.capacity * len(contexts), dtype=torch.int32, device=self.device))
        self.settle_rows = torch.zeros(self.capacity, dtype=torch.int32, device=self.device)
        self.settle_count = torch.zeros(1, dtype=torch.int32, device=self.device)

    checkpoints = property(lambda self: self.pages.checkpoints)
    conv_states = property(lambda self: self.pages.conv_states)
    records = property(lambda self: self.pages.records)

    def make_specs(self, entries, sampled, idx_mapping, persistent_cols, persistent_accepted, *, publish_align=True,
                   fuse_plan_fold=True):
        """The launch specs of one bucket's commit: plan + fold, then the conv
        compaction (``fuse_plan_fold=False``: plan, conv, fold)."""
        entries = tuple(entries)
        if len(entries) != len(self.contexts) or any(e.context is not c for e, c in zip(entries, self.contexts)):
            fail("grouped recovery bucket belongs to a different KV epoch")
        payloads = tuple(e.payload for e in entries)
        rows = len(payloads[0].state_indices)
        if rows < 1 or rows > self.capacity:
            shapes = [tuple(p.state_indices.shape) for p in payloads]
            fail(f"grouped recovery rows out of range: rows={rows}, record capacity={self.capacity}, "
                 f"groups={len(payloads)}, state_indices shapes={shapes}")
        enforce(_bucket_rules(self, entries, payloads, rows, sampled, idx_mapping, persistent_cols,
                              persistent_accepted))
        align = payloads[0].block_table is not None
        groups = N.PlanGroups()
        for g, (p, context) in enumerate(zip(payloads, self.contexts)):
            _fill_plan_group(groups[g], state_indices=p.state_indices, query_start_loc=p.query_start_loc,
                             request_indices=p.request_indices, block_table=p.block_table if align else None,
                             num_computed_tokens=p.num_computed_tokens if align else None, block_size=p.block_size,
                             num_blocks=context.num_blocks)
        flags = N.PLAN_GROUPED | (N.PLAN_ALIGN | (N.PLAN_PUBLISH if publish_align else 0) if align else 0)
        persistent_len = min(persistent_accepted.numel(), persistent_cols.numel() if persistent_cols is not None else 0)
        plan_args = (sampled.data_ptr(), N.dtype_code(sampled.dtype), sampled.stride(0), sampled.numel(), groups,
                     len(payloads), self.source.data_ptr(), self.length.data_ptr(), self.final.data_ptr(),
                     self.boundary.data_ptr(), self.boundary_len.data_ptr(), self.valid.data_ptr(),
                     self.col.data_ptr(), idx_mapping.data_ptr(), N.dtype_code(idx_mapping.dtype),
                     idx_mapping.numel(), None if persistent_cols is None else persistent_cols.data_ptr(),
                     persistent_accepted.data_ptr(), persistent_len, rows, self.capacity, NULL_BLOCK_ID,
                     self.spec_query_len, flags)
        held = [sampled, idx_mapping, persistent_cols, persistent_accepted]
        for p in payloads:
            held += [p.state_indices, p.query_start_loc, p.request_indices, p.block_table, p.num_computed_tokens]
        plan = _LaunchSpec("plan", N.load().gdn_recoverssm_plan, plan_args, self.device, keepalive=(groups, *held))
        plan.flags = flags
        plan.num_groups = len(payloads)
        arrays = (self.length, self.final, self.boundary, self.boundary_len)
        compact = _conv_spec(self.pages, source=self.source, source_dtype=N.DT_I32, source_stride=1, plan=arrays,
                             layer_groups=self.layer_groups, capacity=self.capacity, rows=rows,
                             history=self.conv_history_len, max_blocks=self.max_blocks, align=align,
                             device=self.device)
        fold = _make_fold_spec(pages=self.pages, record_rows=self.capacity, key_heads=self.num_key_heads,
                               key_dtype=self.key_dtype, rows=rows, plan_capacity=self.capacity,
                               num_blocks=self.max_blocks, spec_query_len=self.spec_query_len,
                               layer_groups=self.layer_groups, source=self.source, plan=arrays)
        if not fuse_plan_fold:
            return plan, compact, fold
        return _fuse_plan_fold(plan, fold), compact


# ---------------------------------------------------------------------------
# Deferred grouped commit (docs/GDN-RecoverSSM-实现方案.md:515-527, 563-568)
# ---------------------------------------------------------------------------


class DeferredGroupedCommit:
    """One step's grouped commit with its folds left to the next step's
    verifies (``gdn_recoverssm_verify_deferred``): every bucket's plan is
    stored, the conv states are compacted and the align columns published,
    exactly as ``GroupedCommitCoordinator.commit`` does them; only the folds
    wait.

    ``pending(i)`` gives one ``PendingCommit`` per layer of the step's i-th
    committing cache group (metadata order). All share one row map (next row
    -> pending row), the in-place map until ``continue_with`` re-keys it by
    request. Every pending row must be folded once before its pages are
    reused: by the next verify that continues it, or here, by ``settle``
    (every row the next verifies will not apply, decided on the device) or
    ``flush`` (given rows, or all). Both mark what they fold in the plan, so
    a later settle or flush skips it; a row a verify has applied must not be
    flushed. The object stays valid until the same
    contexts commit again (their plan arrays are reused then): a deferred
    flow alternates two sets of contexts, as the pending step's records must
    not be the ones the next verify writes.
    """

    def __init__(self, entries, placed, rows, device):
        self._entries = tuple(entries)
        self._placed = tuple(placed)  # per entry: (bucket, its group in the bucket, fold spec)
        self.num_rows = int(rows)
        self.rows = torch.arange(max(1, self.num_rows), dtype=torch.int32, device=device)

    def __len__(self):
        return len(self._entries)

    def _plan(self, i):
        bucket, g, _ = self._placed[i]
        seg = slice(g * bucket.capacity, (g + 1) * bucket.capacity)
        return tuple(t[seg] for t in (bucket.source, bucket.length, bucket.final, bucket.boundary,
                                      bucket.boundary_len))

    def pending(self, i) -> tuple:
        """The pending commits of group ``i``'s layers, in its context's layer order."""
        plan = self._plan(i)
        return tuple(PendingCommit(self.rows, *plan, rec, num_rows=self.num_rows)
                     for rec in self._entries[i].context.records)

    def continue_with(self, previous_requests, next_requests) -> list:
        """Key the pending rows by request for the next batch (host-side ids,
        as ``continue_pending``): ``previous_requests[r]`` is the request of
        pending row r, ``next_requests[b]`` that of next row b. Returns the
        sorted pending rows whose request left; ``settle`` or ``flush`` must
        fold them."""
        self.rows, left = _request_row_map(self.num_rows, previous_requests, next_requests, self.rows.device)
        return left

    def _fold(self, bucket, fold, lengths) -> None:
        args = list(fold.args)
        args[_FOLD_LENGTHS_ARG] = lengths.data_ptr()
        _LaunchSpec(fold.name, fold.fn, tuple(args), fold.device, keepalive=fold.keepalive + (lengths,)).launch()

    def _buckets(self):
        seen = {}
        for i, (bucket, g, fold) in enumerate(self._placed):
            seen.setdefault(id(bucket), (bucket, fold, []))[2].append((i, g))
        return seen.values()

    def flush(self, rows=None) -> None:
        """Fold the given pending rows (every planned row when None) of every
        group now, with the ordinary fold, and mark them folded in the plan
        (accepted length 0), so a later flush or settle does not fold them
        again."""
        picked = None
        if rows is not None:
            picked = _picked_rows(rows, self.num_rows, self.rows.device)
            if picked is None:
                return
        for bucket, fold, _ in self._buckets():
            if picked is None:
                self._fold(bucket, fold, bucket.length)
                _MarkFolded(bucket.length, bucket.capacity, num_rows=self.num_rows).launch()
            else:
                # Every group of a bucket is a member of the step: the row list
                # folds the picked rows of each (plan row g * capacity + r).
                _fold_rows_spec(fold, picked).launch()
                _MarkFolded(bucket.length, bucket.capacity, picked).launch()

    def settle(self, next_metadata) -> None:
        """Fold now every pending row that the next step's deferred verifies
        will not apply: group i of ``next_metadata`` (the next step's
        metadata, same group order) continues pending row ``rows[b]`` in its
        row b only when its state index there is that commit's final page.
        Decided on the device; call it before the next verifies."""
        nxt = _step_entries(next_metadata)
        require(len(nxt) == len(self._entries), "the next step has another number of committing groups")
        if self.num_rows == 0:
            return  # nothing is pending
        for bucket, fold, members in self._buckets():
            # The device decides which rows to fold, lists them in the
            # bucket's own arrays and marks them folded in the plan (the rows
            # the verifies apply keep their lengths), one launch for its
            # groups; the fold covers the listed rows only.
            nexts = [None] * (bucket.length.shape[0] // bucket.capacity)
            for i, g in members:
                nexts[g] = nxt[i].payload.state_indices
            _settle_spec(bucket.length, bucket.final, bucket.capacity, self.num_rows, self.rows, nexts,
                         bucket.settle_length, bucket.settle_rows, bucket.settle_count).launch()
            _fold_rows_spec(fold, bucket.settle_rows, bucket.settle_count, lengths=bucket.settle_length,
                            listed=self.num_rows).launch()


# ---------------------------------------------------------------------------
# The coordinator
# ---------------------------------------------------------------------------


def _step_entries(metadata) -> list:
    """The cache groups of a step that carry a RecoverSSM commit."""
    def carries_commit(m) -> bool:
        return all(getattr(m, name, None) is not None for name in ("recoverssm_commit", "recoverssm_builder"))

    committing = [m for m in metadata if carries_commit(m)]
    if any(getattr(m, "recoverssm_context", None) is None for m in committing):
        raise RuntimeError("a serving RecoverSSM commit has no producer binding epoch")
    return [CommitEntry(m, m.recoverssm_commit, m.recoverssm_context) for m in committing]


def _check_step(entries) -> bool:
    """An align-mode step: every group in align mode, all on one set of
    logical rows and one window. Returns whether the step is in align mode."""
    aligned = [e.payload.block_table is not None for e in entries]
    if not any(aligned):
        return False
    first = _rows_of(entries[0])
    enforce((
        ("one recovery step cannot mix align and none ownership", lambda: all(aligned)),
        ("GDN groups must agree on logical rows, query lengths and align block size",
         lambda: isinstance(first, _LogicalRows) and all(_rows_of(e) == first for e in entries)),
        ("GDN groups must agree on the speculative window",
         lambda: len({e.context.spec_query_len for e in entries}) == 1),
    ))
    return True


class GroupedCommitCoordinator:
    """The grouped commit of one model instance's state (one per serving
    state, never shared through a module global). Buckets are cached by the
    identity of their contexts: a cache epoch reuses its buckets and their
    address tables, and a step keeps only the buckets it used, so a released
    epoch's pages are not held."""

    def __init__(self):
        self._buckets: dict = {}        # context identities -> bucket, the last step's only
        self._previous: dict = {}       # a deferred flow's step before it (its contexts alternate)
        self._logged_shapes: set = set()
        self.steps = 0
        self._note_step(0, 0, 0)

    def _note_step(self, launches: int, groups: int, rows: int) -> None:
        """The last step's diagnostics: launches issued, groups committed, rows."""
        self.last_launch_count, self.last_group_count, self.last_rows = launches, groups, rows

    def _bucket_for(self, members) -> GroupedCommitBucket:
        contexts = tuple(e.context for e in members)
        key = tuple(map(id, contexts))
        if key in self._buckets:
            return self._buckets[key]
        if key in self._previous:
            return self._previous[key]
        # A bucket built by prepare_grouped_commit for exactly these contexts is adopted.
        prepared = getattr(members[0].metadata.recoverssm_builder, "_prepared_group_bucket", None)
        if prepared is not None and tuple(map(id, prepared.contexts)) == key:
            return prepared
        return GroupedCommitBucket(contexts)

    def commit(self, metadata, sampled, idx_mapping, persistent_cols, persistent_accepted):
        self._commit(metadata, sampled, idx_mapping, persistent_cols, persistent_accepted, deferred=False)

    def commit_deferred(self, metadata, sampled, idx_mapping, persistent_cols,
                        persistent_accepted) -> DeferredGroupedCommit | None:
        """``commit`` with the folds left to the next step's verifies: plans,
        conv compaction and publication now, and a ``DeferredGroupedCommit``
        that hands each layer its ``PendingCommit`` (None when no group
        commits). The groups must share one set of logical rows and typed
        record buffers. Buckets of the previous step are kept as well, so a
        flow that alternates two sets of contexts reuses both."""
        return self._commit(metadata, sampled, idx_mapping, persistent_cols, persistent_accepted, deferred=True)

    def _commit(self, metadata, sampled, idx_mapping, persistent_cols, persistent_accepted, *, deferred):
        entries = _step_entries(metadata)
        if not entries:
            self._note_step(0, 0, 0)
            return None
        align = _check_step(entries)
        if deferred:
            first = _rows_of(entries[0])
            enforce((
                ("the deferred grouped commit needs every group on one set of logical rows",
                 lambda: isinstance(first, _LogicalRows) and all(_rows_of(e) == first for e in entries)),
                ("the deferred commit needs typed record buffers",
                 lambda: all(e.context.record_layout == "soa" for e in entries)),
            ))
        buckets = _partition(entries)
        used = {}
        placed = {}
        launches = 0
        for members in buckets:
            bucket = self._bucket_for(members)
            used[tuple(id(e.context) for e in members)] = bucket
            specs = bucket.make_specs(members, sampled, idx_mapping, persistent_cols, persistent_accepted,
                                      publish_align=len(buckets) == 1, fuse_plan_fold=not deferred)
            if deferred:
                plan, compact, fold = specs
                specs = (plan, compact)
                for g, e in enumerate(members):
                    placed[id(e)] = (bucket, g, fold)
            for spec in specs:
                spec.launch()
            launches += len(specs)
        rows = len(entries[0].payload.state_indices)
        if align and len(buckets) > 1:
            # The plans of every bucket are stored now: publish where all agree.
            _publish_spec(tuple(used.values()), entries[0].payload.request_indices, idx_mapping, persistent_cols,
                          persistent_accepted, rows).launch()
            launches += 1
        self._previous = self._buckets if deferred else {}
        self._buckets = used
        self.steps += 1
        self._note_step(launches, len(entries), rows)
        shape = (len(entries), len(buckets), launches, deferred)
        if shape not in self._logged_shapes:  # once per step shape
            self._logged_shapes.add(shape)
            logger.info("grouped RecoverSSM commit%s: %d cache groups in %d buckets, %d launches",
                        " (folds deferred)" if deferred else "", *shape[:3])
        if not deferred:
            return None
        device = entries[0].context.checkpoints[0].device
        return DeferredGroupedCommit(entries, [placed[id(e)] for e in entries], rows, device)


# ---------------------------------------------------------------------------
# Preparation before serving
# ---------------------------------------------------------------------------


def _probe_payload(builder, context, block_tables, num_computed_tokens, device):
    """A one-row payload in the serving signature of a builder's group: its
    own native buffers where they already hold a row, blanks otherwise."""
    window = context.spec_query_len
    align = builder.vllm_config.cache_config.mamba_cache_mode == "align"

    def first_rows(t, rows, dtype=torch.int32):
        return t[:rows] if t is not None and getattr(t, "shape", (0,))[0] >= rows else torch.zeros(
            rows, dtype=getattr(t, "dtype", dtype), device=device)

    table = getattr(builder, "spec_state_indices_tensor", None)
    state_table = table[:1] if table is not None and getattr(table, "shape", (0,))[0] >= 1 else torch.zeros(
        (1, window), dtype=torch.int32, device=device)
    block_table = computed = block_size = None
    if align:
        try:  # the builder's cache group selects its table among the bound native tables
            gid = int(builder._gdn_kv_cache_group_id)
            block_table = block_tables.input_block_tables[gid][:1] if gid >= 0 else None
        except (AttributeError, TypeError, IndexError):
            block_table = None
        if block_table is None:
            raise RuntimeError("grouped align preparation requires the bound native group table")
        computed = num_computed_tokens[:1] if num_computed_tokens is not None else torch.zeros(
            1, dtype=torch.int32, device=device)
        block_size = int(builder.kv_cache_spec.block_size)
    return SimpleNamespace(
        state_indices=state_table[:, 0],
        query_start_loc=first_rows(getattr(builder, "spec_query_start_loc", None), 2),
        request_indices=first_rows(getattr(builder, "spec_sequence_indices", None), 1),
        block_table=block_table, num_computed_tokens=computed, block_size=block_size,
        request_rows=(0,), query_lens=(window,),
    )


def prepare_grouped_commit(builders, block_tables=None, *, num_computed_tokens=None):
    """Build the serving buckets before requests arrive and check their launch
    signatures (compile-only: the kernels are built ahead of time).

    Builders are grouped as the coordinator will bucket them (page layout,
    align mode, block size; at most three per bucket); each bucket is bound to
    the real contexts and checked with one-row payloads in the serving
    signature, and left on its builders as ``_prepared_group_bucket`` for the
    coordinator to adopt. Returns the number of launches prepared.
    """
    classes: dict = {}
    for builder in builders:
        context = builder._get_context()
        if context is None:
            continue
        align = builder.vllm_config.cache_config.mamba_cache_mode == "align"
        key = (_PageLayout.of(context), align, int(builder.kv_cache_spec.block_size))
        classes.setdefault(key, []).append((builder, context))
    chunks = [members[i:i + GROUPS_PER_BUCKET] for members in classes.values()
              for i in range(0, len(members), GROUPS_PER_BUCKET)]
    prepared = 0
    buckets, payloads = [], []
    for members in chunks:
        bucket = GroupedCommitBucket(tuple(c for _, c in members))
        dev = bucket.device
        entries = [CommitEntry(None, _probe_payload(b, c, block_tables, num_computed_tokens, dev), c)
                   for b, c in members]
        one = [torch.zeros(1, dtype=torch.int32, device=dev) for _ in range(4)]  # sampled, mapping, cols, accepted
        for spec in bucket.make_specs(entries, *one, publish_align=len(chunks) == 1):
            spec.compile_only()
            prepared += 1
        buckets.append(bucket)
        payloads += [e.payload for e in entries]
        for builder, _ in members:
            builder._prepared_group_bucket = bucket
    if len(buckets) > 1 and payloads[0].block_table is not None:
        if len({p.block_size for p in payloads}) != 1:
            raise ValueError("shared GDN align ownership requires one block size")
        one = torch.zeros(1, dtype=torch.int32, device=buckets[0].device)
        _publish_spec(tuple(buckets), payloads[0].request_indices, one, one, one, 1).compile_only()
        prepared += 1
    return prepared


__all__ = [
    "CommitEntry",
    "DeferredGroupedCommit",
    "GroupedCommitBucket",
    "GroupedCommitCoordinator",
    "prepare_grouped_commit",
]

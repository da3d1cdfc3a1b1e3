"""The C-ABI library: builds, loads without a GPU, exports every declared
symbol, and its ctypes struct layouts match what the C compiler lays out.
No compute entry point is called with real work here (no GPU on this host)."""

import ctypes
import os
import re
import subprocess
import sys
import tempfile

import pytest

from gdn_recoverssm_ascend import _native as N
from gdn_recoverssm_ascend._build import INCLUDE_DIR, LIB_PATH

HEADER = os.path.join(INCLUDE_DIR, "gdn_recoverssm_hip.h")


def _declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(gdn_recoverssm_\w+)\s*\(", text)))


def test_library_is_built():
    assert os.path.exists(LIB_PATH), "run `python -c 'import __graft_entry__ as g; g.build()'` first"


def test_every_declared_symbol_is_exported():
    lib = ctypes.CDLL(LIB_PATH)
    declared = _declared_symbols()
    assert set(declared) == set(N.exported_symbols())
    for name in declared:
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", LIB_PATH], capture_output=True, text=True).stdout
    for name in declared:
        assert re.search(rf"\bT {name}\b", out), f"{name} not exported with C linkage"


def test_abi_version_and_error_channel():
    lib = N.load()
    assert lib.gdn_recoverssm_abi_version() == N.ABI_VERSION == 1
    assert isinstance(lib.gdn_recoverssm_last_error(), bytes)


def test_state_cache_retain_setting():
    """The verify cache hint: default 64 MiB, returns the previous value,
    rejects a negative byte count without changing the setting."""
    import gdn_recoverssm_ascend as G

    lib = N.load()
    prev = lib.gdn_recoverssm_set_state_cache_retain(0)
    try:
        assert prev == 64 << 20
        assert lib.gdn_recoverssm_set_state_cache_retain(-5) == -1
        assert G.set_state_cache_retain(12345) == 0
        with pytest.raises(ValueError, match="GDN RecoverSSM"):
            G.set_state_cache_retain(-1)
        assert G.set_state_cache_retain(prev) == 12345
    finally:
        lib.gdn_recoverssm_set_state_cache_retain(prev)


def test_per_call_cache_hint_field():
    """A call's own cache hint rides in gdn_verify_ext: 0 selects the
    process-wide setting, a positive byte count is used as given, and a
    request to retain nothing becomes a negative field; a negative request
    is refused before anything is built."""
    import torch

    from gdn_recoverssm_ascend.kernels import _retain_arg, _VerifyCall

    assert N.VerifyExt.state_cache_retain.offset == 56 and ctypes.sizeof(N.VerifyExt) == 64

    def field(nbytes):
        c = _VerifyCall(*([None] * 9), 4, True, None, None, _retain_arg(nbytes))
        return c.retain_field

    assert field(None) == 0
    assert field(256 << 20) == 256 << 20
    assert field(0) == -1
    with pytest.raises(ValueError, match="GDN RecoverSSM: the retained state bytes"):
        _retain_arg(-1)
    del torch


def test_invalid_arguments_are_rejected_before_any_launch():
    lib = N.load()
    ext = N.VerifyExt(key_dim=128, value_dim=128)
    cfg = N.i64_array([0] * 27)
    st = lib.gdn_recoverssm_verify(*([None] * 12), cfg, 27, 1.0, ctypes.byref(ext), None)
    assert st == N.GDN_ERR_INVALID
    assert b"28 config fields" in lib.gdn_recoverssm_last_error()
    # geometry: value heads not a multiple of key heads
    cfg = N.i64_array([1, 4, 3, 4, 4, 8, 1, 0] + [0] * 20)
    st = lib.gdn_recoverssm_verify(*([None] * 12), cfg, 28, 1.0, ctypes.byref(ext), None)
    assert st == N.GDN_ERR_INVALID and b"geometry" in lib.gdn_recoverssm_last_error()
    # unsupported key dim
    ext2 = N.VerifyExt(key_dim=512, value_dim=128)
    cfg = N.i64_array([1, 4, 1, 2, 4, 8, 1, 0] + [0] * 20)
    st = lib.gdn_recoverssm_verify(*([None] * 12), cfg, 28, 1.0, ctypes.byref(ext2), None)
    assert st == N.GDN_ERR_UNSUPPORTED
    # fold with the wrong field count
    fext = N.FoldExt(key_dim=128, value_dim=128)
    st = lib.gdn_recoverssm_fold(*([None] * 18), N.i64_array([0] * 16), 16, ctypes.byref(fext), None)
    assert st == N.GDN_ERR_INVALID
    # plan with no groups, conv with a bad element size, publish without outputs
    groups = N.PlanGroups()
    st = lib.gdn_recoverssm_plan(None, 3, 1, 0, groups, 0, *([None] * 7), None, 3, 0, None, None, 0, 1, 1, 0, 4, 0, None)
    assert st == N.GDN_ERR_INVALID
    st = lib.gdn_recoverssm_publish(None, 1, None, 3, 1, 1, None, 3, 1, None, None, 1, 1, None)
    assert st == N.GDN_ERR_INVALID
    # fused plan + fold: the plan block is checked first, then the fold
    # configuration, then that both describe the same rows
    launch = N.PlanLaunch(num_groups=0, groups=ctypes.cast(groups, ctypes.POINTER(N.PlanGroup)))
    st = lib.gdn_recoverssm_plan_fold(ctypes.byref(launch), *([None] * 13), N.i64_array([0] * 17), 17,
                                      ctypes.byref(fext), None)
    assert st == N.GDN_ERR_INVALID and b"num_groups" in lib.gdn_recoverssm_last_error()
    g0 = groups[0]
    # Addresses that are never dereferenced: every call here is rejected before a launch.
    g0.state_indices, g0.query_start_loc = 0x60000, 0x70000
    g0.si_dtype = g0.qsl_dtype = 3
    g0.si_stride = g0.qsl_stride = 1
    launch = N.PlanLaunch(sampled=0x50000, sampled_len=4, sampled_stride=1, sampled_dtype=3, num_groups=1,
                          groups=ctypes.cast(groups, ctypes.POINTER(N.PlanGroup)), lens_plan=0x10000,
                          final_plan=0x20000, boundary_plan=0x30000, boundary_lens_plan=0x40000, num_rows=4,
                          plan_capacity=4, spec_query_len=4)
    tables = [8] * 8
    fcfg = N.i64_array([4, 1, 4, 2, 4, 16, 4, 8, 0, 128 * 128, 128, 512, 128, 256, 128, 4, 1])
    fext1 = N.FoldExt(key_dim=128, value_dim=128, state_k_stride=1)
    st = lib.gdn_recoverssm_plan_fold(ctypes.byref(launch), None, None, None, None, *tables, None, fcfg, 17,
                                      ctypes.byref(fext1), None)
    assert st == N.GDN_ERR_INVALID and b"differ from the plan" in lib.gdn_recoverssm_last_error()
    # Record token strides outside a buffer resource's 32-bit window are refused.
    for field, value in ((12, -1), (14, -128), (12, 1 << 29), (14, 1 << 30)):
        bad = list(fcfg)
        bad[field] = value
        st = lib.gdn_recoverssm_plan_fold(ctypes.byref(launch), None, None, None, None, *tables, None,
                                          N.i64_array(bad), 17, ctypes.byref(fext1), None)
        assert st == N.GDN_ERR_UNSUPPORTED and b"record token strides" in lib.gdn_recoverssm_last_error(), field


def test_plan_outputs_must_not_overlap_its_inputs():
    """A plan whose output arrays share memory with the metadata it reads
    (or with each other) is refused before any launch: in the fused plan +
    fold launch the writer workgroups would store into what the folding
    workgroups are still planning from."""
    lib = N.load()
    groups = N.PlanGroups()
    g0 = groups[0]
    g0.state_indices, g0.query_start_loc = 0x60000, 0x70000
    g0.si_dtype = g0.qsl_dtype = 3
    g0.si_stride = g0.qsl_stride = 1
    base = dict(sampled=0x50000, sampled_len=4, sampled_stride=1, sampled_dtype=3, num_groups=1,
                groups=ctypes.cast(groups, ctypes.POINTER(N.PlanGroup)), lens_plan=0x10000, final_plan=0x20000,
                boundary_plan=0x30000, boundary_lens_plan=0x40000, num_rows=4, plan_capacity=4, spec_query_len=4)
    fcfg = N.i64_array([4, 1, 4, 2, 4, 16, 4, 8, 0, 128 * 128, 128, 512, 128, 256, 128, 4, 1])
    fext = N.FoldExt(key_dim=128, value_dim=128, state_k_stride=1)

    def call(**over):
        launch = N.PlanLaunch(**dict(base, **over))
        return lib.gdn_recoverssm_plan_fold(ctypes.byref(launch), None, None, None, None, *([8] * 8), None, fcfg, 17,
                                            ctypes.byref(fext), None)

    # the final pages written over the state indices the rows are planned from
    assert call(final_plan=0x60000) == N.GDN_ERR_INVALID
    assert b"overlaps the state indices" in lib.gdn_recoverssm_last_error()
    # lengths written over the accepted counts, one element in
    assert call(lens_plan=0x50000 + 12) == N.GDN_ERR_INVALID
    assert b"overlaps the accepted counts" in lib.gdn_recoverssm_last_error()
    # two outputs sharing memory
    assert call(boundary_plan=0x20000 + 8) == N.GDN_ERR_INVALID
    assert b"two plan outputs" in lib.gdn_recoverssm_last_error()
    # adjacent but disjoint ranges pass this check (and fail the next one)
    assert call(lens_plan=0x50000 + 16) == N.GDN_ERR_INVALID
    assert b"differ from the plan" in lib.gdn_recoverssm_last_error()
    # the same through the separate plan entry
    st = lib.gdn_recoverssm_plan(0x50000, 3, 1, 4, groups, 1, None, 0x70000 + 4, 0x20000, 0x30000, 0x40000, None,
                                 None, None, 3, 0, None, None, 0, 4, 4, 0, 4, 0, None)
    assert st == N.GDN_ERR_INVALID and b"overlaps the query offsets" in lib.gdn_recoverssm_last_error()


def test_fold_row_list_is_checked_before_launch():
    """A fold row list (gdn_fold_ext.row_list) needs 1..rows entries, and only
    gdn_recoverssm_fold takes one: the fused plan + fold and the no-allocation
    commit refuse it. Every call here is rejected before a launch (the device
    addresses are never dereferenced)."""
    lib = N.load()
    fcfg = N.i64_array([4, 1, 4, 2, 4, 16, 4, 8, 0, 128 * 128, 128, 512, 128, 256, 128, 4, 1])
    tables = [8] * 8
    plan = [0x10000, 0x20000, 0x30000, 0x40000, 0x50000]  # source and the four plan arrays
    for n in (0, -1, 5):
        fext = N.FoldExt(key_dim=128, value_dim=128, state_k_stride=1, source_dtype=3, source_stride=1,
                         row_list=0x60000, row_list_len=n)
        st = lib.gdn_recoverssm_fold(None, None, None, None, *tables, None, *plan, fcfg, 17, ctypes.byref(fext), None)
        assert st == N.GDN_ERR_INVALID and b"row list" in lib.gdn_recoverssm_last_error(), n
    fext = N.FoldExt(key_dim=128, value_dim=128, state_k_stride=1, row_list=0x60000, row_list_len=2)
    groups = N.PlanGroups()
    g0 = groups[0]
    g0.state_indices, g0.query_start_loc = 0x60000, 0x70000
    g0.si_dtype = g0.qsl_dtype = 3
    g0.si_stride = g0.qsl_stride = 1
    launch = N.PlanLaunch(sampled=0x50000, sampled_len=4, sampled_stride=1, sampled_dtype=3, num_groups=1,
                          groups=ctypes.cast(groups, ctypes.POINTER(N.PlanGroup)), lens_plan=0x10000,
                          final_plan=0x20000, boundary_plan=0x30000, boundary_lens_plan=0x40000, num_rows=4,
                          plan_capacity=8, spec_query_len=4)
    st = lib.gdn_recoverssm_plan_fold(ctypes.byref(launch), None, None, None, None, *tables, None, fcfg, 17,
                                      ctypes.byref(fext), None)
    assert st == N.GDN_ERR_INVALID and b"gdn_recoverssm_fold only" in lib.gdn_recoverssm_last_error()
    launch = N.PlanLaunch(sampled=8, sampled_len=4, sampled_dtype=3, num_groups=1,
                          groups=ctypes.cast(groups, ctypes.POINTER(N.PlanGroup)), num_rows=4, spec_query_len=4,
                          plan_capacity=8)
    st = lib.gdn_recoverssm_commit_noalloc(ctypes.byref(launch), None, None, None, None, *tables, None, fcfg, 17,
                                           ctypes.byref(fext), None, None)
    assert st == N.GDN_ERR_INVALID and b"gdn_recoverssm_fold only" in lib.gdn_recoverssm_last_error()


def test_settle_is_checked_before_launch():
    """gdn_recoverssm_settle refuses 0 or more than 3 groups, pending rows
    beyond the plan, a row map or index array that does not cover a group's
    next rows, a non-index dtype and outputs that share memory with an input
    or with each other, before any HIP call (the addresses are never
    dereferenced). A fold row count without a row list is refused too."""
    lib = N.load()
    L, F, R, X, O, RL, C = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000, 0x60000, 0x70000

    def call(groups=1, nexts=None, **kw):
        a = dict(lengths=L, finals=F, cap=8, num_rows=4, rows=R, rows_len=6, out=O, rl=RL, cnt=C)
        a.update(kw)
        table = (N.SettleNext * max(groups, 1))()
        for g, n in enumerate(nexts or [dict(state_indices=X, stride=1, rows=6, dtype=N.DT_I32)] * groups):
            for k, v in n.items():
                setattr(table[g], k, v)
        return lib.gdn_recoverssm_settle(a["lengths"], a["finals"], groups, a["cap"], a["num_rows"], a["rows"],
                                         a["rows_len"], table, a["out"], a["rl"], a["cnt"], None)

    good = dict(state_indices=X, stride=1, rows=6, dtype=N.DT_I32)
    for kw, msg in [
        (dict(groups=0), b"groups"),
        (dict(groups=4), b"groups"),
        (dict(num_rows=9), b"pending rows"),
        (dict(num_rows=-1), b"pending rows"),
        (dict(cap=N.SETTLE_MAX_ROWS + 8, num_rows=N.SETTLE_MAX_ROWS + 1), b"pending rows"),
        (dict(cap=0, num_rows=0), b"groups"),
        (dict(out=0), b"missing"),
        (dict(cnt=0), b"missing"),
        (dict(rows_len=5), b"cover"),
        (dict(rows=0), b"cover"),
        (dict(nexts=[dict(good, state_indices=0)]), b"cover"),
        (dict(nexts=[dict(good, dtype=N.DT_F32)]), b"cover"),
        (dict(nexts=[dict(good, stride=-1)]), b"cover"),
        (dict(nexts=[dict(good, rows=-1)]), b"cover"),
        (dict(groups=2, nexts=[good, dict(good, rows=7)]), b"group 1"),
        (dict(out=L + 16), b"output lengths overlaps the plan lengths"),
        (dict(groups=2, nexts=[good, good], out=F - 32), b"output lengths overlaps the final pages"),
        (dict(rl=R), b"row list overlaps the row map"),
        (dict(cnt=X + 8, nexts=[dict(good, dtype=N.DT_I64)]), b"row count overlaps the next state indices"),
        (dict(rl=O + 28), b"output lengths overlaps the row list"),
    ]:
        st = call(**kw)
        assert st == N.GDN_ERR_INVALID and msg in lib.gdn_recoverssm_last_error(), (kw, lib.gdn_recoverssm_last_error())
    fcfg = N.i64_array([4, 1, 4, 2, 4, 16, 4, 8, 0, 128 * 128, 128, 512, 128, 256, 128, 4, 1])
    fext = N.FoldExt(key_dim=128, value_dim=128, state_k_stride=1, source_dtype=3, source_stride=1, row_count=C)
    st = lib.gdn_recoverssm_fold(None, None, None, None, *([8] * 8), None, *[0x10000, 0x20000, 0x30000, 0x40000,
                                 0x50000], fcfg, 17, ctypes.byref(fext), None)
    assert st == N.GDN_ERR_INVALID and b"row count applies to a row list" in lib.gdn_recoverssm_last_error()


def test_commit_noalloc_rejects_before_touching_the_device():
    """The no-allocation commit refuses caller plan arrays and a plan larger
    than the library's buffer before any HIP call (none is possible here)."""
    lib = N.load()
    groups = N.PlanGroups()
    fext = N.FoldExt(key_dim=128, value_dim=128, state_k_stride=1)
    cfg = N.i64_array([4, 1, 4, 2, 4, 16, 4, 8, 0, 128 * 128, 128, 512, 128, 256, 128, 4, 1])

    def call(launch, conv=None):
        return lib.gdn_recoverssm_commit_noalloc(ctypes.byref(launch), None, None, None, None, *([8] * 8), None, cfg,
                                                 17, ctypes.byref(fext), conv, None)

    base = dict(sampled=8, sampled_len=4, sampled_dtype=3, num_groups=1,
                groups=ctypes.cast(groups, ctypes.POINTER(N.PlanGroup)), num_rows=4, spec_query_len=4)
    st = call(N.PlanLaunch(**base, plan_capacity=8, lens_plan=8))
    assert st == N.GDN_ERR_INVALID and b"pass NULL" in lib.gdn_recoverssm_last_error()
    st = call(N.PlanLaunch(**dict(base, num_groups=2), plan_capacity=N.NOALLOC_PLAN_ENTRIES // 2 + 1))
    assert st == N.GDN_ERR_INVALID and b"exceed" in lib.gdn_recoverssm_last_error()
    st = call(N.PlanLaunch(**base, plan_capacity=8), ctypes.byref(N.ConvLaunch(conv_dim=40, history=3, window=6,
                                                                              element_bytes=2)))
    assert st == N.GDN_ERR_INVALID and b"conv_compact" in lib.gdn_recoverssm_last_error()


def test_verify_rejects_strides_beyond_32_bits():
    """The kernel takes its element strides in 32 bits: a larger one is
    refused on the host, before any HIP call."""
    lib = N.load()
    ext = N.VerifyExt(key_dim=128, value_dim=128, act_dtype=1, beta_dtype=0, g_dtype=0, state_dtype=0,
                      key_record_dtype=1, qsl_dtype=3, index_dtype=3, out_dtype=1)
    base = [1, 4, 1, 2, 4, 8, 1, 0, 256, 256, 256, 2, 2, 2 * 128 * 128, 128 * 128, 128, 2 * 4 * 128, 4 * 128, 128,
            4 * 128, 4 * 128, 128, 2 * 4, 4, 1, 256, 1, 1]
    for field in (8, 13, 16, 26):
        cfg = list(base)
        cfg[field] = 1 << 31
        st = lib.gdn_recoverssm_verify(*([None] * 12), N.i64_array(cfg), 28, 1.0, ctypes.byref(ext), None)
        assert st == N.GDN_ERR_UNSUPPORTED, field
        assert f"config field {field}".encode() in lib.gdn_recoverssm_last_error(), lib.gdn_recoverssm_last_error()


def test_zero_rows_is_a_noop_without_touching_the_device():
    lib = N.load()
    ext = N.VerifyExt(key_dim=128, value_dim=128, act_dtype=1, out_dtype=1, state_dtype=0, key_record_dtype=1,
                      qsl_dtype=3, index_dtype=3)
    cfg = N.i64_array([0, 0, 1, 2, 4, 8, 1, 0] + [0] * 20)
    assert lib.gdn_recoverssm_verify(*([None] * 12), cfg, 28, 1.0, ctypes.byref(ext), None) == N.GDN_OK


_LAYOUT_PROBE = r"""
#include <stddef.h>
#include <stdio.h>
#include "gdn_recoverssm_hip.h"
#define F(T, f) printf("%s.%s %zu\n", #T, #f, offsetof(T, f));
int main(void) {
  printf("gdn_verify_ext %zu\n", sizeof(gdn_verify_ext));
  F(gdn_verify_ext, state_cache_retain)
  printf("gdn_fold_ext %zu\n", sizeof(gdn_fold_ext));
  printf("gdn_plan_group %zu\n", sizeof(gdn_plan_group));
  printf("gdn_gating_ext %zu\n", sizeof(gdn_gating_ext));
  printf("gdn_pending_commit %zu\n", sizeof(gdn_pending_commit));
  printf("gdn_plan_launch %zu\n", sizeof(gdn_plan_launch));
  printf("gdn_conv_launch %zu\n", sizeof(gdn_conv_launch));
  printf("noalloc_entries %d\n", GDN_NOALLOC_PLAN_ENTRIES);
  F(gdn_conv_launch, conv_token_strides) F(gdn_conv_launch, conv_dim) F(gdn_conv_launch, window)
  F(gdn_conv_launch, element_bytes)
  F(gdn_plan_launch, groups) F(gdn_plan_launch, col_plan) F(gdn_plan_launch, idx_mapping_dtype)
  F(gdn_plan_launch, flags) F(gdn_plan_launch, persistent_len) F(gdn_plan_launch, spec_query_len)
  F(gdn_pending_commit, record_rows) F(gdn_pending_commit, decay_strides) F(gdn_pending_commit, key_per_value_head)
  F(gdn_pending_commit, num_rows)
  F(gdn_gating_ext, softplus_beta) F(gdn_gating_ext, softplus_threshold)
  F(gdn_verify_ext, out_dtype) F(gdn_verify_ext, key_per_value_head)
  F(gdn_fold_ext, source_stride) F(gdn_fold_ext, state_k_stride) F(gdn_fold_ext, row_list)
  F(gdn_fold_ext, row_list_len) F(gdn_fold_ext, row_count)
  printf("gdn_settle_next %zu\n", sizeof(gdn_settle_next));
  F(gdn_settle_next, stride) F(gdn_settle_next, rows) F(gdn_settle_next, dtype)
  F(gdn_plan_group, block_table) F(gdn_plan_group, table_rows) F(gdn_plan_group, num_computed)
  F(gdn_plan_group, computed_dtype) F(gdn_plan_group, num_blocks) F(gdn_plan_group, block_size)
  return 0;
}
"""


def test_ctypes_struct_layout_matches_c_compiler():
    with tempfile.TemporaryDirectory() as tmp:
        src = os.path.join(tmp, "probe.c")
        exe = os.path.join(tmp, "probe")
        open(src, "w").write(_LAYOUT_PROBE)
        subprocess.run(["gcc", "-I", INCLUDE_DIR, src, "-o", exe], check=True)
        lines = subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split("\n")
    got = dict(line.rsplit(" ", 1) for line in lines if line)
    assert int(got["gdn_verify_ext"]) == ctypes.sizeof(N.VerifyExt)
    assert int(got["gdn_fold_ext"]) == ctypes.sizeof(N.FoldExt)
    assert int(got["gdn_plan_group"]) == ctypes.sizeof(N.PlanGroup)
    assert int(got["gdn_gating_ext"]) == ctypes.sizeof(N.GatingExt)
    assert int(got["gdn_pending_commit"]) == ctypes.sizeof(N.PendingCommit)
    assert int(got["gdn_plan_launch"]) == ctypes.sizeof(N.PlanLaunch)
    assert int(got["gdn_conv_launch"]) == ctypes.sizeof(N.ConvLaunch)
    assert int(got["gdn_settle_next"]) == ctypes.sizeof(N.SettleNext)
    assert int(got.pop("noalloc_entries")) == N.NOALLOC_PLAN_ENTRIES
    for key, value in got.items():
        if "." not in key:
            continue
        struct, fld = key.split(".")
        cls = {"gdn_verify_ext": N.VerifyExt, "gdn_fold_ext": N.FoldExt, "gdn_plan_group": N.PlanGroup,
               "gdn_gating_ext": N.GatingExt, "gdn_pending_commit": N.PendingCommit,
               "gdn_plan_launch": N.PlanLaunch, "gdn_conv_launch": N.ConvLaunch,
               "gdn_settle_next": N.SettleNext}[struct]
        assert getattr(cls, fld).offset == int(value), key


def test_config_field_counts_match_reference_abi():
    # csrc/common.h of the reference: 28 verify fields (+ scale), 17 fold fields
    text = open(HEADER).read()
    assert "#define GDN_VERIFY_CONFIG_FIELDS 28" in text and N.VERIFY_CONFIG_FIELDS == 28
    assert "#define GDN_FOLD_CONFIG_FIELDS 17" in text and N.FOLD_CONFIG_FIELDS == 17


def test_native_caller_is_built_against_this_header():
    """The native C-ABI caller the GPU tests run (tests/capi/capi_step) starts
    and rejects a missing argument before any HIP call."""
    import os
    import subprocess

    exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "capi", "capi_step")
    if not os.path.exists(exe):
        pytest.skip("tests/capi/capi_step is built by __graft_entry__.build()")
    r = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=60)
    assert r.returncode == 2 and b"usage" in r.stdout


def test_stale_library_is_refused(tmp_path):
    """A library whose recorded source digest differs from the kernel sources
    beside the package is refused at load, as is the in-tree library without
    a recorded digest; the in-tree build carries the current digest. Run in a
    child process, since the library loads once per process."""
    import shutil

    from gdn_recoverssm_ascend import _build

    assert _build.built_digest(LIB_PATH) == _build.source_digest(), "rebuild: the in-tree library is stale"
    stale = tmp_path / "libstale.so"
    shutil.copy(LIB_PATH, stale)
    (tmp_path / "libstale.so.digest").write_text("0" * 40 + "\n")
    code = (
        "from gdn_recoverssm_ascend import _native\n"
        "try:\n"
        "    _native.load()\n"
        "except RuntimeError as e:\n"
        "    assert 'other kernel sources' in str(e), str(e)\n"
        "else:\n"
        "    raise SystemExit('a stale library loaded')\n"
        "print('ok')\n"
    )
    pkg = os.path.dirname(os.path.dirname(N.__file__))
    env = dict(os.environ, GDN_RECOVERSSM_HIP_LIB=str(stale),
               PYTHONPATH=pkg + os.pathsep + os.environ.get("PYTHONPATH", ""))
    r = subprocess.run([sys.executable, "-c", code], env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       timeout=300)
    out = r.stdout.decode(errors="replace")
    assert r.returncode == 0 and out.strip().endswith("ok"), out


def test_missing_library_fails_loudly(tmp_path):
    """With the HIP library absent, the first call into the package raises
    RuntimeError naming the missing path: there is no CPU fallback to fall
    through to. Run in a child process, since the library loads once per
    process."""
    code = (
        "import torch\n"
        "from gdn_recoverssm_ascend import torch_ops, _native\n"
        "for call in (torch.ops.gdn_recoverssm_hip.abi_version, _native.load):\n"
        "    try:\n"
        "        call()\n"
        "    except RuntimeError as e:\n"
        "        assert 'not found' in str(e) and 'no fallback' in str(e), str(e)\n"
        "    else:\n"
        "        raise SystemExit('no error without the library')\n"
        "print('ok')\n"
    )
    pkg = os.path.dirname(os.path.dirname(N.__file__))
    env = dict(os.environ, GDN_RECOVERSSM_HIP_LIB=str(tmp_path / "absent.so"),
               PYTHONPATH=pkg + os.pathsep + os.environ.get("PYTHONPATH", ""))
    r = subprocess.run([sys.executable, "-c", code], env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       timeout=300)
    out = r.stdout.decode(errors="replace")
    assert r.returncode == 0 and out.strip().endswith("ok"), out

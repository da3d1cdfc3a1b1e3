#!/usr/bin/env python3
"""Verify + commit benchmark for one GDN layer on one MI355X.

One step = ``gdn_recoverssm_verify`` over the whole speculative batch, then the
commit of the accepted prefix (``GDNRecoverSSMCommitContext.commit``: plan +
fold in one launch; the same step followed by the conv compaction is reported
beside it) on the align-mode workload
``align_b256``: 256 sequences, 16 key / 32 value heads, K = V = 128, Q = 4, FP32
state pages, bf16 activations, block size 64 with ~25% of the rows crossing a
block boundary, accepted lengths uniform in {0..4}, 6 padded rows.

``value`` is the achieved HBM bandwidth of the step: algorithmic bytes (the
byte model below, computed from the seeded draws) divided by the measured step
time, with every input resident in HBM before the timed region starts.
Per-kernel durations come from HIP events on the stream the kernels run on.
The verify runs with the library's default cache hint (the last 256 MiB of a
batch's state read with ordinary loads, the rest non-temporally), so the
commit finds the pages it re-reads in the memory-side cache;
``disjoint_pools`` repeats the step on two batches with separate page pools
taking turns, which leaves only that within-step reuse. The line also carries
the other single-layer configurations, the deferred commit, the 48-layer
decode loop (its verifies retain 64 MiB per layer) and the traffic twins of
both kernels.

Algorithmic bytes (f32 state, bf16 activations / keys):
  verify = B_valid*HV*V*K*4 (state, once)  + T*(2*H*K + HV*V)*2 (q, k, v)
         + T*HV*8 (g, beta) + (2B+1)*4 (offsets, slots) + T*HV*V*2 (out)
         + T*HV*V*4 (corrections) + T*H*K*2 (keys) + T*HV*4 (decays)
         + T_null*HV*V*2 (zero outputs of padded rows)
  commit = sum over rows with n > 0 of HV*V*K*4*(2 + boundary written)
         + n*(HV*V*4 + H*K*2 + HV*4)  + 52*B (plan reads and writes)
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "gdn-recoverssm-ascend_amd"))

METRIC = "verify+commit HBM GB/s (% of peak) + µs/spec step, GDN layer B=256 Q=4"
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps before the timed ones (default: 200 for a single-layer step, whose "
                         "timed steps ran 2 us slower each after only 10; 10 for a decode loop, which carries "
                         "its state through them)")
    ap.add_argument("--workload", default="align_b256")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--deferred", action="store_true",
                    help="decode-loop workloads: fold each commit into the next step's verify")
    ap.add_argument("--groups", type=int, default=None,
                    help="decode-loop workloads: commit through the grouped coordinator, the layers in this many "
                         "cache groups")
    ap.add_argument("--loop-steps", type=int, default=None,
                    help="decode-loop workloads: speculative steps to time (default: the workload's own)")
    ap.add_argument("--kernel-only", action="store_true", help="time the step and its kernels only (no conv, gated, deferred or other-configuration lines)")
    ap.add_argument("--copy-calibration", type=int, default=0,
                    help="also run a device copy of this many MiB (PMC scale calibration)")
    return ap.parse_args()


class _HipTimer:
    """HIP events created with hipEventDisableSystemFence, recorded on the
    given stream (torch's Event API does not expose creation flags). Uses the
    HIP runtime torch already loaded."""

    DISABLE_SYSTEM_FENCE = 0x20000000

    def __init__(self, stream_handle):
        import ctypes

        path = None
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64.so" in line:
                    path = line.split()[-1]
                    break
        if path is None:
            raise RuntimeError("HIP runtime not loaded")
        self._ct = ctypes
        self._hip = ctypes.CDLL(path)
        self._stream = ctypes.c_void_p(stream_handle)
        self._events = []

    def event(self):
        ev = self._ct.c_void_p()
        if self._hip.hipEventCreateWithFlags(self._ct.byref(ev), self._ct.c_uint(self.DISABLE_SYSTEM_FENCE)) != 0:
            raise RuntimeError("hipEventCreateWithFlags failed")
        self._events.append(ev)
        return ev

    def record(self, ev):
        if self._hip.hipEventRecord(ev, self._stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def elapsed(self, a, b):
        ms = self._ct.c_float()
        if self._hip.hipEventElapsedTime(self._ct.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def __del__(self):
        for ev in getattr(self, "_events", []):
            self._hip.hipEventDestroy(ev)


def byte_model(w, plan_lens, plan_final, plan_boundary, plan_blen):
    import torch

    s = w.spec
    B, HV, H, K, V = s.rows, s.value_heads, s.key_heads, s.key_dim, s.value_dim
    qsl = w.meta.query_start_loc.cpu().long()
    qlen = (qsl[1:] - qsl[:-1]).clamp(min=0, max=s.window)
    idx = w.meta.state_indices.cpu().long()
    valid = (idx > 0) & (idx < w.num_pages)
    T = int(qlen[valid].sum())
    T_null = int(qlen[~valid].sum())
    verify = (
        int(valid.sum()) * HV * V * K * 4
        + T * (2 * H * K + HV * V) * 2
        + T * HV * 8
        + (2 * B + 1) * 4
        + T * HV * V * 2
        + T * HV * V * 4
        + T * H * K * 2
        + T * HV * 4
        + T_null * HV * V * 2
    )
    n = plan_lens.cpu().long()[:B]
    fin = plan_final.cpu().long()[:B]
    bnd = plan_boundary.cpu().long()[:B]
    blen = plan_blen.cpu().long()[:B]
    active = n > 0
    store_b = active & (bnd > 0) & (bnd < w.num_pages) & (bnd != fin) & (blen > 0) & (blen <= n)
    state_pages = int(active.sum()) * 2 + int(store_b.sum())
    commit = state_pages * HV * V * K * 4 + int(n[active].sum()) * (HV * V * 4 + H * K * 2 + HV * 4) + 52 * B
    return dict(verify=verify, commit=commit, tokens=T, active_rows=int(active.sum()),
                boundary_writes=int(store_b.sum()), accepted_tokens=int(n[active].sum()))


def measured_traffic(workload, kernel):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 PMC
    summary (FETCH_SIZE and WRITE_SIZE, scaled by the copy-kernel calibration
    recorded with them), or None when no summary matches this workload and
    these kernel sources."""
    from gdn_recoverssm_ascend import _build

    path = os.path.join(HERE, "profiles", f"pmc_traffic_{workload}.json")
    if not os.path.exists(path):
        return None, f"no PMC summary for {workload}"
    with open(path) as f:
        prof = json.load(f)
    if prof.get("sources_sha1") != _build.source_digest():
        return None, f"{os.path.relpath(path, HERE)} was taken of other kernel sources"
    k = prof.get("kernels", {}).get(kernel)
    if not k:
        return None, f"{os.path.relpath(path, HERE)} has no {kernel} entry"
    return k["hbm_bytes"], os.path.relpath(path, HERE)


def _probe_lib():
    import ctypes

    from gdn_recoverssm_ascend import _build

    if not os.path.exists(_build.PROBE_LIB_PATH):
        return None
    lib = ctypes.CDLL(_build.PROBE_LIB_PATH)
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.gdn_probe_verify_twin.argtypes = [vp, vp, i64, vp, i64, vp, i64, vp, i64, vp]
    lib.gdn_probe_fold_twin.argtypes = [vp, vp, vp, vp, vp, i64, vp]
    return lib


def _verify_twin(lib, w, layer, nbytes, retain):
    """The verify twin of one layer's launch: its state tiles (the rows before
    the last ``retain`` bytes non-temporally in row runs, the rest in the
    operand layout, as the verify reads them), its small reads and its output
    and record writes. Returns (launch, launch without the small traffic,
    bytes moved, tiles)."""
    import torch

    s = w.spec
    B, HV, H, K, V = s.rows, s.value_heads, s.key_heads, s.key_dim, s.value_dim
    ck = w.checkpoints[layer]
    dev = ck.device
    tile = V * K * 4
    page_b, head_b = ck.stride(0) * 4, ck.stride(1) * 4
    idx = w.meta.state_indices.cpu().long()
    valid = (idx > 0) & (idx < w.num_pages)
    hv = torch.arange(HV)
    tiles = (idx[valid][:, None] * page_b + hv[None, :] * head_b).reshape(-1).to(dev)
    n_v = tiles.numel()
    keep_rows = -(-retain // (HV * V * K * 4))
    nt_rows = max(0, B - keep_rows)
    nt_tiles = int(valid[:nt_rows].sum()) * HV
    T = nbytes["tokens"]
    writes = T * HV * V * (2 + 4) + T * H * K * 2 + T * HV * 4
    small = nbytes["verify"] - n_v * tile - writes
    small_dw = max(0, small // 4 // max(1, (n_v + 1) // 2))  # read once per wave pair (q, k shared)
    write_dw = writes // 4 // n_v
    small_buf = torch.zeros(((n_v + 1) // 2) * small_dw + 1, dtype=torch.float32, device=dev)
    wbuf = torch.empty(n_v * write_dw + 1, dtype=torch.float32, device=dev)
    sink = torch.empty(n_v, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def run(sdw=small_dw, wdw=write_dw):
        st = lib.gdn_probe_verify_twin(ck.data_ptr(), tiles.data_ptr(), n_v, small_buf.data_ptr(), sdw,
                                       wbuf.data_ptr(), wdw, sink.data_ptr(), nt_tiles, stream)
        assert st == 0, f"verify twin: status {st}"

    run.keep = (tiles, small_buf, wbuf, sink)
    v_bytes = n_v * tile + ((n_v + 1) // 2) * small_dw * 4 + n_v * write_dw * 4
    return run, (lambda: run(0, 0)), v_bytes, n_v


def traffic_ceiling(w, nbytes, plan, kernel_us, timer, steps, retain=None):
    """Synthetic twins of the step's two kernels (csrc/probe/traffic_probe.hip):
    the verify's state tiles, small reads and output / record writes, and the
    fold's tile copies (source page -> final and boundary pages, written into a
    scratch pool with the workload's page layout), moved in each kernel's own
    access pattern with no arithmetic, timed as a step (verify twin, then fold
    twin, an event between them) as the kernels are. The twin's time is what
    the memory system sustains for that traffic; kernel_over_twin is the
    kernel's time over it."""
    import torch

    lib = _probe_lib()
    if lib is None:
        return {"note": "the traffic probe library is not built"}
    s = w.spec
    B, HV, K, V = s.rows, s.value_heads, s.key_dim, s.value_dim
    if (K, V) != (128, 128) or w.checkpoints[0].dtype != torch.float32:
        return {"note": "the twins model 64 KiB FP32 tiles (K = V = 128)"}
    dev = w.checkpoints[0].device
    ck = w.checkpoints[0]
    tile = V * K * 4
    page_b, head_b = ck.stride(0) * 4, ck.stride(1) * 4
    hv = torch.arange(HV)
    vtwin, vtwin_reads, v_bytes, n_v = _verify_twin(lib, w, 0, nbytes, STEP_STATE_RETAIN if retain is None else retain)
    n, fin, bnd, blen = (t.cpu().long()[:B] for t in plan)
    src = w.meta.state_indices.cpu().long()
    act = n > 0
    store_b = act & (bnd > 0) & (bnd < w.num_pages) & (bnd != fin) & (blen > 0) & (blen <= n)
    so = (src[act][:, None] * page_b + hv[None, :] * head_b).reshape(-1)
    do = (fin[act][:, None] * page_b + hv[None, :] * head_b).reshape(-1)
    d2 = torch.where(store_b[act][:, None], bnd[act][:, None] * page_b + hv[None, :] * head_b,
                     torch.full((1, HV), -1, dtype=torch.long)).reshape(-1)
    so, do, d2 = so.to(dev), do.to(dev), d2.to(dev)
    n_f = so.numel()
    pool = torch.empty_like(ck)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def ftwin():
        st = lib.gdn_probe_fold_twin(ck.data_ptr(), pool.data_ptr(), so.data_ptr(), do.data_ptr(), d2.data_ptr(),
                                     n_f, stream)
        assert st == 0, f"fold twin: status {st}"

    for _ in range(10):
        vtwin()
        ftwin()
    marks = [[timer.event() for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    for ev in marks:
        timer.record(ev[0])
        vtwin()
        timer.record(ev[1])
        ftwin()
        timer.record(ev[2])
    torch.cuda.synchronize()
    v_us = sum(timer.elapsed(ev[0], ev[1]) for ev in marks) / steps * 1e3
    f_us = sum(timer.elapsed(ev[1], ev[2]) for ev in marks) / steps * 1e3
    r0, r1 = timer.event(), timer.event()
    for _ in range(3):
        vtwin_reads()
    torch.cuda.synchronize()
    timer.record(r0)
    for _ in range(steps):
        vtwin_reads()
    timer.record(r1)
    torch.cuda.synchronize()
    ro_us = timer.elapsed(r0, r1) / steps * 1e3
    f_bytes = n_f * tile * 2 + int(d2.ge(0).sum()) * tile
    torch.cuda.synchronize()
    del pool, vtwin
    torch.cuda.empty_cache()
    return {
        "verify_twin": {"us": round(v_us, 2), "bytes": v_bytes, "gbs": round(v_bytes / (v_us * 1e-6) / 1e9, 1),
                        "reads_only_us": round(ro_us, 2),
                        "reads_only_gbs": round(n_v * tile / (ro_us * 1e-6) / 1e9, 1),
                        "kernel_us": round(kernel_us["verify"], 2),
                        "kernel_over_twin": round(kernel_us["verify"] / v_us, 3)},
        "fold_twin": {"us": round(f_us, 2), "bytes": f_bytes, "gbs": round(f_bytes / (f_us * 1e-6) / 1e9, 1),
                      "kernel_us": round(kernel_us["plan_fold"], 2),
                      "kernel_over_twin": round(kernel_us["plan_fold"] / f_us, 3)},
        "note": "synthetic kernels moving the step's bytes in each kernel's access pattern with no arithmetic "
                "(verify twin: the verify's state tiles, small reads and output / record writes; fold twin: the "
                "committed tiles copied to their final and boundary pages of a scratch pool), timed as a step; "
                "reads_only: the verify twin without its small reads and writes; the verify twin reads the tiles "
                "of the rows before the last retained bytes non-temporally in row runs, as the verify does",
    }


def loop_verify_ceiling(timer, reps=10, layers=6):
    """The decode loop's verify against its twin, both as the loop runs them:
    one launch per layer, back to back over `layers` layers of the loop's
    workload (B=128, each layer's own page pool), the loop's cache hint. The
    twin of each layer moves that launch's bytes in the verify's access
    pattern with no arithmetic."""
    import torch

    from gdn_recoverssm_ascend import workloads as W
    from gdn_recoverssm_ascend.kernels import ReplayRecordBuffers, gdn_recoverssm_verify

    lib = _probe_lib()
    if lib is None:
        return {"note": "the traffic probe library is not built"}
    dev = torch.device("cuda:0")
    w = W.make_workload("decode_loop_l48", layers=layers, gen_device="cuda").to(dev)
    s, m = w.spec, w.meta
    B, Q, H, HV, K, V = s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
    recs = [ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=w.inputs[0].k.dtype)
            for _ in range(layers)]
    specs = []
    for layer in range(layers):
        inp = w.inputs[layer]
        gdn_recoverssm_verify(inp.g, inp.beta, inp.q, inp.k, inp.v, checkpoint_state=w.checkpoints[layer],
                              replay_cache=recs[layer], query_start_loc=m.query_start_loc,
                              state_indices=m.state_indices, spec_query_len=Q, state_cache_retain=LOOP_STATE_RETAIN,
                              _collect=specs)
    nb = byte_model(w, torch.zeros(B, dtype=torch.int32), m.state_indices, m.state_indices,
                    torch.zeros(B, dtype=torch.int32))
    twins = [_verify_twin(lib, w, layer, nb, LOOP_STATE_RETAIN) for layer in range(layers)]

    def timed(fns):
        for _ in range(3):
            for f in fns:
                f()
        e0, e1 = timer.event(), timer.event()
        torch.cuda.synchronize()
        timer.record(e0)
        for _ in range(reps):
            for f in fns:
                f()
        timer.record(e1)
        torch.cuda.synchronize()
        return timer.elapsed(e0, e1) / (reps * len(fns)) * 1e3

    k_us = timed([sp.launch for sp in specs])
    t_us = timed([t[0] for t in twins])
    r_us = timed([t[1] for t in twins])
    vb = nb["verify"]
    del w, recs, specs, twins
    torch.cuda.empty_cache()
    return {"kernel_us": round(k_us, 2), "twin_us": round(t_us, 2), "reads_only_us": round(r_us, 2),
            "bytes": vb, "kernel_frac": round(vb / (k_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "twin_frac": round(vb / (t_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "kernel_over_twin": round(k_us / t_us, 3), "layers_back_to_back": layers,
            "note": "one B=128 layer's verify as the decode loop runs it (launches back to back over several "
                    "layers' pools, 64 MiB retained) against its traffic twin timed the same way"}


def kernel_times(specs, timer, steps):
    """Each launch's average duration in us over `steps` steps, from HIP events
    recorded between consecutive launches on the kernels' stream."""
    import torch

    marks = [[timer.event() for _ in range(len(specs) + 1)] for _ in range(steps)]
    torch.cuda.synchronize()
    for ev in marks:
        timer.record(ev[0])
        for j, sp in enumerate(specs):
            sp.launch()
            timer.record(ev[j + 1])
    torch.cuda.synchronize()
    return {sp.name: sum(timer.elapsed(ev[j], ev[j + 1]) for ev in marks) / steps * 1e3
            for j, sp in enumerate(specs)}


def other_configs(args, timer, skip):
    """The verify + commit step of the other single-layer configurations
    (B=64 from a 512-page pool; B=256 at Q=1; B=256 at Q=8 with geometric
    acceptance), each timed like the main region on its own synthetic batch."""
    import torch

    from gdn_recoverssm_ascend import workloads as W
    from gdn_recoverssm_ascend.kernels import GDNRecoverSSMCommitContext, ReplayRecordBuffers, gdn_recoverssm_verify

    dev = torch.device("cuda:0")
    res = {}
    for name in ("pool512_b64", "decode_q1_b256", "skewed_q8_b256"):
        if name == skip:
            continue
        w = W.make_workload(name, gen_device="cuda").to(dev)
        s = w.spec
        B, Q, H, HV, K, V = s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
        inp, m = w.inputs[0], w.meta
        align = m.block_table is not None
        rec = ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=inp.k.dtype)
        ctx = GDNRecoverSSMCommitContext.from_tensors(w.conv_states, w.checkpoints, [rec], spec_query_len=Q,
                                                      max_num_reqs=B)
        out = torch.empty(1, w.tokens, HV, V, dtype=inp.v.dtype, device=dev)
        specs: list = []
        gdn_recoverssm_verify(inp.g, inp.beta, inp.q, inp.k, inp.v, checkpoint_state=w.checkpoints[0],
                              replay_cache=rec, query_start_loc=m.query_start_loc, state_indices=m.state_indices,
                              spec_query_len=Q, out=out, state_cache_retain=STEP_STATE_RETAIN, _collect=specs)
        specs += list(ctx.make_commit_specs(m.accepted, m.state_indices, m.query_start_loc,
                                            block_table=m.block_table if align else None,
                                            num_computed_tokens=m.num_computed if align else None,
                                            mamba_block_size=m.block_size if align else None, commit_conv=False))
        for _ in range(args.warmup):
            for sp in specs:
                sp.launch()
        e0, e1 = timer.event(), timer.event()
        torch.cuda.synchronize()
        timer.record(e0)
        for _ in range(args.steps):
            for sp in specs:
                sp.launch()
        timer.record(e1)
        torch.cuda.synchronize()
        ms = timer.elapsed(e0, e1) / args.steps
        nb = byte_model(w, ctx.commit_lens, ctx.final_state_indices, ctx.boundary_state_indices,
                        ctx.boundary_recovery_lens)
        total = nb["verify"] + nb["commit"]
        kus = kernel_times(specs, timer, args.steps)
        plan4 = (ctx.commit_lens, ctx.final_state_indices, ctx.boundary_state_indices, ctx.boundary_recovery_lens)
        twin = traffic_ceiling(w, nb, plan4, kus, timer, args.steps)
        res[name] = {"rows": B, "window": Q, "us_per_step": round(ms * 1e3, 2), "bytes": total,
                     "gbs": round(total / (ms * 1e-3) / 1e9, 1),
                     "frac": round(total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "kernels_us": {k: round(v, 2) for k, v in kus.items()},
                     "twins_us": {k: twin[k]["us"] for k in ("verify_twin", "fold_twin") if k in twin},
                     "over_twin": {k: twin[k]["kernel_over_twin"] for k in ("verify_twin", "fold_twin") if k in twin}}
        del w, rec, ctx, out, specs
        torch.cuda.empty_cache()
    return res


def disjoint_pools(args, timer, name):
    """The step on two batches of the workload with separate page pools (seeds
    0 and 1) taking turns: no step finds the pages of the step before it in
    any cache, so the only reuse left is the step's own (the commit reading
    pages its verify has just read)."""
    import torch

    from gdn_recoverssm_ascend import workloads as W
    from gdn_recoverssm_ascend.kernels import GDNRecoverSSMCommitContext, ReplayRecordBuffers, gdn_recoverssm_verify

    dev = torch.device("cuda:0")
    keep, specs, total = [], [], 0
    for seed in (0, 1):
        w = W.make_workload(name, seed=seed, gen_device="cuda").to(dev)
        s, m, inp = w.spec, w.meta, w.inputs[0]
        B, Q, H, HV, K, V = s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
        align = m.block_table is not None
        rec = ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=inp.k.dtype)
        ctx = GDNRecoverSSMCommitContext.from_tensors(w.conv_states, w.checkpoints, [rec], spec_query_len=Q,
                                                      max_num_reqs=B)
        out = torch.empty(1, w.tokens, HV, V, dtype=inp.v.dtype, device=dev)
        sp: list = []
        gdn_recoverssm_verify(inp.g, inp.beta, inp.q, inp.k, inp.v, checkpoint_state=w.checkpoints[0], replay_cache=rec,
                              query_start_loc=m.query_start_loc, state_indices=m.state_indices, spec_query_len=Q,
                              out=out, state_cache_retain=STEP_STATE_RETAIN, _collect=sp)
        sp += list(ctx.make_commit_specs(m.accepted, m.state_indices, m.query_start_loc,
                                         block_table=m.block_table if align else None,
                                         num_computed_tokens=m.num_computed if align else None,
                                         mamba_block_size=m.block_size if align else None, commit_conv=False))
        specs.append(sp)
        keep.append((w, rec, ctx, out))

    def two_steps():
        for sp in specs[0] + specs[1]:
            sp.launch()

    for _ in range(max(1, args.warmup // 2)):
        two_steps()
    e0, e1 = timer.event(), timer.event()
    torch.cuda.synchronize()
    timer.record(e0)
    for _ in range(max(1, args.steps // 2)):
        two_steps()
    timer.record(e1)
    torch.cuda.synchronize()
    pairs = max(1, args.steps // 2)
    us = timer.elapsed(e0, e1) / (2 * pairs) * 1e3
    # The plan arrays hold each batch's plan now that its commits have run.
    for w, _, ctx, _ in keep:
        nb = byte_model(w, ctx.commit_lens, ctx.final_state_indices, ctx.boundary_state_indices,
                        ctx.boundary_recovery_lens)
        total += nb["verify"] + nb["commit"]
    bytes_per_step = total / 2
    del keep, specs
    torch.cuda.empty_cache()
    return {"us_per_step": round(us, 2), "bytes_per_step": int(bytes_per_step),
            "gbs": round(bytes_per_step / (us * 1e-6) / 1e9, 1),
            "frac": round(bytes_per_step / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "note": "the step on two batches with separate page pools taking turns (seeds 0 and 1): no step "
                    "finds the previous step's pages in a cache; only the step's own verify -> commit reuse is left"}


def cold_step(args, timer, name):
    """The step with nothing taken from a cache: two batches of the workload
    with separate page pools (seeds 0 and 1) take turns, and before each
    kernel a read sweep over a 512 MiB scratch buffer (twice the memory-side
    cache, outside the kernel events) evicts what the previous kernels left,
    so the commit finds none of its verify's pages cached. The verifies use
    the library's default cache hint. The step's time is the sum of its two
    kernels' event times."""
    import torch

    from gdn_recoverssm_ascend import workloads as W
    from gdn_recoverssm_ascend.kernels import GDNRecoverSSMCommitContext, ReplayRecordBuffers, gdn_recoverssm_verify

    dev = torch.device("cuda:0")
    keep, specs = [], []
    for seed in (0, 1):
        w = W.make_workload(name, seed=seed, gen_device="cuda").to(dev)
        s, m, inp = w.spec, w.meta, w.inputs[0]
        B, Q, H, HV, K, V = s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
        align = m.block_table is not None
        rec = ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=inp.k.dtype)
        ctx = GDNRecoverSSMCommitContext.from_tensors(w.conv_states, w.checkpoints, [rec], spec_query_len=Q,
                                                      max_num_reqs=B)
        out = torch.empty(1, w.tokens, HV, V, dtype=inp.v.dtype, device=dev)
        sp: list = []
        gdn_recoverssm_verify(inp.g, inp.beta, inp.q, inp.k, inp.v, checkpoint_state=w.checkpoints[0], replay_cache=rec,
                              query_start_loc=m.query_start_loc, state_indices=m.state_indices, spec_query_len=Q,
                              out=out, _collect=sp)
        sp += list(ctx.make_commit_specs(m.accepted, m.state_indices, m.query_start_loc,
                                         block_table=m.block_table if align else None,
                                         num_computed_tokens=m.num_computed if align else None,
                                         mamba_block_size=m.block_size if align else None, commit_conv=False))
        assert [x.name for x in sp] == ["verify", "plan_fold"]
        specs.append(sp)
        keep.append((w, rec, ctx, out))
    sweep = torch.ones(128 << 20, dtype=torch.float32, device=dev)  # 512 MiB, read by every sweep
    sink = torch.empty((), dtype=torch.float32, device=dev)

    def run(steps, marks=None):
        for i in range(steps):
            for j, sp in enumerate(specs[i % 2]):
                torch.sum(sweep, dim=0, out=sink)
                if marks:
                    timer.record(marks[i][2 * j])
                sp.launch()
                if marks:
                    timer.record(marks[i][2 * j + 1])

    steps = max(2, args.steps - args.steps % 2)
    run(max(2, min(args.warmup, 20)))
    marks = [[timer.event() for _ in range(4)] for _ in range(steps)]
    torch.cuda.synchronize()
    run(steps, marks)
    torch.cuda.synchronize()
    verify_us = sum(timer.elapsed(ev[0], ev[1]) for ev in marks) / steps * 1e3
    fold_us = sum(timer.elapsed(ev[2], ev[3]) for ev in marks) / steps * 1e3
    vb = cb = 0
    for w, _, ctx, _ in keep:
        nb = byte_model(w, ctx.commit_lens, ctx.final_state_indices, ctx.boundary_state_indices,
                        ctx.boundary_recovery_lens)
        vb += nb["verify"] / 2
        cb += nb["commit"] / 2
    del keep, specs, sweep
    torch.cuda.empty_cache()

    def rate(b, us):
        return {"us": round(us, 2), "bytes": int(b), "gbs": round(b / (us * 1e-6) / 1e9, 1),
                "frac": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}

    from gdn_recoverssm_ascend import set_state_cache_retain

    default_retain = set_state_cache_retain(0)
    set_state_cache_retain(default_retain)
    line = rate(vb + cb, verify_us + fold_us)
    line["us_per_step"] = line.pop("us")
    line["kernels"] = {"verify": rate(vb, verify_us), "plan_fold": rate(cb, fold_us)}
    line["state_cache_retain"] = default_retain
    line["note"] = ("two batches with separate page pools taking turns, a 512 MiB read sweep before every kernel "
                    "(outside the events): every byte comes from HBM; us_per_step is the two kernels' event "
                    "times; the verifies use the library's default cache hint")
    return line


def cpu_baseline(w_cpu, threads, budget_s=10.0):
    """FP32 torch oracle on the host cores: full verify + plan + fold steps of
    the workload, repeated until about ``budget_s`` seconds of CPU work (at
    least one step); returns (seconds per step, steps run)."""
    import torch

    sys.path.insert(0, os.path.join(HERE, "oracle"))
    import gdn_oracle as O

    torch.set_num_threads(threads)
    s = w_cpu.spec
    inp = w_cpu.inputs[0]
    m = w_cpu.meta
    steps = 0
    t0 = time.perf_counter()
    while steps == 0 or time.perf_counter() - t0 < budget_s:
        res = O.oracle_verify(inp.q, inp.k, inp.v, inp.g, inp.beta, w_cpu.checkpoints[0], m.query_start_loc,
                              m.state_indices, s.window, dtype=torch.float32)
        plan = O.oracle_plan_single(m.accepted, m.state_indices, m.query_start_loc, spec_query_len=s.window,
                                    num_blocks=w_cpu.num_pages, block_table=m.block_table,
                                    num_computed=m.num_computed, block_size=m.block_size)
        O.oracle_fold([w_cpu.checkpoints[0]], [res.correction], [res.key], [res.decay], source=m.state_indices,
                      lengths=plan["commit_lens"], final=plan["final"], boundary=plan["boundary"],
                      boundary_len=plan["boundary_len"], rows=s.rows, num_blocks=w_cpu.num_pages,
                      record_rows=s.rows, dtype=torch.float32)
        steps += 1
    return (time.perf_counter() - t0) / steps, steps


def commit_bytes(spec, n, fin, bnd, blen, num_pages):
    """Algorithmic bytes of one layer's fold for plan rows (n, final, boundary,
    boundary length); same model as ``byte_model``'s commit part."""
    HV, H, K, V = spec.value_heads, spec.key_heads, spec.key_dim, spec.value_dim
    active = n > 0
    store_b = active & (bnd > 0) & (bnd < num_pages) & (bnd != fin) & (blen > 0) & (blen <= n)
    pages = int(active.sum()) * 2 + int(store_b.sum())
    return pages * HV * V * K * 4 + int(n[active].sum()) * (HV * V * 4 + H * K * 2 + HV * 4)


def conv_bytes(spec, n, bnd, blen, num_pages, conv_dim, history, elem):
    """Conv-state compaction bytes of one layer: per committed row, `history`
    positions of every channel read and written to the final slot, and again
    to the boundary slot when one is written."""
    active = n > 0
    store_b = active & (bnd > 0) & (bnd < num_pages) & (blen >= 1)
    return (int(active.sum()) * 2 + int(store_b.sum()) * 2) * conv_dim * history * elem


# The single-layer step (one layer's verify, then its commit) re-reads the
# verify's pages right away: its verifies read the last 256 MiB of their batch
# (the MI355X memory-side cache) with ordinary loads, so the commit finds those
# pages cached, and the rest non-temporally. Passed with every single-layer
# verify below and named in the line's config; the library's own default is
# the decode loop's (LOOP_STATE_RETAIN).
STEP_STATE_RETAIN = 256 << 20

# Cache groups of the decode loop committed through the grouped coordinator:
# four groups of 12 layers, three to a bucket, so two buckets and the
# publication across them.
LOOP_GROUPS = 4

# The decode loop's commit comes after all 48 layers' verifies, so nothing
# re-reads a verify's pages from the memory-side cache; there the verify
# itself runs fastest with the last quarter of a B=128 layer's 256 MiB read
# ordinarily and the rest non-temporally (measured per loop step: every row
# non-temporal 6.71 ms, 32 MiB retained 6.57, 64 MiB 6.54-6.56, 96 MiB 6.60,
# 128 MiB 6.55-6.65, 256 MiB, the default, 6.71-6.76).
LOOP_STATE_RETAIN = 64 << 20


def run_decode_loop(name, *, deferred, steps=None, warmup=10, groups=None):
    """The decode loop; its verifies pass the loop's cache hint
    (``LOOP_STATE_RETAIN``, the library's default), reported in the line."""
    line = _run_decode_loop(name, deferred=deferred, steps=steps, warmup=warmup, groups=groups)
    line["state_cache_retain"] = LOOP_STATE_RETAIN
    return line


def _run_decode_loop(name, *, deferred, steps=None, warmup=10, groups=None):
    """The decode-loop workload: every layer's verify, then one commit (plan,
    conv compaction, fold) across all layers, per speculative step, with the
    state carried from step to step (C += n, the source page becomes the final
    page) and fresh accepted lengths each step. With ``deferred`` each step runs
    the verify that applies the previous step's fold, then plan + conv.

    ``groups=None`` commits through one ``GDNRecoverSSMCommitContext`` of all
    layers. ``groups=k`` commits through ``GroupedCommitCoordinator``, the
    commit the reference's commit proxy drives (layer_patch.py:108-149): the
    layers form k cache groups of equal size on the same rows and block table,
    three groups to a bucket, and an align step over several buckets ends with
    the publication across them; deferred, ``commit_deferred`` plans, compacts
    and publishes and the next verifies apply the folds (every committed row
    continues on its final page, so nothing needs a ``settle``; its cost is
    timed apart). Returns the loop's JSON line as a dict."""
    from types import SimpleNamespace

    import torch

    from gdn_recoverssm_ascend import workloads as W
    from gdn_recoverssm_ascend.grouped_commit import GroupedCommitCoordinator
    from gdn_recoverssm_ascend.kernels import (
        GDNRecoverSSMCommitContext,
        ReplayRecordBuffers,
        gdn_recoverssm_verify,
        gdn_recoverssm_verify_deferred,
    )

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    w = W.make_workload(name, gen_device="cuda").to(dev)
    s = w.spec
    L, B, Q, H, HV, K, V = s.layers, s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
    steps = s.steps if steps is None else steps
    m = w.meta
    sets = 2 if deferred else 1
    recs = [[ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=w.inputs[0].k.dtype)
             for _ in range(L)] for _ in range(sets)]
    state_idx = m.state_indices.clone()
    computed = m.num_computed.clone()
    accepted = torch.zeros(B, dtype=torch.int32, device=dev)
    gen = torch.Generator().manual_seed(7)
    acc_all = torch.stack([W.sample_accepted(s, B, gen) for _ in range(steps + warmup)]).to(dev)
    outs = [torch.empty(1, w.tokens, HV, V, dtype=w.inputs[0].v.dtype, device=dev) for _ in range(L)]
    commit_kw = dict(block_table=m.block_table, num_computed_tokens=computed, mamba_block_size=m.block_size,
                     commit_conv=True)
    coord = None
    if groups is None:
        ctxs = [GDNRecoverSSMCommitContext.from_tensors(w.conv_states, w.checkpoints, recs[i], spec_query_len=Q,
                                                        max_num_reqs=B) for i in range(sets)]
        cspecs, pendings = [], []
        for i in range(sets):
            specs_i: list = []
            if deferred:
                pendings.append(ctxs[i].commit_deferred(accepted, state_idx, m.query_start_loc, _collect=specs_i,
                                                        **commit_kw))
            else:
                specs_i = list(ctxs[i].make_commit_specs(accepted, state_idx, m.query_start_loc, **commit_kw))
            cspecs.append(specs_i)

        def plan_arrays(i):
            c = ctxs[i % sets]
            return (c.commit_lens, c.final_state_indices, c.boundary_state_indices, c.boundary_recovery_lens)
    else:
        if L % groups:
            raise ValueError(f"{L} layers do not split into {groups} equal cache groups")
        per = L // groups
        ctxs = [[GDNRecoverSSMCommitContext.from_tensors(w.conv_states[g * per:(g + 1) * per],
                                                         w.checkpoints[g * per:(g + 1) * per],
                                                         recs[i][g * per:(g + 1) * per], spec_query_len=Q,
                                                         max_num_reqs=B) for g in range(groups)] for i in range(sets)]
        payload = SimpleNamespace(state_indices=state_idx, query_start_loc=m.query_start_loc,
                                  request_indices=m.request_indices.to(dev), block_table=m.block_table,
                                  num_computed_tokens=computed, block_size=m.block_size,
                                  request_rows=tuple(range(B)), query_lens=tuple([Q] * B))
        metas = [[SimpleNamespace(recoverssm_commit=payload, recoverssm_builder=SimpleNamespace(),
                                  recoverssm_context=c) for c in ctxs[i]] for i in range(sets)]
        idx_mapping = m.idx_mapping.to(dev)
        pcols = torch.full((B,), -1, dtype=torch.int32, device=dev)
        pacc = torch.zeros(B, dtype=torch.int32, device=dev)
        coord = GroupedCommitCoordinator()
        deferred_step = []
        for i in range(sets):
            if deferred:
                deferred_step.append(coord.commit_deferred(metas[i], accepted, idx_mapping, pcols, pacc))
            else:
                coord.commit(metas[i], accepted, idx_mapping, pcols, pacc)
        buckets = list(coord._buckets.values()) + list(coord._previous.values())
        first_bucket = [next(b for b in buckets if b.contexts[0] is ctxs[i][0]) for i in range(sets)]
        pendings = [[p for g in range(groups) for p in deferred_step[i].pending(g)] for i in range(sets)] \
            if deferred else []

        def plan_arrays(i):
            b = first_bucket[i % sets]
            return (b.length, b.final, b.boundary, b.boundary_len)
    vspecs = []
    for i in range(sets):
        specs_i = []
        for layer in range(L):
            inp = w.inputs[layer]
            kw = dict(checkpoint_state=w.checkpoints[layer], replay_cache=recs[i][layer],
                      query_start_loc=m.query_start_loc, state_indices=state_idx, spec_query_len=Q, out=outs[layer],
                      _collect=specs_i)
            if deferred:
                gdn_recoverssm_verify_deferred(inp.g, inp.beta, inp.q, inp.k, inp.v,
                                               pending=pendings[1 - i][layer], **kw)
            else:
                gdn_recoverssm_verify(inp.g, inp.beta, inp.q, inp.k, inp.v, state_cache_retain=LOOP_STATE_RETAIN,
                                      **kw)
        vspecs.append(specs_i)
    hist_lens = torch.empty(steps, 4, B, dtype=torch.int32, device=dev)

    def plan_of(i):
        return tuple(t[:B] for t in plan_arrays(i))

    def commit(i):
        if coord is None:
            for sp in cspecs[i % sets]:
                sp.launch()
        elif deferred:
            coord.commit_deferred(metas[i % sets], accepted, idx_mapping, pcols, pacc)
        else:
            coord.commit(metas[i % sets], accepted, idx_mapping, pcols, pacc)

    def carry(i):
        # The scheduler's part: committed rows advance by n and continue on
        # their final page.
        lens_, fin_ = plan_of(i)[:2]
        computed.add_(lens_ if lens_.dtype == computed.dtype else lens_.to(computed.dtype))
        torch.where(lens_ > 0, fin_.to(state_idx.dtype), state_idx, out=state_idx)

    def carried_step(i):
        accepted.copy_(acc_all[i])
        for sp in vspecs[i % sets]:
            sp.launch()
        commit(i)
        carry(i)

    def restart():
        state_idx.copy_(start_idx)
        computed.copy_(start_c)
        # no pending commit for the first deferred verify
        for lengths in ([plan_arrays(i)[0] for i in range(sets)] if coord is None else [b.length for b in buckets]):
            lengths.zero_()

    stream = torch.cuda.current_stream(dev)
    timer = _HipTimer(stream.cuda_stream)
    start_idx, start_c = m.state_indices.clone(), m.num_computed.clone()

    # Each step's inputs from the scheduler (accepted lengths, state indices,
    # computed tokens) are prepared before the timed region: a first pass runs
    # the loop with the state carried on the device and records every step's
    # metadata; the timed passes replay those steps with launches bound to
    # them, so a timed step is the 48 verifies and the commit, nothing else.
    restart()
    meta_si, meta_c = [], []
    for i in range(steps):
        meta_si.append(state_idx.clone())
        meta_c.append(computed.clone())
        carried_step(i)
    end_si, end_c = state_idx.clone(), computed.clone()  # the metadata after the last step
    torch.cuda.synchronize()

    def bind_step(i):
        si, cc, acc = meta_si[i], meta_c[i], acc_all[i]
        vs: list = []
        for layer in range(L):
            inp = w.inputs[layer]
            kw = dict(checkpoint_state=w.checkpoints[layer], replay_cache=recs[i % sets][layer],
                      query_start_loc=m.query_start_loc, state_indices=si, spec_query_len=Q, out=outs[layer],
                      _collect=vs)
            if deferred:
                gdn_recoverssm_verify_deferred(inp.g, inp.beta, inp.q, inp.k, inp.v,
                                               pending=pendings[1 - i % sets][layer], **kw)
            else:
                gdn_recoverssm_verify(inp.g, inp.beta, inp.q, inp.k, inp.v, state_cache_retain=LOOP_STATE_RETAIN,
                                      **kw)
        ckw = dict(block_table=m.block_table, num_computed_tokens=cc, mamba_block_size=m.block_size,
                   commit_conv=True)
        if coord is None:
            cs: list = []
            if deferred:
                ctxs[i % sets].commit_deferred(acc, si, m.query_start_loc, _collect=cs, **ckw)
            else:
                cs = list(ctxs[i % sets].make_commit_specs(acc, si, m.query_start_loc, **ckw))

            def commit_step():
                for sp in cs:
                    sp.launch()
        else:
            pl = SimpleNamespace(**dict(vars(payload), state_indices=si, num_computed_tokens=cc))
            mt = [SimpleNamespace(recoverssm_commit=pl, recoverssm_builder=SimpleNamespace(), recoverssm_context=c)
                  for c in ctxs[i % sets]]

            def commit_step():
                if deferred:
                    coord.commit_deferred(mt, acc, idx_mapping, pcols, pacc)
                else:
                    coord.commit(mt, acc, idx_mapping, pcols, pacc)
        return vs, commit_step

    bound = [bind_step(i) for i in range(steps)]

    def step(i, record=None, marks=None):
        vs, commit_step = bound[i]
        if marks:
            timer.record(marks[0])
        for sp in vs:
            sp.launch()
        if marks:
            timer.record(marks[1])
        commit_step()
        if marks:
            timer.record(marks[2])
        if record is not None:
            for j, t in enumerate(plan_of(i)):
                hist_lens[record, j].copy_(t)

    restart()
    for i in range(warmup):
        step(i % steps)
    torch.cuda.synchronize()
    restart()
    t0, t1 = timer.event(), timer.event()
    torch.cuda.synchronize()
    timer.record(t0)
    for i in range(steps):
        step(i)
    timer.record(t1)
    torch.cuda.synchronize()
    total_ms = timer.elapsed(t0, t1)

    # Per-phase split over a second pass of the same steps (pending state
    # restarted); the plans are recorded for the byte count here, after each
    # step's last event, not in the timed pass.
    restart()
    ev = [(timer.event(), timer.event(), timer.event()) for _ in range(steps)]
    torch.cuda.synchronize()
    for i in range(steps):
        step(i, record=i, marks=ev[i])
    torch.cuda.synchronize()
    verify_ms = sum(timer.elapsed(a, b) for a, b, _ in ev) / steps
    commit_ms = sum(timer.elapsed(b, c) for _, b, c in ev) / steps
    settle_us = settle_left_us = flush_us = None
    if coord is not None and deferred:
        # Every row here continues on its final page, so no step needs a
        # settle; a serving loop whose batch changes calls it (or flush(rows))
        # before the verifies. Its cost with nothing to fold: per bucket the
        # settle kernel and a fold over the rows it lists (none here).
        # The next step's metadata (the last step's carried forward): every
        # pending row continues on its final page. The first call loads its
        # kernels; timed are the calls after it.
        state_idx.copy_(end_si)
        computed.copy_(end_c)
        deferred_step[1].settle(metas[0])
        s0, s1 = timer.event(), timer.event()
        torch.cuda.synchronize()
        timer.record(s0)
        for _ in range(5):
            deferred_step[1].settle(metas[0])
        timer.record(s1)
        torch.cuda.synchronize()
        settle_us = timer.elapsed(s0, s1) / 5 * 1e3
        # What a step whose batch lost two requests pays: a settle whose row
        # map gives those two rows' slots to new requests (it folds their
        # pending commits through the counted row list), and, instead, a
        # flush of two given rows. Both mark what they fold, so every call
        # takes two other committed rows (the first of each kind loads its
        # kernels; timed are the five after it); the row maps are built
        # before the timed calls.
        committed = [r for r, n in enumerate(deferred_step[1]._plan(0)[1][:B].tolist()) if n > 0]
        pairs = [committed[2 * k:2 * k + 2] for k in range(12)]
        maps = []
        for pair in pairs[:6]:
            mp = torch.arange(B, dtype=torch.int32)
            mp[pair] = -1
            maps.append(mp.to(dev))
        deferred_step[1].rows = maps[0]
        deferred_step[1].settle(metas[0])
        torch.cuda.synchronize()
        timer.record(s0)
        for mp in maps[1:]:
            deferred_step[1].rows = mp
            deferred_step[1].settle(metas[0])
        timer.record(s1)
        torch.cuda.synchronize()
        settle_left_us = timer.elapsed(s0, s1) / 5 * 1e3
        deferred_step[1].flush(rows=pairs[6])
        torch.cuda.synchronize()
        timer.record(s0)
        for pair in pairs[7:]:
            deferred_step[1].flush(rows=pair)
        timer.record(s1)
        torch.cuda.synchronize()
        flush_us = timer.elapsed(s0, s1) / 5 * 1e3
    lens, fin, bnd, blen = plan_of(0)

    nb = byte_model(w, lens, fin, bnd, blen)  # verify part is the same every step
    verify_b = nb["verify"] * L
    hl = hist_lens.cpu().long()
    conv_dim, conv_len = w.conv_states[0].shape[1:]
    hist = conv_len - Q + 1
    commit_b = conv_b = 0
    tokens_committed = 0
    for i in range(steps):
        n_, f_, b_, bl_ = hl[i]
        commit_b += commit_bytes(s, n_, f_, b_, bl_, w.num_pages) * L + 52 * B
        conv_b += conv_bytes(s, n_, b_, bl_, w.num_pages, conv_dim, hist, w.conv_states[0].element_size()) * L
        tokens_committed += int(n_[n_ > 0].sum())
    step_ms = total_ms / steps
    total_b = verify_b * steps + commit_b + conv_b
    gbs = total_b / (total_ms * 1e-3) / 1e9
    mode = "deferred commit (fold applied by the next verify)" if deferred else "verify then commit"
    line = {
        "metric": f"decode loop: {L} GDN layers verify + one grouped commit per step, B={B} Q={Q}, state carried"
                  + (", deferred commit" if deferred else ""),
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(step_ms, 4),
        "us_per_step": round(step_ms * 1e3, 1),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": s.name, "layers": L, "rows": B, "key_heads": H, "value_heads": HV, "key_dim": K,
                   "value_dim": V, "window": Q, "mode": "align", "block_size": m.block_size, "pages_per_layer": w.num_pages,
                   "commit": "one context" if groups is None else f"coordinator, {groups} cache groups"},
        "phases_us_per_step": {"verify_all_layers": round(verify_ms * 1e3, 1), "commit": round(commit_ms * 1e3, 1)},
        "bytes_per_step": {"verify": verify_b, "commit": round(commit_b / steps), "conv": round(conv_b / steps)},
        "tokens_committed_per_step": round(tokens_committed / steps, 1),
        "mode": mode,
    }
    if coord is not None:
        line["launches_per_commit"] = coord.last_launch_count
    if settle_us is not None:
        line["settle_us"] = round(settle_us, 1)
        line["settle_two_left_us"] = round(settle_left_us, 1)
        line["flush_two_rows_us"] = round(flush_us, 1)
    if deferred:
        # The step's state reads that the deferred commit removes: one page read
        # per committed (row, layer).
        saved = sum(int((hist_lens[i, 0] > 0).sum()) for i in range(steps)) * L * HV * V * K * 4
        line["hbm_bytes_per_step"] = round((total_b - saved) / steps)
        line["hbm_gbs"] = round((total_b - saved) / (total_ms * 1e-3) / 1e9, 1)
        line["note"] = "value divides the ordinary flow's algorithmic bytes by this loop's time"
    del w, recs, ctxs, outs, vspecs, pendings
    coord = None
    torch.cuda.empty_cache()
    return line


def decode_loop(args):
    """--workload decode_loop_l48 [--deferred] [--groups k]: the loop's own JSON line."""
    line = run_decode_loop(args.workload, deferred=args.deferred, steps=args.loop_steps, warmup=args.warmup,
                           groups=args.groups)
    print(json.dumps(line), flush=True)
    return 0


def decode_loop_summary(warmup):
    """The decode-loop configuration (48 layers, B=128, Q=4, align, 64 carried
    steps) for the default bench line: per-step time, sustained bandwidth and
    the phase split, verify then commit and with the deferred commit."""
    keys = ("us_per_step", "value", "hbm_frac", "steps", "warmup", "phases_us_per_step", "bytes_per_step",
            "tokens_committed_per_step")
    res = {}
    for mode, deferred, groups in (("ordinary", False, None), ("deferred", True, None),
                                   ("coordinator_ordinary", False, LOOP_GROUPS),
                                   ("coordinator_deferred", True, LOOP_GROUPS)):
        line = run_decode_loop("decode_loop_l48", deferred=deferred, warmup=warmup, groups=groups)
        entry = {k: line[k] for k in keys}
        if groups is not None:
            entry["commit"] = line["config"]["commit"]
            entry["launches_per_commit"] = line["launches_per_commit"]
            if "settle_us" in line:
                entry["settle_us"] = line["settle_us"]
                entry["settle_two_left_us"] = line["settle_two_left_us"]
                entry["flush_two_rows_us"] = line["flush_two_rows_us"]
        entry["gbs"] = entry.pop("value")
        if deferred:
            entry["equivalent_gbs"] = entry.pop("gbs")
            entry["equivalent_frac"] = entry.pop("hbm_frac")
            entry["hbm_bytes_per_step"] = line["hbm_bytes_per_step"]
            entry["hbm_gbs"] = line["hbm_gbs"]
        res[mode] = entry
    import torch

    res["verify_ceiling"] = loop_verify_ceiling(_HipTimer(torch.cuda.current_stream().cuda_stream))
    res["config"] = run_decode_loop_config()
    res["state_cache_retain"] = LOOP_STATE_RETAIN
    res["note"] = ("gbs = algorithmic bytes of the whole loop (48 verifies, plan + fold, conv compaction per step) / "
                   "loop time; each step's scheduler inputs (accepted lengths, state indices, computed tokens) "
                   "are recorded by a first pass that carries the state and are in place before the timed "
                   "region; the deferred flow's equivalent_gbs divides the ordinary flow's bytes by its time; "
                   "the ordinary verifies retain the last state_cache_retain bytes of each layer's state "
                   "(the deferred verify reads every row non-temporally); coordinator_*: the same loop committed "
                   f"through GroupedCommitCoordinator with the layers in {LOOP_GROUPS} cache groups (two buckets "
                   "and the publication across them); no request leaves, so the deferred loop needs no settle "
                   "(settle_us: one settle with nothing to fold; settle_two_left_us: one settle after two "
                   "requests left, folding their commits across every layer through the counted row list; "
                   "flush_two_rows_us: the same two rows' commits folded by a flush through the fold's row "
                   "list instead)")
    return res


def run_decode_loop_config():
    from gdn_recoverssm_ascend import workloads as W

    s = W.get_spec("decode_loop_l48")
    return {"workload": s.name, "layers": s.layers, "rows": s.rows, "key_heads": s.key_heads,
            "value_heads": s.value_heads, "key_dim": s.key_dim, "value_dim": s.value_dim, "window": s.window,
            "mode": "align", "block_size": s.block_size, "steps": s.steps}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the verify/commit path shards by rows and heads with no exchange step)", file=sys.stderr)
        return 2
    sys.path.insert(0, os.path.join(HERE, "gdn-recoverssm-ascend_amd"))
    from gdn_recoverssm_ascend import workloads as W

    if W.get_spec(args.workload).layers > 1:
        if args.warmup is None:
            args.warmup = 10
        return decode_loop(args)
    if args.warmup is None:
        args.warmup = 200
    import torch

    from gdn_recoverssm_ascend import workloads as W
    from gdn_recoverssm_ascend.kernels import GDNRecoverSSMCommitContext, ReplayRecordBuffers, gdn_recoverssm_verify

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    want_cpu = not args.no_cpu_baseline
    w_cpu = W.make_workload(args.workload) if want_cpu else None
    w = w_cpu.to(dev) if want_cpu else W.make_workload(args.workload, gen_device="cuda").to(dev)
    s = w.spec
    B, Q, H, HV, K, V = s.rows, s.window, s.key_heads, s.value_heads, s.key_dim, s.value_dim
    inp = w.inputs[0]
    rec = ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=inp.k.dtype)
    ctx = GDNRecoverSSMCommitContext.from_tensors(w.conv_states, w.checkpoints, [rec], spec_query_len=Q, max_num_reqs=B)
    out = torch.empty(1, w.tokens, HV, V, dtype=inp.v.dtype, device=dev)
    m = w.meta
    align = m.block_table is not None
    verify_specs: list = []
    gdn_recoverssm_verify(inp.g, inp.beta, inp.q, inp.k, inp.v, checkpoint_state=w.checkpoints[0], replay_cache=rec,
                          query_start_loc=m.query_start_loc, state_indices=m.state_indices, spec_query_len=Q, out=out,
                          state_cache_retain=STEP_STATE_RETAIN, _collect=verify_specs)
    align_kw = dict(block_table=m.block_table if align else None,
                    num_computed_tokens=m.num_computed if align else None,
                    mamba_block_size=m.block_size if align else None)
    # The step's commit: plan + fold in one launch (the conv compaction is
    # outside the step's byte model and is measured after it further down).
    commit_specs = ctx.make_commit_specs(m.accepted, m.state_indices, m.query_start_loc, commit_conv=False, **align_kw)
    by_name = {sp.name: sp for sp in commit_specs}
    step_specs = verify_specs + [by_name["plan_fold"]]

    def step():
        for sp in step_specs:
            sp.launch()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    timer = _HipTimer(stream.cuda_stream)

    # Timed region 1: K plain steps -> value and ms_per_step.
    t0, t1 = timer.event(), timer.event()
    torch.cuda.synchronize()
    timer.record(t0)
    for _ in range(args.steps):
        step()
    timer.record(t1)
    torch.cuda.synchronize()
    step_ms = timer.elapsed(t0, t1) / args.steps

    # Timed region 2: the same K steps with an event between consecutive
    # launches, on the stream the kernels run on -> per-kernel durations.
    # The events skip the system-scope fence, so they neither flush the
    # caches nor hold the next launch back.
    names = [sp.name for sp in step_specs]
    marks = [[timer.event() for _ in range(len(step_specs) + 1)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    for i in range(args.steps):
        ev = marks[i]
        timer.record(ev[0])
        for j, sp in enumerate(step_specs):
            sp.launch()
            timer.record(ev[j + 1])
    torch.cuda.synchronize()
    marked_step_ms = timer.elapsed(marks[0][0], marks[-1][-1]) / args.steps
    kernel_ms = {n: sum(timer.elapsed(ev[j], ev[j + 1]) for ev in marks) / args.steps for j, n in enumerate(names)}

    # The whole commit as the reference runs it also compacts the conv states:
    # the same K steps with the conv compaction launched after plan + fold
    # (it reads the plan that launch stores).
    full_ms = None
    if not args.kernel_only:
        full_specs = verify_specs + list(
            ctx.make_commit_specs(m.accepted, m.state_indices, m.query_start_loc, commit_conv=True, **align_kw))
        assert [sp.name for sp in full_specs[len(verify_specs):]] == ["plan_fold", "conv"]
        for _ in range(args.warmup):
            for sp in full_specs:
                sp.launch()
        f0, f1 = timer.event(), timer.event()
        torch.cuda.synchronize()
        timer.record(f0)
        for _ in range(args.steps):
            for sp in full_specs:
                sp.launch()
        timer.record(f1)
        torch.cuda.synchronize()
        full_ms = timer.elapsed(f0, f1) / args.steps

    # The gated verify (gating and q/k L2 norm fused in) against the plain one,
    # each over back-to-back launches on the same batch.
    fused = None
    if not args.kernel_only:
        from gdn_recoverssm_ascend.kernels import gdn_recoverssm_verify_gated

        gen = torch.Generator(device=dev).manual_seed(3)
        a_raw = torch.randn(w.tokens, HV, generator=gen, device=dev)
        b_raw = torch.randn(w.tokens, HV, generator=gen, device=dev)
        A_log = torch.randn(HV, generator=gen, device=dev)
        dt_bias = torch.randn(HV, generator=gen, device=dev)
        rec32 = ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=torch.float32)
        gated_specs: list = []
        gdn_recoverssm_verify_gated(a_raw, b_raw, inp.q, inp.k, inp.v, A_log=A_log, dt_bias=dt_bias,
                                    checkpoint_state=w.checkpoints[0], replay_cache=rec32,
                                    query_start_loc=m.query_start_loc, state_indices=m.state_indices,
                                    spec_query_len=Q, out=out, state_cache_retain=STEP_STATE_RETAIN, _collect=gated_specs)

        def alone(sp, reps=20):
            for _ in range(3):
                sp.launch()
            e0, e1 = timer.event(), timer.event()
            torch.cuda.synchronize()
            timer.record(e0)
            for _ in range(reps):
                sp.launch()
            timer.record(e1)
            torch.cuda.synchronize()
            return timer.elapsed(e0, e1) / reps

        T_ = w.tokens
        fused = {
            "verify_us": round(alone(verify_specs[0]) * 1e3, 2),
            "verify_gated_l2norm_us": round(alone(gated_specs[0]) * 1e3, 2),
            "producer_round_trip_bytes": T_ * HV * (4 + 4) * 2 + T_ * H * K * 2 * 2 * 2,
            "note": "gated verify reads raw a, b (fp32), q, k and writes FP32 key records; the producer "
                    "round trip counts g/beta written and re-read and q/k normalised, written and re-read",
        }

    nbytes = byte_model(w, ctx.commit_lens, ctx.final_state_indices, ctx.boundary_state_indices, ctx.boundary_recovery_lens)
    total = nbytes["verify"] + nbytes["commit"]

    # The deferred commit: each step runs the verify that also applies the
    # previous step's fold, then the plan (the fold is left to the next step).
    # Two record sets alternate; the same batch repeats, as in the main region.
    deferred = None
    if not args.kernel_only:
        from gdn_recoverssm_ascend.kernels import gdn_recoverssm_verify_deferred

        recs2 = [rec, ReplayRecordBuffers.allocate(B, HV, H, Q, V, K, device=dev, key_dtype=inp.k.dtype)]
        ctx2 = [ctx, GDNRecoverSSMCommitContext.from_tensors(w.conv_states, w.checkpoints, [recs2[1]],
                                                            spec_query_len=Q, max_num_reqs=B)]
        commit_kw = dict(block_table=m.block_table if align else None,
                         num_computed_tokens=m.num_computed if align else None,
                         mamba_block_size=m.block_size if align else None, commit_conv=False)
        pend = [None, None]
        dspecs = [[], []]
        for i in range(2):
            specs_i: list = []
            pend[i] = ctx2[i].commit_deferred(m.accepted, m.state_indices, m.query_start_loc, _collect=specs_i,
                                              **commit_kw)
            dspecs[i] = specs_i
        # Each step plans the same commit (source pages -> final pages); the
        # verify that applies it names each committed row's final page, as a
        # carried batch does, so every pending fold is applied.
        for sp in dspecs[0]:
            sp.launch()
        idx_next = torch.where(ctx2[0].commit_lens[:B] > 0, ctx2[0].final_state_indices[:B],
                               m.state_indices).contiguous()
        vdef = [[], []]
        for i in range(2):
            gdn_recoverssm_verify_deferred(inp.g, inp.beta, inp.q, inp.k, inp.v, checkpoint_state=w.checkpoints[0],
                                           replay_cache=recs2[i], pending=pend[1 - i][0],
                                           query_start_loc=m.query_start_loc, state_indices=idx_next,
                                           spec_query_len=Q, out=out, _collect=vdef[i])

        def dstep(i):
            vdef[i][0].launch()  # applies the fold planned in the other context
            for sp in dspecs[i]:
                sp.launch()

        for sp in dspecs[1]:
            sp.launch()  # a plan for the first deferred verify to apply
        for i in range(args.warmup):
            dstep(i % 2)
        torch.cuda.synchronize()
        d0, d1 = timer.event(), timer.event()
        timer.record(d0)
        for i in range(args.steps):
            dstep(i % 2)
        timer.record(d1)
        torch.cuda.synchronize()
        dms = timer.elapsed(d0, d1) / args.steps
        # HBM bytes of a deferred step: verify's, plus the fold's writes and
        # record reads; the fold's read of the state is the one removed.
        s_bytes = HV * V * K * 4
        fold_read_state = nbytes["active_rows"] * s_bytes
        actual = nbytes["verify"] + nbytes["commit"] - fold_read_state
        deferred = {
            "us_per_step": round(dms * 1e3, 2),
            "equivalent_gbs": round(total / (dms * 1e-3) / 1e9, 1),
            "equivalent_frac": round(total / (dms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "hbm_bytes_per_step": actual,
            "hbm_gbs": round(actual / (dms * 1e-3) / 1e9, 1),
            "note": "verify_deferred (applies the previous step's fold) + plan per step; equivalent_gbs divides the "
                    "ordinary step's algorithmic bytes by this step time",
        }
    gbs = total / (step_ms * 1e-3) / 1e9
    ceiling = None
    if not args.kernel_only:
        plan4 = (ctx.commit_lens, ctx.final_state_indices, ctx.boundary_state_indices, ctx.boundary_recovery_lens)
        ceiling = traffic_ceiling(w, nbytes, plan4, {k: v * 1e3 for k, v in kernel_ms.items()}, timer, args.steps)
    others = None if args.kernel_only else other_configs(args, timer, s.name)
    pools = None if args.kernel_only else disjoint_pools(args, timer, s.name)
    cold = None if args.kernel_only else cold_step(args, timer, s.name)
    # The 48-layer decode loop at its own size (its own 10 warmup steps, after
    # which the carried state restarts from the seeded start).
    loop = None if args.kernel_only else decode_loop_summary(warmup=10)

    # The same step with packed FP32 records, one [corr(V) | key(K) | decay]
    # row per (row, value head, token) (kernels.py:687-697), instead of the
    # typed planes with bf16 keys shared by a key head's value heads.
    packed = None
    if not args.kernel_only:
        prec = torch.zeros(B, HV, Q, V + K + 1, dtype=torch.float32, device=dev)
        pctx = GDNRecoverSSMCommitContext.from_tensors(w.conv_states, w.checkpoints, [prec], spec_query_len=Q,
                                                       max_num_reqs=B)
        pspecs: list = []
        gdn_recoverssm_verify(inp.g, inp.beta, inp.q, inp.k, inp.v, checkpoint_state=w.checkpoints[0],
                              replay_cache=prec, query_start_loc=m.query_start_loc, state_indices=m.state_indices,
                              spec_query_len=Q, out=out, state_cache_retain=STEP_STATE_RETAIN, _collect=pspecs)
        pspecs += list(pctx.make_commit_specs(m.accepted, m.state_indices, m.query_start_loc, commit_conv=False,
                                              **align_kw))
        for _ in range(args.warmup):
            for sp in pspecs:
                sp.launch()
        p0, p1 = timer.event(), timer.event()
        torch.cuda.synchronize()
        timer.record(p0)
        for _ in range(args.steps):
            for sp in pspecs:
                sp.launch()
        timer.record(p1)
        torch.cuda.synchronize()
        pms = timer.elapsed(p0, p1) / args.steps
        T_, acc_ = nbytes["tokens"], nbytes["accepted_tokens"]
        typed_rec, packed_rec = HV * V * 4 + H * K * 2 + HV * 4, HV * (V + K + 1) * 4
        pbytes = total + (T_ + acc_) * (packed_rec - typed_rec)
        packed = {
            "us_per_step": round(pms * 1e3, 2),
            "bytes": pbytes,
            "gbs": round(pbytes / (pms * 1e-3) / 1e9, 1),
            "frac": round(pbytes / (pms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "note": "verify + plan_fold with packed FP32 records [corr|key|decay] per value head; bytes = the typed "
                    "step's with each written and each folded token's record at (V+K+1)*4 per value head",
        }
    full_step = None
    if full_ms is not None:
        conv_dim, conv_len = w.conv_states[0].shape[1:]
        conv_b = conv_bytes(s, ctx.commit_lens[:B].cpu(), ctx.boundary_state_indices[:B].cpu(),
                            ctx.boundary_recovery_lens[:B].cpu(), w.num_pages, conv_dim, conv_len - Q + 1,
                            w.conv_states[0].element_size())
        full_step = {
            "us_per_step": round(full_ms * 1e3, 2),
            "conv_bytes": conv_b,
            "gbs": round((total + conv_b) / (full_ms * 1e-3) / 1e9, 1),
            "frac": round((total + conv_b) / (full_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "conv_us": round((full_ms - step_ms) * 1e3, 2),
            "note": "verify, plan + fold, then the conv compaction (the reference's whole commit); conv_bytes "
                    "counts the kept history positions read and written, conv_us is the step-time difference",
        }

    per_kernel = {}
    for name, ms in kernel_ms.items():
        b = {"verify": nbytes["verify"], "plan_fold": nbytes["commit"]}.get(name)
        entry = {"us": round(ms * 1e3, 2)}
        if b is not None:
            entry.update(bytes=b, gbs=round(b / (ms * 1e-3) / 1e9, 1), frac=round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4))
        per_kernel[name] = entry
    dominant = max(("verify", "plan_fold"), key=lambda n: kernel_ms.get(n, 0.0)) if kernel_ms else "plan_fold"
    dk = per_kernel.get(dominant, {})
    traffic, traffic_src = measured_traffic(s.name, dominant)
    roofline = {
        "kernel": dominant,
        "bound": "hbm",
        "achieved": dk.get("gbs"),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": dk.get("frac"),
        "traffic": traffic,
        "traffic_source": traffic_src,
        "algorithmic_bytes": dk.get("bytes"),
        "avg_us": dk.get("us"),
    }

    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20) // 4
        a = torch.ones(n, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()

    cpu = None
    if want_cpu:
        # torch.set_num_threads(os.cpu_count()), whatever share of those CPUs
        # this process may run on (reported beside it).
        threads = max(1, os.cpu_count() or 1)
        secs, cpu_steps = cpu_baseline(w_cpu, threads)
        cpu = {
            "value": round(total / secs / 1e9, 3),
            "unit": "GB/s",
            "cores": threads,
            "cpus_available": len(os.sched_getaffinity(0)),
            "kind": "port",
            "sample": f"{cpu_steps} full verify+plan+fold steps of {s.name} (all {B} rows, the same bytes per step "
                      f"as value) with the FP32 torch oracle, about 10 s of CPU work; {secs * 1e3:.0f} ms/step",
            "ms_per_step": round(secs * 1e3, 1),
        }

    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "us_per_step": round(step_ms * 1e3, 2),
        "us_per_step_with_kernel_events": round(marked_step_ms * 1e3, 2),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": s.name, "rows": B, "key_heads": H, "value_heads": HV, "key_dim": K, "value_dim": V,
            "window": Q, "mode": "align" if align else "none", "block_size": m.block_size,
            "state": "f32", "activations": "bf16", "key_records": "bf16",
            "state_cache_retain": STEP_STATE_RETAIN,
        },
        "bytes": {**nbytes, "step": total},
        "kernels": per_kernel,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "fused_gating": fused,
        "with_conv_compaction": full_step,
        "packed_records": packed,
        "deferred_commit": deferred,
        "traffic_ceiling": ceiling,
        "other_configs": others,
        "disjoint_pools": pools,
        "cold_step": cold,
        "decode_loop": loop,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

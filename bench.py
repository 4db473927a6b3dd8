#!/usr/bin/env python3
"""Benchmark: one GPU's share of a live-state reshard on MI355X.

Default workload: Llama2-7B-shaped state (bf16 param + f32 master / exp_avg /
exp_avg_sq), TP4,PP2 -> TP2,PP2, destination (pp0, tp0) = layers 0-15 plus the
vocabulary-parallel embedding, from two source TP shards resident in HBM.
A step is one full reshard: pack (sources -> per-peer buffers) + unpack
(buffers -> destination shards), each a single kernel launch.

Prints ONE JSON line.  ``value`` is the whole-job algorithmic throughput
B_alg / t in GB/s with B_alg = 3P + D (pack reads and writes P, unpack reads P
and writes D); ``roofline`` is for the slower of the two kernels, timed with
HIP events on the stream the kernels run on; ``cpu_baseline`` times the
reference-style torch-CPU reshard (chunk/contiguous/cat) on a bounded sample
of the same workload on this host's cores, scaled to the same unit.
``direct_gather`` reports the buffer-free route (one launch, P + D bytes) that
applies when every source shard is resident on this GPU; ``api`` times the
drop-in operator end to end (``schedule_param_transfer`` for every rank, then
``execute_param_transfer`` with the sources resident).

``parity`` is checked outside the timed regions, tensor by tensor and byte
for byte, against the pack + unpack result: the direct gather, the drop-in
operator (fresh and arena destinations) and -- with the CPU baseline on --
the torch-CPU reshard, which runs on host copies of the same seeded source
shards the GPU resharded.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from dataclasses import replace
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBPS = 8000.0
DEFAULT_TILE = 16384   # the library's default tile size (sr_plan_options.tile_bytes = 0)
METRIC = "reshard ms and achieved HBM GB/s (% of peak) per GPU share; speedup vs CPU ref"


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default=None, help="workload key (default: the Llama2-7B share)")
    ap.add_argument("--tile-bytes", type=int, default=0)
    ap.add_argument("--max-blocks", type=int, default=0)
    ap.add_argument("--temporal", action="store_true",
                    help="ordinary cached loads/stores instead of streaming ones")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--host-sources", action="store_true",
                    help="also time the direct route with sources copied from pinned host memory "
                         "(PCIe-inclusive; pins the share's source bytes on the host)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="minimum timed CPU work per thread count")
    ap.add_argument("--cpu-layers", type=int, default=0,
                    help="time a sample with this many destination-stage layers (0: the full share)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="only run a flat copy of BYTES through the library (counter calibration)")
    ap.add_argument("--row-sweep", type=int, default=0, metavar="BYTES",
                    help="strided dim -1 pieces (cat / split) of several row widths against a flat "
                         "copy, BYTES read and written per case, then exit")
    ap.add_argument("--api-phases", action="store_true",
                    help="host-time breakdown of the drop-in execute_param_transfer call for --config "
                         "(--steps calls, each followed by a gather of the whole share for comparison)")
    ap.add_argument("--handoff", action="store_true",
                    help="only run the live migration of the workload between old and new processes on "
                         "this GPU (migration_save / migration_load) and print its timings, then exit")
    ap.add_argument("--handoff-wait-release", action="store_true",
                    help="with --handoff: the new world allocates its destinations only after the old "
                         "world has released its state, even when the device has room for both")
    ap.add_argument("--handoff-return-early", action="store_true",
                    help="with --handoff: the new world returns once its state is adopted, without "
                         "waiting for the old world's release (migration_load(return_before_release=True))")
    ap.add_argument("--handoff-mode", choices=("whole", "waves"), default=None,
                    help="with --handoff: force the hand-off's order (default: whole when it fits)")
    ap.add_argument("--handoff-wave-bytes", type=int, default=None,
                    help="with --handoff-mode waves: bytes per wave (default: a third of the free memory)")
    ap.add_argument("--handoff-squeeze", type=float, default=None, metavar="F",
                    help="with --handoff: hold device memory once every process is up until only F x the "
                         "old state is free (F < 1: a whole hand-off does not fit)")
    ap.add_argument("--checkpoint", metavar="DIR", default=None,
                    help="only run the checkpoint-based migration of the workload (the reference's "
                         "comparator to live migration): the old world's processes checkpoint_save into a "
                         "new directory inside DIR (removed afterwards), then new processes checkpoint_load "
                         "it on this GPU; print the timings, then exit")
    ap.add_argument("--host-state", action="store_true",
                    help="only time the checkpoint-resume reshard of --config from source shards in host "
                         "memory (result on device='cpu' and on the GPU) beside the torch-CPU reference, "
                         "--steps timed calls each, then exit")
    ap.add_argument("--traffic-file", default=str(ROOT / "profiles" / "traffic.json"),
                    help="measured HBM bytes per launch (from rocprofv3 --pmc), if present")
    ap.add_argument("--json-out", default=None)
    return ap.parse_args(argv)


def to_ometa(m):
    from oracle import reshard_oracle as O
    return O.OMeta(name=m.name, itemsize=m.dtype.itemsize, shape=tuple(int(s) for s in m.shape),
                   tp=None if m.tp_meta is None else tuple(m.tp_meta), kind=m.kind,
                   kind_args=tuple(m.kind_args), rows=m.rows)


def cpu_baseline(w, threads: int, min_seconds: float, layers: int = 0, srcs=None, keep_output: bool = False):
    """Time the torch-CPU restatement of the reference's CPU reshard on the
    destination share of ``w`` (or, with ``layers`` > 0, on a sample whose
    destination stage holds that many decoder layers): one untimed run, then
    timed runs until ``min_seconds`` have passed.  ``srcs`` are the seeded
    source shards as CPU tensors (``{rank: {name: {field: tensor}}}``, the
    host copies of what the GPU resharded); without them (the sample) they
    are generated with the workload's seed on the CPU.  Returns (seconds per
    run, algorithmic bytes of the share, runs, decoder layers of the share,
    the untimed run's output if ``keep_output``, the bytes the CPU path moves:
    P read + D written)."""
    import torch
    from oracle import reshard_oracle as O
    from oracle.torch_ref import execute_torch_cpu
    from suika_amd.inventory import layer_partition
    from suika_amd.workloads import make_source_state

    ws = w
    if layers:
        n_layer = max(w.src.pp, w.dst.pp) * layers
        ws = replace(w, model=replace(w.model, n_layer=n_layer))
    spl, tpl = ws.layouts()
    osrc = {r: {n: to_ometa(m) for n, m in metas.items()} for r, metas in spl.layout.items()}
    odst = {r: {n: to_ometa(m) for n, m in metas.items()} for r, metas in tpl.layout.items()}
    ops = [op for op in O.schedule(osrc, odst) if op.dst == ws.dst_rank]
    dt = ws.dtypes
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    kept = None
    try:
        if srcs is None:
            srcs = make_source_state(ws, sorted({op.src for op in ops}), "cpu")
        out = execute_torch_cpu(ops, ws.dst_rank, srcs, list(ws.src_fields), ws.recast_map)
        if keep_output:
            kept = out
        del out
        runs, total = 0, 0.0
        while total < min_seconds or runs == 0:
            t0 = time.perf_counter()
            out = execute_torch_cpu(ops, ws.dst_rank, srcs, list(ws.src_fields), ws.recast_map)
            total += time.perf_counter() - t0
            del out
            runs += 1
        del srcs
    finally:
        torch.set_num_threads(prev)
    # algorithmic bytes of the share, same definition as the GPU figure
    from suika_amd.plan import ReshardPlan, SlotSpec
    ops_p = ws.ops()
    specs = {(op.src_rank, op.param_name, f): SlotSpec(tuple(op.src_meta.actual_shape()), dt[f])
             for op in ops_p for f in ws.src_fields}
    plan = ReshardPlan(ops_p, specs, list(ws.src_fields), recast=ws.recast_map)
    b_alg = plan.pack_bytes + plan.unpack_bytes
    b_min = int(plan.info.pack_bytes_read + plan.info.unpack_bytes_written)
    plan.close()
    dst_pp = ws.dst.coord(ws.dst_rank)[0]
    n_dst_layers = layer_partition(ws.model.n_layer, ws.dst.pp)[dst_pp]
    return total / runs, b_alg, runs, n_dst_layers, kept, b_min


def mismatches(keys, got, want, device=None) -> list:
    """(name, field) of every destination tensor whose bytes differ between
    two results (tensors moved to ``device`` one at a time to compare)."""
    import torch
    bad = []
    for name, f in keys:
        a, b = got[name][f], want[name][f]
        if device is not None:
            a, b = a.to(device), b.to(device)
        if a.shape != b.shape or a.dtype != b.dtype or \
                not torch.equal(a.reshape(-1).view(torch.uint8), b.reshape(-1).view(torch.uint8)):
            bad.append(f"{name}/{f}")
    return bad


def calibrate_copy(nbytes: int, steps: int) -> dict:
    """A flat device copy of ``nbytes`` through the library (one piece): the
    known-size kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE."""
    import torch
    from suika_amd.plan import PlanOptions, ReshardPlan, SlotSpec
    from suika_amd.meta import TensorMeta, TransferOp
    cols = 4096
    rows = nbytes // 4 // cols
    m = TensorMeta(name="copy", dtype=torch.float32, shape=(rows, cols))
    op = TransferOp("copy", 0, 0, m, m, m)
    plan = ReshardPlan([op], {(0, "copy", "param"): SlotSpec((rows, cols), torch.float32)}, ["param"])
    dev = torch.device("cuda", 0)
    a = torch.empty((rows, cols), dtype=torch.float32, device=dev).fill_(1.0)
    bufs = plan.alloc_buffers(dev)
    sp, bp = plan.src_pointers({0: {"copy": {"param": a}}}), plan.buf_pointers(bufs)
    s = torch.cuda.current_stream()
    plan.pack_ptrs(sp, bp, s)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(steps):
        plan.pack_ptrs(sp, bp, s)
    e1.record(s)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    plan.close()
    return {"calibration": "flat copy through sr_pack_kernel", "bytes_read": rows * cols * 4,
            "bytes_written": rows * cols * 4, "ms": round(ms, 4),
            "GBps": round(2 * rows * cols * 4 / ms / 1e6, 1)}


ROW_SWEEP_BYTES = (256, 512, 768, 1024, 2048, 4096, 16384)


def row_sweep(nbytes: int, steps: int) -> list:
    """Bandwidth of strided pieces against a flat copy of the same bytes,
    through sr_gather.  "cat": two [R, C] f32 sources written as the column
    halves of one [R, 2C] destination (the dim -1 merge: strided writes).
    "split": one [R, 2C] source read as two [R, C] destinations (the dim -1
    split: strided reads).  "slice": one band of C columns read out of an
    [R, 8C] source (one destination's piece of a dim -1 split eight ways:
    sparse strided reads over eight times the bytes).  A row of C f32 is the
    row width swept; every case reads and writes ``nbytes``.  Two contiguous
    RECAST cases (the fused fp32 -> bf16 unpack) come first."""
    import ctypes
    import torch
    from suika_amd import _lib
    L = _lib.lib()
    dev = torch.device("cuda", 0)
    s = torch.cuda.current_stream()
    F32 = _lib.SR_DT_F32

    BF16 = _lib.SR_DT_BF16
    tdt = {F32: torch.float32, BF16: torch.bfloat16}

    def run(src_shapes, dst_shapes, pieces, kind=_lib.SR_PIECE_COPY):
        # shapes are (rows, cols) of f32, or (rows, cols, sr dtype)
        src_shapes = [s3 if len(s3) == 3 else (*s3, F32) for s3 in src_shapes]
        dst_shapes = [s3 if len(s3) == 3 else (*s3, F32) for s3 in dst_shapes]
        src = (_lib.SrTensor * len(src_shapes))(*[_lib.SrTensor(r, c, d, 0) for r, c, d in src_shapes])
        dst = (_lib.SrTensor * len(dst_shapes))(*[_lib.SrTensor(r, c, d, 0) for r, c, d in dst_shapes])
        if kind == _lib.SR_PIECE_COPY:
            recs = [_lib.SrPiece(kind, 0, si, di, -1, 0, r, c, 0, sc, 0, dc) for si, di, r, c, sc, dc in pieces]
        elif kind == _lib.SR_PIECE_ZERO:   # (dst, rows, cols)
            recs = [_lib.SrPiece(kind, 0, -1, di, -1, 0, r, c, 0, 0, 0, 0) for di, r, c in pieces]
        else:   # RECAST: (src, f32 dst or -1, bf16 dst2, rows, cols)
            recs = [_lib.SrPiece(kind, 0, si, di, d2, 0, r, c, 0, 0, 0, 0) for si, di, d2, r, c in pieces]
        pcs = (_lib.SrPiece * len(recs))(*recs)
        h = ctypes.c_void_p()
        _lib.check(L.sr_plan_create(src, len(src_shapes), dst, len(dst_shapes), 1, pcs, len(recs), None,
                                    ctypes.byref(h)), "sr_plan_create", L)
        a = [torch.ones((r, c), dtype=tdt[d], device=dev) for r, c, d in src_shapes]
        b = [torch.empty((r, c), dtype=tdt[d], device=dev) for r, c, d in dst_shapes]
        vp = ctypes.c_void_p
        sp = (vp * len(a))(*[t.data_ptr() for t in a])
        dp = (vp * len(b))(*[t.data_ptr() for t in b])
        sh = vp(s.cuda_stream)
        for _ in range(2):
            _lib.check(L.sr_gather(h, sp, dp, sh), "sr_gather", L)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(s)
        for _ in range(steps):
            _lib.check(L.sr_gather(h, sp, dp, sh), "sr_gather", L)
        e1.record(s)
        torch.cuda.synchronize()
        L.sr_plan_destroy(h)
        del a, b
        return e0.elapsed_time(e1) / steps

    out = []
    # the write-only ceiling through the library's own store path: one
    # ZERO piece (the zero fill of padded vocabulary rows) over ``nbytes``
    r, c = nbytes // 4 // 4096, 4096
    ms = run([], [(r, c)], [(0, r, c)], kind=_lib.SR_PIECE_ZERO)
    print(f"[bench] row sweep zero fill: {ms:.3f} ms", file=sys.stderr, flush=True)
    out.append({"pattern": "zero_fill", "row_bytes": None, "rows": r, "bytes_moved": r * c * 4,
                "ms": round(ms, 4), "GBps": round(r * c * 4 / (ms * 1e-3) / 1e9, 1),
                "pct_of_peak": round(100 * r * c * 4 / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 2)})
    # the fused fp32 -> bf16 recast of unpack, contiguous: f32 + bf16 copies
    # (4 bytes read, 6 written per element) and the bf16 copy alone (4 read, 2
    # written), each reading ``nbytes``
    r, c = nbytes // 4 // 4096, 4096
    for name, dshapes, pcs in (("recast", [(r, c), (r, c, BF16)], [(0, 0, 1, r, c)]),
                               ("recast_bf16_only", [(r, c, BF16)], [(0, -1, 0, r, c)])):
        ms = run([(r, c)], dshapes, pcs, kind=_lib.SR_PIECE_RECAST)
        moved = r * c * (4 + 2 + (4 if name == "recast" else 0))
        print(f"[bench] row sweep {name}: {ms:.3f} ms", file=sys.stderr, flush=True)
        out.append({"pattern": name, "row_bytes": None, "rows": r, "bytes_moved": moved, "ms": round(ms, 4),
                    "GBps": round(moved / (ms * 1e-3) / 1e9, 1),
                    "pct_of_peak": round(100 * moved / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 2)})
    for width in ROW_SWEEP_BYTES:
        c = width // 4
        r = nbytes // (2 * width)
        cases = {
            "flat": ([(r, 2 * c)], [(r, 2 * c)], [(0, 0, r, 2 * c, 0, 0)]),
            "cat": ([(r, c), (r, c)], [(r, 2 * c)], [(0, 0, r, c, 0, 0), (1, 0, r, c, 0, c)]),
            "split": ([(r, 2 * c)], [(r, c), (r, c)], [(0, 0, r, c, 0, 0), (0, 1, r, c, c, 0)]),
            # the fifth of eight bands of 2R rows: nbytes read, nbytes written
            "slice": ([(2 * r, 8 * c)], [(2 * r, c)], [(0, 0, 2 * r, c, 4 * c, 0)]),
        }
        for name, (ss, ds, pcs) in cases.items():
            if name == "flat" and width != ROW_SWEEP_BYTES[0]:
                continue
            ms = run(ss, ds, pcs)
            moved = 2 * r * 2 * width
            print(f"[bench] row sweep {name} row {width} B: {ms:.3f} ms", file=sys.stderr, flush=True)
            out.append({"pattern": name, "row_bytes": width if name != "flat" else None, "rows": r,
                        "bytes_moved": moved, "ms": round(ms, 4),
                        "GBps": round(moved / (ms * 1e-3) / 1e9, 1),
                        "pct_of_peak": round(100 * moved / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 2)})
    return out


def api_latency(w, sources, dev, repeats: int = 3, check=None) -> dict:
    """Wall time of the drop-in path: schedule_param_transfer for every rank,
    then execute_param_transfer for this GPU's share with all sources
    resident (fake-source dicts), route "direct".  One untimed call first;
    the caching allocator stays warm between calls (releasing and re-mapping
    ~24 GB per call would time the driver, not the operator)."""
    import statistics

    import torch
    from suika_amd import execute_param_transfer, schedule_param_transfer

    spl, tpl = w.layouts()
    fields = [(f, "normal") for f in w.src_fields]
    sched_ms, exec_ms = [], {False: [], True: []}
    for arena in (False, True):
        for i in range(repeats + 1):
            t0 = time.perf_counter()
            ops = schedule_param_transfer(spl, tpl)
            t1 = time.perf_counter()
            fake = {r: {n: dict(e) for n, e in sd.items()} for r, sd in sources.items()}
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            out = execute_param_transfer(ops, {}, dev, fields, rank=w.dst_rank,
                                         fake_source_state_dicts=fake, recast=w.recast_map,
                                         arena=arena)
            torch.cuda.synchronize()
            t3 = time.perf_counter()
            if check is not None and i == repeats:
                check(arena, out)
            del out, fake
            if i:
                sched_ms.append((t1 - t0) * 1e3)
                exec_ms[arena].append((t3 - t2) * 1e3)
    return {"route": "direct",
            "schedule_param_transfer_ms": round(statistics.median(sched_ms), 2),
            "execute_param_transfer_ms": round(statistics.median(exec_ms[False]), 2),
            "execute_param_transfer_arena_ms": round(statistics.median(exec_ms[True]), 2),
            "runs": repeats,
            "includes": "region lowering, sr_plan_create, destination allocation (warm caching "
                        "allocator), device-side tile/offset/item tables, gather launch, synchronize"}


class _PhaseTimer:
    """A ``prof`` object as execute_param_transfer takes it (start / stop by
    region name, like the reference's profiler): host seconds per region."""

    def __init__(self):
        self.total, self._open = {}, {}

    def start(self, name, **_):
        self._open[name] = time.perf_counter()

    def stop(self, name, **_):
        self.total[name] = self.total.get(name, 0.0) + time.perf_counter() - self._open.pop(name)


def api_phases(w, sources, dev, calls: int) -> dict:
    """Host-time breakdown of the drop-in call (route "direct", fresh
    destinations) on this GPU's share, sources resident.  Each of ``calls``
    timed calls (after 3 untimed) is followed by one gather of the whole
    share as a single plan (HIP events), so call and copy time come from the
    same moments of the box.  Regions: the executor's own prof regions
    (prologue: the rank's ops and the launch groups; gather: per group, the
    native call that plans, allocates the destinations and launches; post
    process: the result dict; wait: the kernels still running).  The parts
    of a group's native call are timed on the same groups by calling them
    one by one (plan; destination tensors; launch)."""
    import statistics

    import torch
    from suika_amd import execute_param_transfer, schedule_param_transfer
    from suika_amd.migration import _pipeline_groups
    from suika_amd.plan import PlanOptions, ReshardPlan

    ops = schedule_param_transfer(*w.layouts())
    mine = [op for op in ops if op.dst_rank == w.dst_rank]
    fields = [(f, "normal") for f in w.src_fields]
    normal = list(w.src_fields)
    stream = torch.cuda.current_stream()
    whole, wsp = ReshardPlan.from_sources(mine, lambda r: sources[r], normal, dev, recast=w.recast_map,
                                          options=PlanOptions(gather_only=True))
    wdst, wdp = whole.alloc_dst_ptrs(dev)

    def one_call(prof=None):
        fake = {r: {n: dict(e) for n, e in sd.items()} for r, sd in sources.items()}
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = execute_param_transfer(ops, {}, dev, fields, rank=w.dst_rank, fake_source_state_dicts=fake,
                                     recast=w.recast_map, prof=prof)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        del out, fake
        return dt

    def one_gather():
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        whole.gather_ptrs(wsp, wdp, stream)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3

    for _ in range(3):
        one_call()
        one_gather()
    call_s, gather_s, regions = [], [], {}
    for _ in range(calls):
        timer = _PhaseTimer()
        call_s.append(one_call(timer))
        gather_s.append(one_gather())
        for k, v in timer.total.items():
            regions.setdefault(k, []).append(v)
    # the parts of the native per-group call, one by one on the same groups
    elem = sum(w.dtypes[f].itemsize for f in w.src_fields)
    groups = _pipeline_groups(mine, elem, 8, len(normal) + len(w.recast_map)).cut()
    opts = PlanOptions(gather_only=True)
    parts = {"plan": [], "destinations": [], "launch": []}
    for _ in range(calls):
        t = {k: 0.0 for k in parts}
        plans = []
        for g in groups:
            t0 = time.perf_counter()
            plan, sp = ReshardPlan.from_sources(g, lambda r: sources[r], normal, dev, recast=w.recast_map,
                                                options=opts)
            t1 = time.perf_counter()
            dst, dp = plan.alloc_dst_ptrs(dev)
            t2 = time.perf_counter()
            plan.gather_ptrs(sp, dp, stream)
            t3 = time.perf_counter()
            t["plan"] += t1 - t0
            t["destinations"] += t2 - t1
            t["launch"] += t3 - t2
            plans.append((plan, dst))
        torch.cuda.synchronize()
        for plan, _ in plans:
            plan.close()
        del plans
        for k in parts:
            parts[k].append(t[k])
    whole.close()
    del wdst

    def ms(v):
        return round(statistics.median(v) * 1e3, 3)

    call, gather = ms(call_s), ms(gather_s)
    return {"config": w.key, "calls": calls, "launch_groups": len(groups),
            "names": len({op.param_name for op in mine}), "ops": len(mine),
            "call_ms": call, "gather_ms": gather, "over_gather": round(call / gather - 1.0, 4),
            "regions_ms": {k: ms(v) for k, v in regions.items()},
            "group_parts_ms": {k: ms(v) for k, v in parts.items()}}


def host_sources_leg(plan, sources, sp, dp, stream, repeats: int = 3) -> dict:
    """PCIe-inclusive rate of the direct route: the share's sources start in
    pinned host memory (as after a checkpoint read), are copied into their HBM
    tensors (one host-to-device copy per tensor, from one pinned allocation),
    and one gather follows on the same stream.  Not the headline value: the
    C ABI takes device pointers, so this adds the host link in front of it."""
    import torch
    tensors = [sources[r][n][f] for (r, n, f) in plan.src_keys]
    offs, total = [], 0
    for t in tensors:
        total = (total + 255) // 256 * 256
        offs.append(total)
        total += t.numel() * t.element_size()
    print(f"[bench] host sources: pinning {total / 1e9:.2f} GB", file=sys.stderr, flush=True)
    host = torch.empty(total, dtype=torch.uint8, pin_memory=True)
    views = [host[o:o + t.numel() * t.element_size()].view(t.dtype).view(t.shape)
             for o, t in zip(offs, tensors)]
    for v, t in zip(views, tensors):
        v.copy_(t)
    torch.cuda.synchronize()
    h2d, gat = [], []
    for _ in range(repeats + 1):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record(stream)
        for v, t in zip(views, tensors):
            t.copy_(v, non_blocking=True)
        e[1].record(stream)
        plan.gather_ptrs(sp, dp, stream)
        e[2].record(stream)
        torch.cuda.synchronize()
        h2d.append(e[0].elapsed_time(e[1]))
        gat.append(e[1].elapsed_time(e[2]))
    h2d, gat = h2d[1:], gat[1:]
    del views, host
    h_ms = sum(h2d) / len(h2d)
    g_ms = sum(gat) / len(gat)
    b_gather = plan.gather_bytes
    return {"source_bytes": total, "tensors": len(tensors), "runs": repeats,
            "h2d_ms": round(h_ms, 2), "h2d_GBps": round(total / (h_ms * 1e-3) / 1e9, 1),
            "gather_ms": round(g_ms, 3), "total_ms": round(h_ms + g_ms, 2),
            "pcie_inclusive_GBps": round(b_gather / ((h_ms + g_ms) * 1e-3) / 1e9, 1),
            "note": "gather bytes (P + D) over host-to-device copies + gather; not the headline value"}


class _PhaseTimes:
    """A profiler for execute_param_transfer's ``prof``: host wall time per
    bracket (ms, summed over the call)."""

    def __init__(self):
        self.ms = {}
        self._t0 = {}

    def start(self, name):
        self._t0[name] = time.perf_counter()

    def stop(self, name):
        self.ms[name] = self.ms.get(name, 0.0) + (time.perf_counter() - self._t0.pop(name)) * 1e3


def host_state_leg(w, dev, repeats: int, cpu_seconds: float) -> dict:
    """The reference's checkpoint-resume reshard (migration.py:1235-1244) on
    the share of ``w``: the source shards in pageable host memory (as
    torch.load returns them), resharded by execute_param_transfer with the
    result on ``device="cpu"`` (the reference's call) and on the GPU (the
    on-load of migration.py:583).  Beside them: the torch-CPU reshard of the
    same host tensors (the reference's own path) and the whole source tensors
    copied to HBM before a gather (what checkpoint_load did before staging
    only piece bytes).  Wall time of the call, host to host (or host to HBM);
    the first call of each kind is untimed."""
    import torch
    from suika_amd import _lib, execute_param_transfer
    from suika_amd.workloads import make_source_state
    ops = w.ops()
    ranks = sorted({op.src_rank for op in ops})
    print(f"[bench] host state {w.key}: generating sources", file=sys.stderr, flush=True)
    src_dev = make_source_state(w, ranks, dev)
    host = {r: {n: {f: t.cpu() for f, t in e.items()} for n, e in sd.items()} for r, sd in src_dev.items()}
    del src_dev
    torch.cuda.empty_cache()
    esf = [(f, "normal") for f in w.src_fields]
    threads = len(os.sched_getaffinity(0))
    print(f"[bench] host state: torch-CPU reshard, {threads} threads", file=sys.stderr, flush=True)
    t_cpu, _, runs_cpu, _, want, b_min = cpu_baseline(w, threads, cpu_seconds, srcs=host, keep_output=True)
    keys = [(n, f) for n, e in want.items() for f in e]
    out = {"workload": w.description or w.key, "key": w.key, "runs": repeats, "B_min_bytes": b_min,
           "cpu_reference": {"ms": round(t_cpu * 1e3, 2), "threads": threads, "runs": runs_cpu,
                             "GBps": round(b_min / t_cpu / 1e9, 2), "cpu_model": cpu_model(),
                             "what": "torch-CPU chunk/contiguous/cat reshard (oracle/torch_ref.py) of the "
                                     "same host tensors"},
           "parity": {"tensors": len(keys), "mismatched": 0}}

    def call(device):
        prof = _PhaseTimes()
        c0 = _lib.stage_counters()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        res = execute_param_transfer(ops, {}, device, esf, rank=w.dst_rank, prof=prof,
                                     fake_source_state_dicts=host, recast=w.recast_map)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3
        c1 = _lib.stage_counters()
        return res, ms, prof.ms, (c1.host_piece_bytes - c0.host_piece_bytes, c1.host_bytes_up - c0.host_bytes_up,
                                  c1.bytes_down - c0.bytes_down)

    for device in ("cpu", "cuda"):
        walls, phases = [], {}
        for i in range(repeats + 1):
            res, ms, ph, moved = call(device)
            if i == 0:
                bad = mismatches(keys, res, want, device=dev if device == "cuda" else None)
                out["parity"]["mismatched"] += len(bad)
                if bad:
                    out["parity"].setdefault("first_mismatches", {})[device] = bad[:5]
                    print(f"[bench] PARITY: device={device} differs in {len(bad)} tensors", file=sys.stderr,
                          flush=True)
            else:
                walls.append(ms)
                for k, v in ph.items():
                    phases[k] = phases.get(k, 0.0) + v / repeats
            del res
        ms = sum(walls) / len(walls)
        out[f"device_{device}"] = {
            "ms": round(ms, 2), "ms_runs": [round(x, 2) for x in walls],
            "speedup_vs_cpu_reference": round(t_cpu * 1e3 / ms, 2),
            "piece_bytes_up": moved[0], "window_bytes_up": moved[1], "bytes_down": moved[2],
            "host_link_GBps": round((moved[1] + moved[2]) / (ms * 1e-3) / 1e9, 1),
            "phases_ms": {k.replace("execute ", ""): round(v, 2) for k, v in sorted(phases.items())}}
        print(f"[bench] host state device={device}: {ms:.1f} ms (CPU reference {t_cpu * 1e3:.1f} ms)",
              file=sys.stderr, flush=True)

    # what checkpoint_load did before: whole source tensors to HBM, then the gather
    needed = {}
    for op in ops:
        needed.setdefault(op.src_rank, set()).add(op.param_name)
    walls = []
    for i in range(repeats + 1):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fake = {r: {n: {f: t.to(dev) for f, t in host[r][n].items()} for n in names} for r, names in needed.items()}
        res = execute_param_transfer(ops, {}, dev, esf, rank=w.dst_rank, fake_source_state_dicts=fake,
                                     recast=w.recast_map)
        torch.cuda.synchronize()
        if i:
            walls.append((time.perf_counter() - t0) * 1e3)
        whole = sum(t.numel() * t.element_size() for sd in fake.values() for e in sd.values() for t in e.values())
        del res, fake
    out["whole_tensors_then_gather"] = {"ms": round(sum(walls) / len(walls), 2), "bytes_up": whole,
                                        "what": "every source tensor a piece reads copied to HBM with "
                                                ".to(device) (pageable), then the drop-in gather"}
    return out


# ---------------------------------------------------------------- live hand-off leg

def _state_optimizer(params):
    """An optimizer that only holds mixed-precision state per parameter (an
    f32 master copy and Adam moments next to a bf16 parameter) and keeps its
    dtypes when loaded: torch's Optimizer.load_state_dict casts floating
    state to the parameter's dtype."""
    import torch

    class MixedPrecisionState(torch.optim.Optimizer):
        def __init__(self, ps):
            super().__init__(ps, {})

        def load_state_dict(self, state_dict):
            params = [p for g in self.param_groups for p in g["params"]]
            self.state.clear()
            for idx, st in state_dict["state"].items():
                p = params[idx]
                self.state[p] = {k: (v.to(device=p.device) if torch.is_tensor(v) else v) for k, v in st.items()}

        def step(self, closure=None):
            raise NotImplementedError("state holder only")

    return MixedPrecisionState(params)


def _seeded_global(w, name: str, shape, device):
    """Seeded global tensors of one name (per-name seed, so any process can
    regenerate them): master ~ N(0, 0.02), exp_avg ~ N(0, 1e-3), exp_avg_sq =
    |N(0, 1e-6)|, bf16 param = RNE(master)."""
    import zlib

    import torch
    from suika_amd.workloads import FIELD_STD
    gen = torch.Generator(device=device)
    gen.manual_seed((w.seed * 1000003 + zlib.crc32(name.encode())) & 0x7FFFFFFFFFFFFFFF)
    dt = w.dtypes
    base = "master" if "master" in w.src_fields else "param"
    out = {}
    for f in (base, "exp_avg", "exp_avg_sq"):
        if f not in w.src_fields:
            continue
        g = torch.randn(shape, generator=gen, dtype=torch.float32, device=device).mul_(FIELD_STD[f])
        if f == "exp_avg_sq":
            g.abs_()
        out[f] = g
    if base == "master" and "param" in w.src_fields:
        out["param"] = out["master"].to(dt["param"])
    return {f: t.to(dt[f]) for f, t in out.items()}


def _timed_log(sink):
    def log(msg):
        sink.append((time.time(), msg))
    return log


def _expected_shard(G, meta):
    """The shard ``meta`` describes, cut from its global tensor ``G`` by
    closed form, written here so the hand-off leg's seeding and check share
    no code with the product's geometry: ``torch.chunk`` along the split dim
    (the reference's column and row splits, tensor_parallel.py:200-204,
    378-381); for a fused QKV weight, the same chunk of each projection's
    rows; for a vocabulary-parallel table, the rank's chunk of the table
    padded with zero rows to a multiple of pad_multiple x TP."""
    import torch
    if meta.tp_meta is None:
        return G
    dim, idx, deg = (int(v) for v in meta.tp_meta)
    if meta.kind == "vocab_pad":
        step = int(meta.kind_args[0]) * deg
        rows = -(-G.shape[0] // step) * step
        padded = torch.zeros((rows,) + tuple(G.shape[1:]), dtype=G.dtype, device=G.device)
        padded[:G.shape[0]] = G
        return torch.chunk(padded, deg, dim=0)[idx].contiguous()
    if meta.kind == "qkv_heads":
        nq, nkv, hd = (int(v) for v in meta.kind_args)
        q, k, v = torch.split(G, [nq * hd, nkv * hd, nkv * hd], dim=0)
        return torch.cat([torch.chunk(x, deg, dim=0)[idx] for x in (q, k, v)], dim=0)
    return torch.chunk(G, deg, dim=dim)[idx].contiguous()


def _handoff_old(rank, key, port, queues, events, opts):
    import traceback

    import torch
    import torch.distributed as dist
    try:
        os.environ.update(MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port))
        from suika_amd import migration_save
        from suika_amd.workloads import CONFIGS
        w = CONFIGS[key]
        dist.init_process_group("gloo", rank=rank, world_size=w.src.world)
        dev = torch.device("cuda", 0)
        torch.cuda.set_device(dev)
        model, opt = _seed_old_rank(w, rank, dev)
        log = []
        events.put(("ready", rank, None))
        if opts.get("gate") is not None:
            assert opts["gate"].wait(600), "the bench never opened the gate"
        migration_save(queues[rank], model, opt, other_context={"iter": 1}, log_func=_timed_log(log),
                       handoff_mode=opts.get("mode"), wave_bytes=opts.get("wave_bytes"))
        events.put(("saved", rank, log))
    except BaseException:
        events.put(("error", rank, traceback.format_exc()))
    finally:
        import torch.distributed as dist
        if dist.is_initialized():
            dist.destroy_process_group()


def _handoff_new(rank, key, port, queues, events, opts):
    import traceback

    import torch
    import torch.distributed as dist
    try:
        os.environ.update(MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port))
        from suika_amd import migration_load
        from suika_amd.inventory import build_module
        from suika_amd.workloads import CONFIGS
        w = CONFIGS[key]
        dist.init_process_group("gloo", rank=rank, world_size=w.dst.world)
        dev = torch.device("cuda", 0)
        torch.cuda.set_device(dev)
        pfield = "param" if "param" in w.src_fields else "master"
        model = build_module(w.model, w.dst, rank, w.dtypes[pfield], device="meta")
        if opts.get("gate") is not None:
            # first-use costs and allocations in place before the bench takes
            # the device memory it holds
            from suika_amd.handoff import _WarmUp
            _WarmUp(dev, optimizer=True).run()
            torch.cuda.synchronize()
            events.put(("ready-new", rank, None))
            assert opts["gate"].wait(600), "the bench never opened the gate"
        log = []
        t0 = time.time()
        opt, ctx = migration_load(queues[rank], model, lambda: _state_optimizer(model.parameters()),
                                  log_func=_timed_log(log), wait_for_release=opts.get("wait_for_release"),
                                  return_before_release=opts.get("return_before_release", False))
        t1 = time.time()
        rec = _check_new_rank(w, rank, model, opt, dev)
        rec.update(log=log, t_call=t0, t_return=t1)
        events.put(("loaded", rank, rec))
    except BaseException:
        events.put(("error", rank, traceback.format_exc()))
    finally:
        import torch.distributed as dist
        if dist.is_initialized():
            dist.destroy_process_group()


def _settle_device(limit_s: float = 30.0) -> float:
    """Wait until the device's free memory stops rising (an earlier run's
    processes may still be returning theirs: allocations from memory in
    that state were 20-30x slower) and return the seconds waited."""
    import torch
    torch.cuda.set_device(0)
    t0 = time.time()
    last = torch.cuda.mem_get_info()[0]
    while time.time() - t0 < limit_s:
        time.sleep(0.5)
        free = torch.cuda.mem_get_info()[0]
        if free <= last + (64 << 20):
            break
        last = free
    return time.time() - t0


def handoff_leg(key: str, timeout_s: float = 600.0, wait_for_release=None, mode=None, wave_bytes=None,
                squeeze=None, return_before_release=False) -> dict:
    """Live migration of workload ``key`` between processes on this GPU: the
    old plan's ranks (seeded state) call migration_save, the new plan's ranks
    migration_load; every received tensor is checked bit for bit.

    ``squeeze``: once every process is up, this process holds device memory
    until only that fraction of the old state is free, so the old world
    picks its order (waves when the whole does not fit) under a real
    shortage."""
    import multiprocessing as mp
    import queue as _queue
    import socket

    from suika_amd.handoff import RESERVE_BYTES, dummy_migration_IPC_state_dict
    from suika_amd.workloads import CONFIGS
    w = CONFIGS[key]
    old_ws, new_ws = w.src.world, w.dst.world
    assert old_ws + new_ws <= 16, "at most 16 processes on the GPU"
    ctx = mp.get_context("spawn")
    queues = [(ctx.Queue(), ctx.Queue()) for _ in range(max(old_ws, new_ws))]
    for q in queues[old_ws:]:          # guards of new ranks without an old counterpart
        q[0].put(dummy_migration_IPC_state_dict)
    events = ctx.Queue()
    results = {}
    deadline = time.time() + timeout_s
    opts = {"wait_for_release": wait_for_release, "mode": mode, "wave_bytes": wave_bytes,
            "return_before_release": return_before_release}
    if squeeze is not None:
        opts["gate"] = ctx.Event()

    def wait_for(kind, count):
        while sum(1 for ev, _ in results if ev == kind) < count:
            try:
                ev, rank, payload = events.get(timeout=max(1.0, deadline - time.time()))
            except _queue.Empty:
                raise RuntimeError(f"hand-off leg: timed out waiting for {kind}; have {sorted(results)}")
            if ev == "error":
                raise RuntimeError(f"hand-off leg: rank {rank} failed:\n{payload}")
            results[(ev, rank)] = payload
            print(f"[bench] hand-off: {ev} {rank}", file=sys.stderr, flush=True)

    def port():
        with socket.socket() as s_:
            s_.bind(("127.0.0.1", 0))
            return s_.getsockname()[1]

    procs = []
    held = {}
    settled = _settle_device()
    try:
        p_old, p_new = port(), port()
        for r in range(old_ws):
            procs.append(ctx.Process(target=_handoff_old, args=(r, key, p_old, queues, events, opts)))
            procs[-1].start()
        wait_for("ready", old_ws)
        for r in range(new_ws):
            procs.append(ctx.Process(target=_handoff_new, args=(r, key, p_new, queues, events, opts)))
            procs[-1].start()
        if squeeze is not None:
            import torch
            wait_for("ready-new", new_ws)
            torch.cuda.set_device(0)
            torch.cuda.synchronize()
            free, _ = torch.cuda.mem_get_info()
            hold = free - int(squeeze * _old_state_bytes(w))
            assert hold > 0, "the device already has less free memory than asked for"
            held["t"] = torch.empty(hold, dtype=torch.uint8, device="cuda")
            torch.cuda.synchronize()
            held["free"] = torch.cuda.mem_get_info()[0]
            print(f"[bench] hand-off: holding {hold / 1e9:.1f} GB, {held['free'] / 1e9:.2f} GB free",
                  file=sys.stderr, flush=True)
            opts["gate"].set()
        wait_for("loaded", new_ws)
        wait_for("saved", old_ws)
        for p in procs:
            p.join(timeout=max(1.0, deadline - time.time()))
    finally:
        for p in procs:
            if p.is_alive():
                p.kill()
                p.join(10)
        if held.pop("t", None) is not None:
            import torch
            torch.cuda.empty_cache()

    def at(log, text):
        return next(t for t, m in log if text in m)

    def low_water(log):
        m = next(m for _, m in log if "low-water free device memory" in m)
        return float(m.rsplit("memory", 1)[1].split()[0]) * 1e9

    old_logs = [results[("saved", r)] for r in range(old_ws)]
    new_recs = [results[("loaded", r)] for r in range(new_ws)]
    start = min(at(l, "is_scale_up") for l in old_logs)         # handshake done
    order_line = next(m for _, m in old_logs[0] if "hand-off whole" in m or "hand-off in waves" in m)
    whole = "hand-off whole" in order_line
    end = max(rec["t_return"] for rec in new_recs)
    adopted = max(at(rec["log"], "model state adopted") for rec in new_recs)
    device_free = max(at(l, "migration_save: end") for l in old_logs)
    out = {
        "workload": w.description or key, "old_ranks": old_ws, "new_ranks": new_ws,
        "state_bytes_received": sum(rec["bytes"] for rec in new_recs),
        "order": order_line.split(": ", 1)[1],
        "handoff_ms": round((end - start) * 1e3, 1),
        "handoff_ms_note": ("wall time from the old world's handshake to the last new rank's return from "
                            "migration_load: pack, queue messages, IPC mapping, reshard, load_state_dict; "
                            "new processes are fresh (first HIP use included)"),
        "state_adopted_ms": round((adopted - start) * 1e3, 1),
        "device_free_ms": round((device_free - start) * 1e3, 1),
        "end_points_note": ("state adopted: the last new rank's load_state_dict done; device free: the last "
                            "old rank has released its state and the hand-off allocations (its return from "
                            "migration_save); both from the handshake"),
        "return_before_release": bool(return_before_release),
        "device_settle_s": round(settled, 2),
    }
    if whole:
        # the old state's release once the new world has mapped the hand-off
        # and allocated (or asked for the memory): its tensors freed and the
        # allocator's cache returned to the device (one hipFree per segment)
        noted = [next(t for t, m in l if "has allocated its destinations" in m or "waits for this state's" in m)
                 for l in old_logs]
        out.update(
            pack_ms_max=round(max((at(l, "packed") - at(l, "hand-off whole")) * 1e3 for l in old_logs), 2),
            release_ms_max=round(max((at(l, "state released") - t) * 1e3 for l, t in zip(old_logs, noted)), 2),
            reshard_ms_max=round(max((at(rec["log"], "resharded in") - at(rec["log"], "destinations of")) * 1e3
                                     for rec in new_recs), 2),
            destinations_waited_for_release=any("after the old world released" in m
                                                for rec in new_recs for _, m in rec["log"]))
    if squeeze is not None:
        lows = [low_water(l) for l in old_logs] + [low_water(rec["log"]) for rec in new_recs]
        out["memory"] = {
            "old_state_bytes": _old_state_bytes(w),
            "free_at_start_bytes": held["free"],
            "peak_beyond_start_bytes": int(held["free"] - min(lows)),
            "reserve_bytes": RESERVE_BYTES * (old_ws + new_ws),
            "note": ("this process held device memory until squeeze x the old state was free; peak = free "
                     "memory at the start less the lowest free memory any rank sampled (after each pack "
                     "and each reshard)")}
    out.update({
        "parity": {"tensors": sum(rec["tensors"] for rec in new_recs),
                   "mismatched": sum(rec["mismatched"] for rec in new_recs),
                   "first_mismatches": [b for rec in new_recs for b in rec["bad"]][:5],
                   "against": ("the same seeded global tensors cut for each new rank by the closed form in "
                               "bench.py (torch.chunk, per-projection QKV chunks, zero-padded vocabulary)")},
        "per_new_rank_log_ms": [
            {m.split(":", 1)[1].strip()[:40]: round((t - rec["t_call"]) * 1e3, 1) for t, m in rec["log"]}
            for rec in new_recs],
        "per_old_rank_log_ms": [
            {m.split(":", 1)[1].strip()[:40]: round((t - start) * 1e3, 1) for t, m in l} for l in old_logs],
        "timing_lines": {"old": [[m for _, m in l if " ms" in m] for l in old_logs],
                         "new": [[m for _, m in rec["log"] if " ms" in m] for rec in new_recs]},
    })
    return out


def _old_state_bytes(w) -> int:
    """Device bytes of every old rank's fields."""
    spl, _ = w.layouts()
    n = 0
    for metas in spl.layout.values():
        for m in metas.values():
            numel = 1
            for d in m.actual_shape():
                numel *= int(d)
            n += numel * sum(w.dtypes[f].itemsize for f in w.src_fields)
    return n


def _seed_old_rank(w, rank: int, dev):
    """An old rank's model (parameters on ``dev``) and state optimizer holding
    its shard of the seeded global state."""
    import torch
    from suika_amd.inventory import build_module
    pfield = "param" if "param" in w.src_fields else "master"
    model = build_module(w.model, w.src, rank, w.dtypes[pfield], device=dev)
    opt = _state_optimizer(model.parameters())
    metas = w.layouts()[0].layout[rank]
    for name, p in model.named_parameters():
        glob = _seeded_global(w, name, tuple(int(x) for x in metas[name].shape), dev)
        with torch.no_grad():
            p.copy_(_expected_shard(glob[pfield], metas[name]))
        opt.state[p] = {f: _expected_shard(glob[f], metas[name]).clone() for f in w.src_fields if f != pfield}
        del glob
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return model, opt


def _check_new_rank(w, rank: int, model, opt, dev) -> dict:
    """Every tensor a new rank received against the seeded state cut for it
    by the closed form above."""
    import torch
    pfield = "param" if "param" in w.src_fields else "master"
    metas = w.layouts()[1].layout[rank]
    state = opt.state_dict()["state"]
    n, bad = 0, []
    for idx, (name, p) in enumerate(model.named_parameters()):
        glob = _seeded_global(w, name, tuple(int(x) for x in metas[name].shape), dev)
        got = {pfield: p, **{f: state[idx][f] for f in w.src_fields if f != pfield}}
        for f, t in got.items():
            want = _expected_shard(glob[f], metas[name])
            n += 1
            if t.dtype != want.dtype or t.shape != want.shape or \
                    not torch.equal(t.reshape(-1).view(torch.uint8), want.reshape(-1).view(torch.uint8)):
                bad.append(f"{name}/{f}")
        del glob
    nbytes = sum(p.numel() * p.element_size() for p in model.parameters()) + \
        sum(t.numel() * t.element_size() for e in state.values() for t in e.values() if torch.is_tensor(t))
    return {"tensors": n, "bad": bad[:5], "mismatched": len(bad), "bytes": nbytes}


def _ckpt_old(rank, key, port, ckpt_dir, events):
    import traceback

    import torch
    import torch.distributed as dist
    try:
        os.environ.update(MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port))
        from suika_amd import checkpoint_save
        from suika_amd.workloads import CONFIGS
        w = CONFIGS[key]
        dist.init_process_group("gloo", rank=rank, world_size=w.src.world)
        dev = torch.device("cuda", 0)
        torch.cuda.set_device(dev)
        model, opt = _seed_old_rank(w, rank, dev)
        dist.barrier()
        t0 = time.time()
        checkpoint_save(model, opt, {"iter": 1}, ckpt_dir)
        dist.barrier()
        events.put(("saved", rank, {"t_call": t0, "t_return": time.time()}))
    except BaseException:
        events.put(("error", rank, traceback.format_exc()))
    finally:
        import torch.distributed as dist
        if dist.is_initialized():
            dist.destroy_process_group()


def _ckpt_new(rank, key, port, ckpt_dir, start, events):
    import traceback

    import torch
    import torch.distributed as dist
    try:
        os.environ.update(MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port))
        from suika_amd import checkpoint_load
        from suika_amd.inventory import build_module
        from suika_amd.workloads import CONFIGS
        w = CONFIGS[key]
        dist.init_process_group("gloo", rank=rank, world_size=w.dst.world)
        dev = torch.device("cuda", 0)
        torch.cuda.set_device(dev)
        pfield = "param" if "param" in w.src_fields else "master"
        model = build_module(w.model, w.dst, rank, w.dtypes[pfield], device="meta")
        events.put(("ready", rank, None))
        start.wait()
        t0 = time.time()
        opt, ctx = checkpoint_load(model, lambda: _state_optimizer(model.parameters()), ckpt_dir, device=dev)
        t1 = time.time()
        rec = _check_new_rank(w, rank, model, opt, dev)
        rec.update(t_call=t0, t_return=t1)
        events.put(("loaded", rank, rec))
    except BaseException:
        events.put(("error", rank, traceback.format_exc()))
    finally:
        import torch.distributed as dist
        if dist.is_initialized():
            dist.destroy_process_group()


def checkpoint_leg(key: str, ckpt_dir: str, timeout_s: float = 900.0) -> dict:
    """Checkpoint-based migration of workload ``key`` on this GPU, the
    reference's comparator to live migration (Suika/migration.py:1156-1305):
    the old plan's ranks (seeded state) checkpoint_save into ``ckpt_dir``,
    then the new plan's ranks, started and waiting, checkpoint_load it; every
    received tensor is checked bit for bit."""
    import multiprocessing as mp
    import queue as _queue
    import shutil
    import socket

    from suika_amd.workloads import CONFIGS
    w = CONFIGS[key]
    old_ws, new_ws = w.src.world, w.dst.world
    assert max(old_ws, new_ws) <= 16, "at most 16 processes on the GPU"
    os.makedirs(ckpt_dir, exist_ok=True)
    # the files hold the whole model state once
    per_elem = sum(w.dtypes[f].itemsize for f in w.src_fields)
    need = sum(m.numel() for metas in w.layouts()[0].layout.values() for m in metas.values()) * per_elem
    free = shutil.disk_usage(ckpt_dir).free
    assert need <= free, f"checkpoint leg: {need / 1e9:.1f} GB needed in {ckpt_dir}, {free / 1e9:.1f} GB free"
    # a directory of its own inside ckpt_dir, removed afterwards: nothing
    # already in ckpt_dir is written over or deleted
    import tempfile
    ckpt_dir = tempfile.mkdtemp(prefix="suika_checkpoint_leg_", dir=ckpt_dir)
    ctx = mp.get_context("spawn")
    events = ctx.Queue()
    start = ctx.Event()
    results = {}
    deadline = time.time() + timeout_s

    def wait_for(kind, count):
        while sum(1 for ev, _ in results if ev == kind) < count:
            try:
                ev, rank, payload = events.get(timeout=max(1.0, deadline - time.time()))
            except _queue.Empty:
                raise RuntimeError(f"checkpoint leg: timed out waiting for {kind}; have {sorted(results)}")
            if ev == "error":
                raise RuntimeError(f"checkpoint leg: rank {rank} failed:\n{payload}")
            results[(ev, rank)] = payload
            print(f"[bench] checkpoint: {ev} {rank}", file=sys.stderr, flush=True)

    def port():
        with socket.socket() as s_:
            s_.bind(("127.0.0.1", 0))
            return s_.getsockname()[1]

    procs = []
    try:
        p_old, p_new = port(), port()
        for r in range(old_ws):
            procs.append(ctx.Process(target=_ckpt_old, args=(r, key, p_old, ckpt_dir, events)))
            procs[-1].start()
        wait_for("saved", old_ws)
        for p in procs:
            p.join(timeout=max(1.0, deadline - time.time()))
        # the new world starts once the old one has exited, as after a restart
        new_procs = [ctx.Process(target=_ckpt_new, args=(r, key, p_new, ckpt_dir, start, events))
                     for r in range(new_ws)]
        for p in new_procs:
            p.start()
        procs += new_procs
        wait_for("ready", new_ws)
        start.set()
        wait_for("loaded", new_ws)
        for p in new_procs:
            p.join(timeout=max(1.0, deadline - time.time()))
    finally:
        for p in procs:
            if p.is_alive():
                p.kill()
                p.join(10)
        shutil.rmtree(ckpt_dir, ignore_errors=True)

    saved = [results[("saved", r)] for r in range(old_ws)]
    loaded = [results[("loaded", r)] for r in range(new_ws)]
    save_ms = (max(r["t_return"] for r in saved) - min(r["t_call"] for r in saved)) * 1e3
    load_ms = (max(r["t_return"] for r in loaded) - min(r["t_call"] for r in loaded)) * 1e3
    return {
        "workload": w.description or key, "old_ranks": old_ws, "new_ranks": new_ws,
        "state_bytes_received": sum(r["bytes"] for r in loaded),
        "save_ms": round(save_ms, 1), "load_ms": round(load_ms, 1),
        "checkpoint_ms": round(save_ms + load_ms, 1),
        "checkpoint_ms_note": ("checkpoint_save of every old rank (first call to the last return, with a "
                               "barrier after) plus checkpoint_load of every new rank (processes started and "
                               "waiting; first call to the last return); process start and exit excluded"),
        "parity": {"tensors": sum(r["tensors"] for r in loaded),
                   "mismatched": sum(r["mismatched"] for r in loaded),
                   "first_mismatches": [b for r in loaded for b in r["bad"]][:5],
                   "against": "the same seeded global tensors cut for each new rank"},
    }


def cpu_model() -> str:
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return "unknown"


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU's share of the reshard; --gpus {args.gpus} is not "
              "supported by this build (the cross-GPU exchange is not implemented).", file=sys.stderr)
        return 2

    import torch
    from suika_amd.plan import PlanOptions, ReshardPlan, SlotSpec
    from suika_amd.workloads import BENCH_CONFIG, CONFIGS, make_source_state

    if args.calibrate_copy:
        torch.cuda.set_device(0)
        print(json.dumps(calibrate_copy(args.calibrate_copy, args.steps)), flush=True)
        return 0
    if args.row_sweep:
        torch.cuda.set_device(0)
        for rec in row_sweep(args.row_sweep, args.steps):
            print(json.dumps(rec), flush=True)
        return 0

    key = args.config or BENCH_CONFIG
    if args.handoff:
        rec = handoff_leg(key, wait_for_release=True if args.handoff_wait_release else None,
                          mode=args.handoff_mode, wave_bytes=args.handoff_wave_bytes,
                          squeeze=args.handoff_squeeze, return_before_release=args.handoff_return_early)
        print(json.dumps({"handoff": rec}), flush=True)
        return 0 if rec["parity"]["mismatched"] == 0 else 1
    if args.checkpoint:
        rec = checkpoint_leg(key, args.checkpoint)
        print(json.dumps({"checkpoint": rec}), flush=True)
        return 0 if rec["parity"]["mismatched"] == 0 else 1
    w = CONFIGS[key]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.host_state:
        rec = host_state_leg(w, dev, args.steps, args.cpu_seconds)
        print(json.dumps({"host_state": rec}), flush=True)
        return 0 if rec["parity"]["mismatched"] == 0 else 1
    if args.api_phases:
        ranks = sorted({op.src_rank for op in w.ops()})
        print(f"[bench] api phases {key}: generating sources", file=sys.stderr, flush=True)
        rec = api_phases(w, make_source_state(w, ranks, dev), dev, args.steps)
        print(json.dumps({"api_phases": rec}), flush=True)
        return 0
    print(f"[bench] workload {key}: planning", file=sys.stderr, flush=True)
    ops = w.ops()
    dt = w.dtypes
    specs = {(op.src_rank, op.param_name, f): SlotSpec(tuple(op.src_meta.actual_shape()), dt[f])
             for op in ops for f in w.src_fields}
    opts = PlanOptions(tile_bytes=args.tile_bytes, max_blocks=args.max_blocks,
                       nontemporal=not args.temporal)
    plan = ReshardPlan(ops, specs, list(w.src_fields), recast=w.recast_map, options=opts)
    info = plan.info
    P = int(info.pack_bytes_read)
    D = int(info.unpack_bytes_written)
    b_pack = plan.pack_bytes
    b_unpack = plan.unpack_bytes
    b_alg = b_pack + b_unpack
    b_min = P + D

    print(f"[bench] generating {P / 1e9:.2f} GB of source shards on {dev}", file=sys.stderr, flush=True)
    sources = make_source_state(w, plan.peers, dev)
    bufs = plan.alloc_buffers(dev)
    dst = plan.alloc_dst(dev)
    sp = plan.src_pointers(sources)
    bp = plan.buf_pointers(bufs)
    dp = plan.dst_pointers(dst)
    stream = torch.cuda.current_stream()

    for _ in range(args.warmup):
        plan.pack_ptrs(sp, bp, stream)
        plan.unpack_ptrs(bp, dp, stream)
    torch.cuda.synchronize()

    K = args.steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(K)]
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    start.record(stream)
    for k in range(K):
        ev[k][0].record(stream)
        plan.pack_ptrs(sp, bp, stream)
        ev[k][1].record(stream)
        plan.unpack_ptrs(bp, dp, stream)
        ev[k][2].record(stream)
    end.record(stream)
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - wall0
    total_ms = start.elapsed_time(end) / K
    pack_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / K
    unpack_ms = sum(e[1].elapsed_time(e[2]) for e in ev) / K
    print(f"[bench] pack {pack_ms:.3f} ms  unpack {unpack_ms:.3f} ms  step {total_ms:.3f} ms  "
          f"wall {wall_s * 1e3 / K:.3f} ms/step", file=sys.stderr, flush=True)

    # Parity, outside the timed region: the pack + unpack result is kept and
    # every other route (gather, the drop-in operator) and the torch-CPU
    # reshard of the same seeded shards must reproduce it byte for byte.
    keys = list(plan.dst_keys)
    ref = {}
    for name, f in keys:
        ref.setdefault(name, {})[f] = dst[name][f].clone()
    parity = {"tensors": len(keys), "mismatched": 0, "routes": {}}

    def record(route, bad):
        parity["routes"][route] = len(bad)
        parity["mismatched"] += len(bad)
        if bad:
            parity.setdefault("first_mismatches", {})[route] = bad[:5]
            print(f"[bench] PARITY: {route} differs in {len(bad)} tensors, first {bad[:3]}",
                  file=sys.stderr, flush=True)

    # The direct route (sources resident on this GPU, no buffers): one gather
    # launch per reshard, P read + D written.  Reported beside the main line.
    for e in dst.values():
        for t in e.values():
            t.view(torch.uint8).fill_(0xA5)
    for _ in range(2):
        plan.gather_ptrs(sp, dp, stream)
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    g0.record(stream)
    for _ in range(K):
        plan.gather_ptrs(sp, dp, stream)
    g1.record(stream)
    torch.cuda.synchronize()
    gather_ms = g0.elapsed_time(g1) / K
    b_gather = plan.gather_bytes
    record("gather_vs_pack_unpack", mismatches(keys, dst, ref))
    host_leg = host_sources_leg(plan, sources, sp, dp, stream) if args.host_sources else None

    # End to end through the drop-in operator: execute_param_transfer with
    # every source resident on this GPU (route "direct").  Host wall time from
    # the call to the synchronised result: region lowering, sr_plan_create,
    # destination allocation, device-side table setup and the gather launch.
    del dst
    api = api_latency(w, sources, dev, repeats=3,
                      check=lambda arena, out: record("execute_param_transfer" + ("_arena" if arena else ""),
                                                      mismatches(keys, out, ref)))

    value = b_alg / (total_ms * 1e-3) / 1e9
    pack_gbps = b_pack / (pack_ms * 1e-3) / 1e9
    unpack_gbps = b_unpack / (unpack_ms * 1e-3) / 1e9
    dom = "sr_unpack_kernel" if unpack_ms >= pack_ms else "sr_pack_kernel"
    dom_ms = max(pack_ms, unpack_ms)
    dom_bytes = b_unpack if unpack_ms >= pack_ms else b_pack
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9

    traffic = None
    tf = Path(args.traffic_file)
    if tf.exists():
        try:
            tdata = json.loads(tf.read_text())
            ent = tdata.get(key, {}).get(dom)
            if ent is not None and ent.get("tile_bytes") == (args.tile_bytes or DEFAULT_TILE) \
                    and ent.get("max_blocks", 0) == args.max_blocks \
                    and bool(ent.get("nontemporal", True)) == (not args.temporal):
                traffic = ent["bytes_per_launch"]
        except Exception as e:  # a malformed file must not hide the measurement
            print(f"[bench] ignoring {tf}: {e}", file=sys.stderr)

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic",
        "config": {
            "workload": w.description or key,
            "key": key,
            "fields": list(w.src_fields) + [t for t, _ in w.recast],
            "pieces": plan.n_pieces,
            "P_bytes": P,
            "D_bytes": D,
            "B_alg_bytes": b_alg,
            "B_min_bytes": b_min,
            "tile_bytes": args.tile_bytes or DEFAULT_TILE,
            "max_blocks": args.max_blocks,
            "nontemporal": not args.temporal,
        },
        "reshard_ms": round(total_ms, 4),
        "pack_ms": round(pack_ms, 4),
        "unpack_ms": round(unpack_ms, 4),
        "pct_of_peak": round(100.0 * value / PEAK_HBM_GBPS, 2),
        "B_min_GBps": round(b_min / (total_ms * 1e-3) / 1e9, 1),
        "pack_GBps": round(pack_gbps, 1),
        "unpack_GBps": round(unpack_gbps, 1),
        "direct_gather": {"ms": round(gather_ms, 4), "bytes": b_gather,
                          "GBps": round(b_gather / (gather_ms * 1e-3) / 1e9, 1),
                          "pct_of_peak": round(100 * b_gather / (gather_ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 2)},
        "api": api,
        "host_sources": host_leg,
        "roofline": {
            "bound": "hbm",
            "kernel": dom,
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": None,
        "parity": parity,
    }

    # the CPU reshard runs on host copies of the same seeded shards
    srcs_cpu = None
    if not args.no_cpu_baseline and not args.cpu_layers:
        print(f"[bench] copying {P / 1e9:.2f} GB of source shards to the host", file=sys.stderr, flush=True)
        srcs_cpu = {r: {n: {f: t.cpu() for f, t in e.items()} for n, e in sd.items()}
                    for r, sd in sources.items()}
    del sources, bufs
    torch.cuda.empty_cache()

    if not args.no_cpu_baseline:
        threads = len(os.sched_getaffinity(0))
        print(f"[bench] CPU baseline: torch-CPU reshard, {threads} threads", file=sys.stderr,
              flush=True)
        t_n, b_n, runs_n, nl, cpu_out, bmin_n = cpu_baseline(w, threads, args.cpu_seconds, args.cpu_layers,
                                                             srcs=srcs_cpu, keep_output=srcs_cpu is not None)
        if cpu_out is not None:
            print("[bench] comparing every destination tensor with the torch-CPU reshard",
                  file=sys.stderr, flush=True)
            record("vs_torch_cpu_reference", mismatches(keys, cpu_out, ref, device=dev))
            parity["cpu_reference"] = ("torch-CPU reshard (oracle/torch_ref.py: the reference's fake-source "
                                       "chunk/contiguous/cat loop) of the same seeded source shards")
            del cpu_out
        t_1, b_1, runs_1, nl1, _, bmin_1 = cpu_baseline(w, 1, args.cpu_seconds, args.cpu_layers, srcs=srcs_cpu)
        del srcs_cpu
        # the bytes the CPU path moves (P read + D written: no buffers) per second
        rate_n = bmin_n / t_n / 1e9
        rate_1 = bmin_1 / t_1 / 1e9
        full_ms = b_min / (rate_n * 1e9) * 1e3
        what = "the full destination share" if not args.cpu_layers else \
            f"a sample with {nl} destination-stage layers"
        result["cpu_baseline"] = {
            "value": round(rate_n, 2),
            "unit": "GB/s",
            "cores": threads,
            "kind": "port",
            "sample": (f"torch-CPU chunk/contiguous/cat reshard (oracle/torch_ref.py) of {what}, "
                       f"seeded source shards (host copies of the GPU's inputs), "
                       f"{bmin_n / 1e9:.2f} GB moved (P + D), {runs_n} timed runs of {t_n:.3f} s"),
            "value_bytes": "B_min = P + D, the bytes the CPU path reads and writes",
            "B_alg_GBps": round(b_n / t_n / 1e9, 2),
            "ms": round(full_ms, 1),
            "one_thread_GBps": round(rate_1, 2),
            "one_thread_ms": round(b_min / (rate_1 * 1e9) * 1e3, 1),
            "one_thread_sample": f"{runs_1} timed runs of {t_1:.3f} s",
            "cpu_model": cpu_model(),
            "speedup_gpu_vs_cpu": round(full_ms / total_ms, 1),
        }
        print(f"[bench] CPU {rate_n:.2f} GB/s ({threads} thr), 1 thr {rate_1:.2f} GB/s", file=sys.stderr,
              flush=True)

    del ref
    plan.close()
    line = json.dumps(result)
    print(line, flush=True)
    if args.json_out:
        Path(args.json_out).write_text(line + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())

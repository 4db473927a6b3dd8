"""Drop-in state-migration operators running on the HIP reshard engine.

Same names, arguments and error behaviour as the reference's operators:

* ``execute_param_transfer``              -- Suika/migration.py:397-556
* ``schedule_and_execute_param_transfer`` -- Suika/migration.py:558-598
* ``merge_model_and_optimizer_state_dict`` / ``split_...``
                                          -- Suika/migration.py:675-746

``execute_param_transfer`` compiles the TransferOps that land on this rank
into a ``ReshardPlan`` and runs it on the GPU, either as one gather pass
(sources -> destination) or as pack -> per-peer buffers -> unpack.  On one
GPU all peers' shards are resident in this GPU's HBM
(``fake_source_state_dicts`` holds them, as in the reference's checkpoint
path, migration.py:1223-1244).  Sources may also live in host memory, as the
reference's checkpoint path loads them (migration.py:477-482, 583), and the
result may be asked for on ``device="cpu"`` (:1235-1244): then only the
pieces' bytes go to the GPU, packed by host threads through pinned windows
(``sr_stage_pack``), the GPU unpacks them, and a host result comes back
through the same windows (``sr_download``).  There is no CPU reshard: without
a GPU the call raises.  A cross-GPU exchange between pack and unpack is not
part of this build: ops from a remote rank without a local copy of its shards
raise ``NotImplementedError``.

Deliberate difference: pieces are placed in ascending global order.  The
reference appends pieces whose source is the executing rank after all others
(migration.py:454-459, 492, 508-509), which concatenates a TP merge out of
order when that rank owns a leading piece; this build implements the
intended ``cat`` in ascending piece order.
"""
from __future__ import annotations

import bisect
import contextlib
import gc
import time
from dataclasses import replace
from typing import Any, Callable, Dict, List, Mapping, Optional, Tuple, Union

import numpy as np
import torch
import torch.distributed as dist
from torch import Tensor
from torch.nn import Module
from torch.optim import Optimizer

from .meta import (CHUNK, QKV_HEADS, ParamLayout, Schedule, TensorMeta, TransferOp,
                   get_named_parameters_and_persistent_buffers, schedule_param_transfer)
from . import _lib
from .plan import PlanOptions, ReshardPlan, download

StateDict = Dict[str, Dict[str, Tensor]]


_GATHER_ONLY = PlanOptions(gather_only=True)


class _NoProf:
    def start(self, *a, **k):
        pass

    def stop(self, *a, **k):
        pass


def _is_meta_field(field_type) -> bool:
    return not (isinstance(field_type, str) and field_type == "normal")


def forcefully_free_tensor(tensor: Tensor) -> None:
    """Release a tensor's storage now (Suika/utils.py:255-260)."""
    if isinstance(tensor, torch.Tensor):
        if tensor.untyped_storage().resizable():
            tensor.untyped_storage().resize_(0)
        else:
            tensor.data = torch.empty(0, device="meta")


def cuda_gc() -> None:
    """Collect garbage and return cached device memory to the driver
    (Suika/utils.py:248-253): Python's collector, then torch's cache, a
    device synchronisation and the release of unused IPC handles."""
    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
        torch.cuda.synchronize()
        torch.cuda.ipc_collect()


def _current_rank(world) -> int:
    if dist.is_available() and dist.is_initialized():
        return dist.get_rank(world)
    return 0


def execute_param_transfer(
    transfer_ops: List[TransferOp],
    source_state_dict: StateDict,
    device: torch.device,
    expected_sub_fields: List[Tuple[str, Union[str, TensorMeta]]],
    world: Optional[dist.ProcessGroup] = None,
    log_func: Optional[Callable] = None,
    prof=None,
    forcefully_free: bool = False,
    fake_source_state_dicts: Optional[Dict[int, StateDict]] = None,
    *,
    rank: Optional[int] = None,
    recast: Optional[Mapping[str, str]] = None,
    plan_options: Optional[PlanOptions] = None,
    stream: Optional[torch.cuda.Stream] = None,
    route: str = "direct",
    arena: bool = False,
    pipeline: int = 8,
) -> StateDict:
    """Execute a transfer schedule for this rank; returns its target state.

    ``source_state_dict`` (this rank's own shards) is cleared in place, as in
    the reference (migration.py:527).  Normal sub-fields move through the HIP
    kernels; 1-element sub-fields (e.g. AdamW ``step``) are copied whole
    (migration.py:443-446, 479-487).  Extensions: ``rank`` overrides
    ``dist.get_rank(world)``; ``recast`` maps a bf16 target field to the f32
    field it is rounded from; ``plan_options`` tunes the kernels; ``route``
    is ``"direct"`` (one gather pass from the resident sources, the default
    since every source is on this GPU) or ``"buffers"`` (pack into per-peer
    buffers, then unpack: the path an exchange between GPUs goes through);
    ``arena`` places every destination tensor in one allocation (field by
    field over all tensors, schedule order within a field, 256-byte
    aligned), for a model that adopts them with
    ``load_state_dict(assign=True)``; ``pipeline`` cuts the transfer into up
    to that many launch groups of whole tensors, each planned on the host
    while the GPU runs the previous one (largest tensors first, sized by a
    cost model of host planning and GPU copy time); ``stream`` runs the
    kernels on that stream, after the work already queued on the current
    stream (which may be producing the sources).  The returned dict lists
    the tensors in schedule order whatever the launch order.  The call
    returns when the kernels are done.

    ``device`` is where the new state is returned: a GPU, or ``"cpu"`` (the
    reference's checkpoint_load, migration.py:1235-1244), whose result is
    resharded on the current GPU and copied back to host memory.  Sources
    in host memory (the fake-source mode, migration.py:477-482) are staged:
    only the bytes of the pieces this rank reads cross to the GPU, packed by
    host threads into the peer-buffer layout, and the GPU unpacks them; such
    a transfer runs as one launch group (the host copies set its pace).
    """
    assert route in ("direct", "buffers"), f"unknown route {route!r}"
    _lib.lib()   # raises when the HIP library is missing: there is no other path
    quiet = log_func is None
    if quiet:
        log_func = lambda msg: None  # noqa: E731
    if prof is None:
        prof = _NoProf()
    if not isinstance(device, torch.device):
        device = torch.device(device)
    assert device.type in ("cuda", "cpu"), \
        f"execute_param_transfer returns state on a GPU or in host memory; got device {device}"
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    # the GPU the reshard runs on: the device asked for, or for host results
    # the current one (the kernels do the work either way; no CPU path)
    if device.type == "cpu" and not torch.cuda.is_available():
        raise RuntimeError("execute_param_transfer reshards on the GPU engine, also for device='cpu'; "
                           "no GPU is available")
    gpu = device if device.type == "cuda" else torch.device("cuda", torch.cuda.current_device())
    if rank is None:
        rank = _current_rank(world)

    prof.start("execute prologue")
    # this rank's ops, grouped by tensor with each tensor's elements, in one
    # pass over the schedule
    scheduled = type(transfer_ops) is Schedule   # its rank positions and encoding tables ride along
    encoding = transfer_ops.encoding() if scheduled else None
    runs = _lib.host().rank_runs(transfer_ops, int(rank), transfer_ops.positions_of(rank) if scheduled else None,
                                 encoding)
    ops = runs[0]
    normal = [f for f, t in expected_sub_fields if not _is_meta_field(t)]
    scalars = [f for f, t in expected_sub_fields if _is_meta_field(t)]
    recast = dict(recast or {})

    def source(r: int) -> StateDict:
        if fake_source_state_dicts is not None and r in fake_source_state_dicts:
            return fake_source_state_dicts[r]
        if r == rank:
            return source_state_dict
        raise NotImplementedError(
            f"[{rank}]: piece from rank {r} needs a cross-GPU exchange, which this one-GPU build "
            "does not implement; pass the peer shards as fake_source_state_dicts")

    # bytes per element of each moved field, from the first op's sources
    first = source(ops[0].src_rank).get(ops[0].param_name, {}) if ops and normal else {}
    itemsize = [first[f].element_size() if f in first else 0 for f in normal]
    elem_bytes = sum(itemsize)   # over all moved fields (balances the launch groups)
    n_copies = sum(1 for sf in recast.values() if sf in normal)   # bf16 recast targets
    groups = _pipeline_groups(ops, elem_bytes, pipeline, len(normal) + n_copies, runs=runs[1:])
    # fresh destinations of the direct route: their allocations are made on
    # a helper thread from here on, tensor by tensor in launch order, while
    # this thread plans the groups (each tensor's elements: its pieces';
    # each field's element size: the first source's)
    blocks = None
    if not arena and route == "direct" and device.type == "cuda" and any(itemsize) and \
            all(first[f].is_cuda for f in normal if f in first):
        copies = set(recast.values())
        launch = getattr(groups, "launch_order", None)   # the order the groups take the tensors in
        if launch is None:
            launch = np.arange(len(runs[3]), dtype=np.int64)
        blocks = _lib.host().start_blocks(gpu.index, launch, runs[3], runs[6], itemsize,
                                          [1 if f in copies else 0 for f in normal])
    # the staged route (sources in host memory, or results for the host)
    # packs on the host and unpacks on the GPU: its plans keep both phases
    stage_options = replace(plan_options, gather_only=False) if plan_options is not None else None
    if route == "direct":   # the plans only ever gather
        plan_options = _GATHER_ONLY if plan_options is None else replace(plan_options, gather_only=True)
    arena_views = _arena_views(ops, source, normal, recast, device) if arena else None
    ahead = (runs[5], blocks) if blocks is not None else None
    # the direct route's launch groups: planned, allocated and gathered in
    # one native call each
    gather = ReshardPlan.gatherer(source, normal, device, recast=recast, options=plan_options, rank=rank,
                                  stream=stream, encoding=encoding) \
        if route == "direct" and device.type == "cuda" else None
    target: StateDict = {}
    plans: List[ReshardPlan] = []
    buffers: List[List[Tensor]] = []

    def staged(todo: List[TransferOp]) -> None:
        """The transfer of ``todo`` from sources wherever they are: the
        pieces' bytes packed on the host (or on the GPU for sources there)
        into peer buffers in HBM, the unpack on the GPU, and for host results
        the copy back.  It runs in groups of whole tensors of about
        ``_stage_group_bytes`` piece bytes each: a group's buffers are
        released once it is unpacked, and a host result's download (its own
        stream, the device-to-host direction of the link) overlaps the next
        group's upload."""
        if todo is ops:
            order, starts, numel = runs[1], runs[2], runs[3]
        else:
            order, starts, numel = _lib.host().name_runs(todo)[:3]
        picks = _stage_groups(np.asarray(numel, dtype=np.int64) * max(1, elem_bytes))
        # buffers allocated on the current stream may be released per group
        # only when the kernels run on that stream
        cur = torch.cuda.current_stream(gpu)
        keep_buffers = stream is not None and stream != cur
        down = pending = None
        if device.type == "cpu":
            down = _Download.stream(gpu)
            pending = []
        try:
            for pick in picks:
                group = todo if len(picks) == 1 else _lib.host().take_ops(todo, order, starts, pick)
                prof.start("execute stage plan")
                try:
                    plan, src_ptrs = ReshardPlan.from_sources(group, source, normal, gpu, recast=recast,
                                                              options=stage_options, rank=rank, host_ok=True)
                finally:
                    prof.stop("execute stage plan")
                plans.append(plan)
                bufs = plan.alloc_buffers(gpu)
                buf_ptrs = [b.data_ptr() for b in bufs]
                prof.start("execute stage pack")
                plan.stage_pack_ptrs(src_ptrs, buf_ptrs, stream)
                prof.stop("execute stage pack")
                names = dict.fromkeys(op.param_name for op in group)
                if device.type == "cuda":
                    if arena_views is None:
                        part, dst_ptrs = plan.alloc_dst_ptrs(device)
                    else:
                        part = {name: arena_views[name] for name in names}
                        dst_ptrs = plan.bind_dst_ptrs(part, device)
                    plan.unpack_ptrs(buf_ptrs, dst_ptrs, stream)
                else:
                    # the GPU's result in one temporary allocation, then host
                    # memory, on the download stream after the unpack
                    hbm = plan.alloc_dst(gpu, arena=True)
                    plan.unpack_ptrs(buf_ptrs, plan.bind_dst_ptrs(hbm, gpu), stream)
                    unpacked = torch.cuda.Event()
                    unpacked.record(stream or cur)
                    prof.start("execute stage host tensors")
                    if arena_views is not None:
                        part = {name: arena_views[name] for name in names}
                    else:
                        part = {name: {f: torch.empty(t.shape, dtype=t.dtype) for f, t in ent.items()}
                                for name, ent in hbm.items()}
                    prof.stop("execute stage host tensors")
                    pairs = [(t, part[name][f]) for name, ent in hbm.items() for f, t in ent.items()]
                    del hbm
                    pending.append(_Download.submit(gpu, down, unpacked, pairs))
                    del pairs
                if keep_buffers:
                    buffers.append(bufs)
                del bufs
                target.update(part)
        finally:
            if pending is not None:
                # every download ends before the call returns (or raises)
                prof.start("execute stage download wait")
                errors = [e for e in (job.result() for job in pending) if e is not None]
                prof.stop("execute stage download wait")
                if errors:
                    raise errors[0]

    def _device_group(group: List[TransferOp]) -> None:
        """One launch group from sources on the device: planned, allocated
        and gathered in one native call (direct route), or packed into peer
        buffers and unpacked (buffers route).  A source in host memory
        raises ``_lib.HostSourceError`` before any allocation or launch."""
        if route == "direct":
            # plan (shapes, dtypes and addresses read from the source
            # tensors, each checked once), the destinations (fresh, or
            # the arena's views) and the gather into them: one native
            # call
            part = None
            if arena_views is not None:
                part = {name: arena_views[name] for name in dict.fromkeys(op.param_name for op in group)}
            prof.start("execute gather")
            try:
                plan, part = gather(group, part, ahead)
            finally:
                prof.stop("execute gather")
            plans.append(plan)
            target.update(part)
            return
        prof.start("execute schedule lowering")
        # shapes, dtypes and addresses read from the source tensors (each
        # checked once: contiguous, on this device)
        try:
            plan, src_ptrs = ReshardPlan.from_sources(group, source, normal, device, recast=recast,
                                                      options=plan_options, rank=rank)
        finally:
            prof.stop("execute schedule lowering")
        plans.append(plan)
        if arena_views is None:
            # fresh tensors of the planned shapes: their addresses need no check
            part, dst_ptrs = plan.alloc_dst_ptrs(device)
        else:
            part = {name: arena_views[name] for name in dict.fromkeys(op.param_name for op in group)}
            dst_ptrs = plan.bind_dst_ptrs(part, device)
        bufs = plan.alloc_buffers(device)
        buffers.append(bufs)
        buf_ptrs = [b.data_ptr() for b in bufs]
        prof.start("execute pack")
        plan.pack_ptrs(src_ptrs, buf_ptrs, stream)
        prof.stop("execute pack")
        prof.start("execute unpack")
        plan.unpack_ptrs(buf_ptrs, dst_ptrs, stream)
        prof.stop("execute unpack")
        target.update(part)

    # A full pass of Python's cyclic collector over a large heap (tens of ms)
    # would stall the host between launch groups and idle the GPU; it is
    # paused for the call (reference counting still frees memory).
    if stream is not None:
        # the sources (and memory the allocator hands out) may still be in
        # use by work queued on the current stream
        cur = torch.cuda.current_stream(gpu)
        if stream != cur:
            stream.wait_stream(cur)
    gc_was_enabled = gc.isenabled()
    gc.disable()
    prof.stop("execute prologue")
    try:
        with (contextlib.nullcontext() if gpu.index == torch.cuda.current_device()
              else torch.cuda.device(gpu)):
            # Each group is planned on the host while the GPU runs the
            # previous group's launch.  A source in host memory sends the
            # rest of the transfer through the staged route.
            done: List[List[TransferOp]] = []
            for group in (() if device.type == "cpu" else groups):
                try:
                    _device_group(group)
                except _lib.HostSourceError:
                    if blocks is not None:
                        blocks.finish()
                    done_names = {op.param_name for g in done for op in g}
                    staged([op for op in ops if op.param_name not in done_names] if done_names else ops)
                    break
                done.append(group)
            else:
                if device.type == "cpu":
                    staged(ops)
            if blocks is not None:
                blocks.finish()   # blocks no tensor took (another dtype, say) are freed
        if not quiet:
            log_func(f"=== reshard plan: {sum(p.n_pieces for p in plans)} pieces in {len(plans)} "
                     f"launch group(s), {sum(p.info.buffer_bytes for p in plans) / 1e6:.1f} MB of buffers ===")

        # The rest of the host work runs while the last launches finish.
        # 1-element sub-fields ride along whole; the first op's source wins,
        # matching tensors[0].clone() of migration.py:538.
        prof.start("execute post process")
        for f in scalars:
            for op in ops:
                entry = target.get(op.param_name)
                if entry is None or f in entry:
                    continue
                src_entry = source(op.src_rank)[op.param_name]
                if f in src_entry:
                    entry[f] = src_entry[f].to(device).clone()

        # names in schedule order (launch groups take the largest first),
        # recast targets first, then the sub-fields in their order
        field_order = list(recast) + [f for f, _ in expected_sub_fields if f not in recast]
        ordered: StateDict = _lib.host().ordered_result(ops, target, field_order)
        if gc_was_enabled and not (stream or torch.cuda.current_stream(gpu)).query():
            # the youngest generation, thousands of objects made by this call
            # (tensors, dicts), is collected while the last launches still
            # run, where it costs nothing, instead of on the caller's first
            # allocation afterwards; once the kernels are done it would only
            # delay the return, and the interpreter collects it later as
            # after any call that returns many objects
            gc.collect(0)
        prof.stop("execute post process")
    finally:
        # destroying a plan waits for its launches: buffers and sources may
        # be released afterwards whatever stream the kernels ran on
        if blocks is not None:
            blocks.finish()
        prof.start("execute wait")
        for plan in plans:
            plan.close()
        prof.stop("execute wait")
        if gc_was_enabled:
            gc.enable()
    del buffers

    if forcefully_free:
        # the source tensors the reference's freed pieces share storage with
        # (migration.py:539-541); the rest stays untouched
        for op in ops:
            entry = source(op.src_rank).get(op.param_name, {})
            if _piece_aliases_source(op):
                for f in normal:
                    if f in entry:
                        forcefully_free_tensor(entry[f])
            for f in scalars:
                t = entry.get(f)
                if isinstance(t, Tensor) and t.device == device:
                    forcefully_free_tensor(t)
    source_state_dict.clear()
    return ordered


# Piece bytes per launch group of the staged route: about 1/STAGE_GROUPS of
# the transfer, between the two bounds (a group costs about a millisecond of
# planning; the first upload and the last download do not overlap).
STAGE_GROUPS = 16
STAGE_GROUP_MIN = 32 << 20
STAGE_GROUP_MAX = 1 << 30


def _stage_groups(tensor_bytes: np.ndarray) -> List[np.ndarray]:
    """Tensor indices (order of first appearance) cut into consecutive
    groups of about max(STAGE_GROUP_MIN, min(STAGE_GROUP_MAX, total /
    STAGE_GROUPS)) bytes; a tensor larger than that is a group of its own."""
    n = len(tensor_bytes)
    if n == 0:
        return [np.arange(0)]
    total = int(tensor_bytes.sum())
    target = max(STAGE_GROUP_MIN, min(STAGE_GROUP_MAX, total // STAGE_GROUPS))
    out, start, acc = [], 0, 0
    for i in range(n):
        acc += int(tensor_bytes[i])
        if acc >= target:
            out.append(np.arange(start, i + 1))
            start, acc = i + 1, 0
    if start < n:
        out.append(np.arange(start, n))
    return out


class _Download:
    """Downloads of host results, one at a time on a worker thread (so that
    a group's download overlaps the next group's upload on the calling
    thread) and on one stream per device (default priority): the download
    stream waits for the group's unpack, then sr_download copies every
    (device, host) pair.  ``submit`` returns a future whose result is None
    or the exception raised.  A forked child makes its own worker."""

    _pool = None
    _pid = None
    _streams: Dict[int, torch.cuda.Stream] = {}

    @classmethod
    def _ensure(cls) -> None:
        import os
        if cls._pool is None or cls._pid != os.getpid():
            from concurrent.futures import ThreadPoolExecutor
            cls._pool = ThreadPoolExecutor(max_workers=1, thread_name_prefix="suika-download")
            cls._pid = os.getpid()
            cls._streams = {}

    @classmethod
    def stream(cls, gpu: torch.device) -> torch.cuda.Stream:
        cls._ensure()
        if gpu.index not in cls._streams:
            cls._streams[gpu.index] = torch.cuda.Stream(gpu)
        return cls._streams[gpu.index]

    @classmethod
    def submit(cls, gpu, stream, after, pairs):
        cls._ensure()

        def job():
            try:
                with torch.cuda.device(gpu):
                    stream.wait_event(after)
                    download(pairs, stream)
                return None
            except BaseException as e:   # handed to the caller, which raises it
                return e
        return cls._pool.submit(job)


def _tp_deg(meta) -> int:
    tp = getattr(meta, "tp_meta", None)
    return 1 if tp is None else int(tp[2])


def _piece_aliases_source(op: TransferOp) -> bool:
    """Whether the reference's piece of ``op`` shares the source tensor's
    storage, so that its ``forcefully_free`` (migration.py:539-541) releases
    the source.  ``get_send_tensor`` (:290-312) sends the source itself when
    it is at least as fine as the piece, and otherwise
    ``chunk(n, slice_dim)[k].contiguous()``: a view of the source when the
    chunk is contiguous (split along the first dimension of extent above 1),
    a copy otherwise (a row-parallel split).  A vocabulary piece is a row
    range (a view); a head-granular QKV piece concatenates three chunks (a
    copy).  A 1-element field is sent as ``tensor.to(device)``: the tensor
    itself when it is already on the device."""
    src, piece = op.src_meta, op.dst_meta
    if getattr(piece, "rows", None) is not None:
        return True
    if _tp_deg(src) >= _tp_deg(piece):
        return True
    if getattr(src, "kind", CHUNK) == QKV_HEADS:
        return False
    shape = [int(x) for x in src.shape]
    tp = getattr(piece, "tp_meta", None) or getattr(src, "tp_meta", None)
    dim = tp[0] % len(shape) if shape else 0
    local = list(shape)
    local[dim] //= max(1, _tp_deg(src))
    return all(x == 1 for x in local[:dim])


# Cost model of a launch group, measured on MI355X: the host plans a group
# (sources read, lowering, plan, destination tensors, launch) in about
# PLAN_NS_PER_GROUP plus PLAN_NS_PER_TENSOR per destination tensor, and the
# gather moves GATHER_BYTES_PER_NS algorithmic bytes (read + written) per ns.
PLAN_NS_PER_GROUP = 60_000
PLAN_NS_PER_TENSOR = 1_000
GATHER_BYTES_PER_NS = 6_100
# Floor of a measured per-tensor planning time: a group planned faster than
# PLAN_NS_PER_GROUP still costs its tensors something (allocating one alone
# takes longer than this).
MIN_PLAN_NS_PER_TENSOR = 100
# GPU work of the first launch group: the host then plans the second while
# it runs.
FIRST_GROUP_NS = 100_000
# Share of a group's GPU time the next group's planning may take.
PLAN_SHARE = 0.9
# Fewest tensors of a group that is not the last: when the previous group's
# GPU time covers the planning of fewer, the host is the bottleneck and the
# rest is planned as one group.
MIN_GROUP_TENSORS = 4


def _arena_views(ops: List[TransferOp], source: Callable[[int], StateDict], fields: List[str],
                 recast: Mapping[str, str], device: torch.device) -> StateDict:
    """Every destination tensor of the transfer on the storage of one
    allocation, laid out before any plan is built: field by field (bf16
    recast targets first, then the moved fields), tensors in schedule order
    within a field, each at a 256-byte aligned offset.  Launch groups then
    write into it.  The shapes (the destination shards'), dtypes, layout and
    tensors are computed by the host extension in one pass."""
    targets = [t for t, sf in recast.items() if sf in fields]
    order = targets + [f for f in fields if f not in recast]
    return _lib.host().arena_tensors(ops, source, order, targets, device)


_clock_ns = time.perf_counter_ns   # the launch groups' planning timer


class _LaunchGroups:
    """The launch groups of one rank's ops, cut as the call goes: whole
    tensors per group (all ops of a name stay together, so each group's plan
    covers its destinations completely), each group planned on the host
    while the GPU runs the previous one.

    A two-stage pipeline (host planning, then GPU copy) finishes soonest
    when the jobs heavy on the second stage go first (Johnson's rule): the
    tensors are taken largest first, so the GPU starts on a large tensor
    planned in little time, and the small tensors, cheap to copy but as
    costly to plan as large ones, come last.  The first group carries
    FIRST_GROUP_NS of GPU work; each next group holds as many tensors as the
    host can plan in PLAN_SHARE of the previous group's GPU time, at the
    host's planning rate measured on the groups so far (PLAN_NS_PER_TENSOR
    until a group of at least MIN_GROUP_TENSORS names was timed); the rest
    forms the last group once a next group would hold fewer than
    MIN_GROUP_TENSORS names or less GPU time than its own planning overhead
    (PLAN_NS_PER_GROUP), or at the ``pipeline``-th group.  Within a group
    the tensors stay largest first (``launch_order``, the order in which
    their destinations are allocated ahead), each tensor's ops in schedule
    order.

    Iterating yields the groups; the time between two requests is taken as
    the planning time of the group handed out first.  ``elem_bytes`` is the
    bytes per element over all moved fields, ``tensors_per_name`` the
    destination tensors per name (fields and recast copies)."""

    def __init__(self, ops: List[TransferOp], elem_bytes: int, pipeline: int, tensors_per_name: int = 1,
                 runs=None):
        self.ops = list(ops)
        self.pipeline = int(pipeline)
        self.per_name = max(1, int(tensors_per_name))
        # op indices tensor by tensor, tensors in order of first appearance,
        # and each tensor's elements (``runs``: already computed for ``ops``,
        # from rank_runs with the tensors largest first and the running total
        # of their elements in that order)
        r = runs if runs is not None else _lib.host().name_runs(self.ops)
        self.order, self.starts, numel = r[:3]
        self.n = len(numel)
        scale = 2.0 * elem_bytes / GATHER_BYTES_PER_NS           # GPU ns per element
        if scale > 0:
            if len(r) > 7:
                self.rank, total = r[6], r[7]
            else:
                self.rank = np.argsort(-numel, kind="stable")   # largest first
                total = np.cumsum(numel[self.rank]).tolist()
            self._cum = [t * scale for t in total]               # GPU ns of the first k tensors
        else:
            self.rank = np.arange(self.n, dtype=np.int64)
            self._cum = [0.0] * self.n
        self.plan_ns = float(PLAN_NS_PER_TENSOR)                 # per destination tensor

    def _gpu(self, a: int, b: int) -> float:
        return self._cum[b - 1] - (self._cum[a - 1] if a else 0.0)

    @property
    def launch_order(self) -> np.ndarray:
        """Tensor indices in the order the groups hold them: largest first,
        or order of first appearance when the transfer is not cut."""
        if self.pipeline <= 1 or self.n <= 1:
            return np.arange(self.n, dtype=np.int64)
        return self.rank

    def _take(self, a: int, b: int) -> List[TransferOp]:
        return _lib.host().take_ops(self.ops, self.order, self.starts, self.rank[a:b])

    def _next_end(self, start: int, end: int, groups: int) -> int:
        """End of the group after [start, end), the group number `groups`."""
        if groups >= self.pipeline:
            return self.n
        per_tensor = self.plan_ns * self.per_name
        fits = (self._gpu(start, end) * PLAN_SHARE - PLAN_NS_PER_GROUP) / per_tensor
        if fits < MIN_GROUP_TENSORS:
            return self.n
        nxt = min(self.n, end + int(fits))
        # a group that is not the last pays its planning overhead back only
        # if the GPU runs it at least that long (while the host plans on)
        if nxt < self.n and self._gpu(end, nxt) < PLAN_NS_PER_GROUP:
            return self.n
        return nxt

    def __iter__(self):
        if self.pipeline <= 1 or self.n <= 1:
            yield self.ops
            return
        end = min(self.n, bisect.bisect_left(self._cum, FIRST_GROUP_NS) + 1)
        start, groups = 0, 1
        while True:
            t0 = _clock_ns()
            yield self._take(start, end)
            spent = _clock_ns() - t0
            if end >= self.n:
                return
            names = end - start
            if names >= MIN_GROUP_TENSORS:
                self.plan_ns = max(float(MIN_PLAN_NS_PER_TENSOR),
                                   (spent - PLAN_NS_PER_GROUP) / (names * self.per_name))
            start, end = end, self._next_end(start, end, groups + 1)
            groups += 1

    def cut(self) -> List[List[TransferOp]]:
        """All groups at once, at the prior planning rate (no timing)."""
        if self.pipeline <= 1 or self.n <= 1:
            return [self.ops]
        bounds = [0, min(self.n, bisect.bisect_left(self._cum, FIRST_GROUP_NS) + 1)]
        while bounds[-1] < self.n:
            bounds.append(self._next_end(bounds[-2], bounds[-1], len(bounds)))
        return [self._take(a, b) for a, b in zip(bounds[:-1], bounds[1:])]


def _pipeline_groups(ops: List[TransferOp], elem_bytes: int, pipeline: int,
                     tensors_per_name: int = 1, runs=None):
    """The launch groups of ``ops`` (an iterable of op lists, see
    ``_LaunchGroups``)."""
    return _LaunchGroups(ops, elem_bytes, pipeline, tensors_per_name, runs)


def schedule_and_execute_param_transfer(
    source_param_layout: ParamLayout,
    target_param_layout: ParamLayout,
    source_state_dict: StateDict,
    other_context_dict: Dict[str, Any],
    device: torch.device,
    world: Optional[dist.ProcessGroup],
    prof,
    forcefully_free: bool,
    log_func=None,
    **kwargs,
) -> StateDict:
    """Schedule + execute + synchronize (Suika/migration.py:558-598)."""
    if not isinstance(device, torch.device):
        device = torch.device(device)
    if prof is None:
        prof = _NoProf()
    prof.start("schedule")
    schedule = schedule_param_transfer(source_param_layout, target_param_layout)
    prof.stop("schedule")
    prof.start("execute")
    target = execute_param_transfer(
        transfer_ops=schedule, source_state_dict=source_state_dict, device=device,
        expected_sub_fields=other_context_dict["expected_sub_fields"], world=world,
        forcefully_free=forcefully_free, prof=prof, log_func=log_func, **kwargs)
    if device.type == "cuda":
        torch.cuda.synchronize(device=device)
    prof.stop("execute")
    return target


def merge_model_and_optimizer_state_dict(model: Module, optimizer: Optional[Optimizer],
                                         other_context: Optional[Any]) -> Tuple[Dict, Dict]:
    """{name: {"param", **optimizer.state[idx]}} plus the sub-field list
    (Suika/migration.py:675-711)."""
    model_state_dict = model.state_dict()
    if optimizer:
        osd = optimizer.state_dict()
        other_context_dict = {"other_context": other_context, "param_groups": osd["param_groups"]}
        opt_state = osd["state"]
    else:
        opt_state = {}
        other_context_dict = {"other_context": other_context}
    merged: Dict[str, Dict[str, Tensor]] = {}
    for idx, (name, _) in enumerate(get_named_parameters_and_persistent_buffers(model)):
        entry = {"param": model_state_dict[name]}
        entry.update(opt_state.get(idx, {}))
        merged[name] = entry
        if "expected_sub_fields" not in other_context_dict:
            other_context_dict["expected_sub_fields"] = [
                (f, TensorMeta(t) if t.numel() == 1 else "normal") for f, t in entry.items()]
    return merged, other_context_dict


def split_model_and_optimizer_state_dict(model: Module, merged_state_dict: Dict[str, Dict[str, Tensor]],
                                         other_context_dict: Dict[str, Any]) -> Tuple[Dict, Dict, Any]:
    """Inverse of the merge, re-indexed by the new model's order
    (Suika/migration.py:722-746)."""
    model_state_dict = {}
    by_name = {}
    for name, entry in merged_state_dict.items():
        model_state_dict[name] = entry["param"]
        del entry["param"]
        by_name[name] = entry
    by_index = {idx: by_name[name]
                for idx, (name, _) in enumerate(get_named_parameters_and_persistent_buffers(model))}
    optimizer_state_dict = {"state": by_index,
                            "param_groups": other_context_dict.get("param_groups", None)}
    return model_state_dict, optimizer_state_dict, other_context_dict["other_context"]

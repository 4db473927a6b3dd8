"""Live state migration between processes on one GPU.

Suika's ``migration_save`` / ``migration_load`` (Suika/migration.py:1357-1727)
hand a job's model and optimizer state from the processes of its old plan to
the processes of its new plan.  The two sets of processes run side by side;
each guard process owns a pair of queues shared by its old and new rank
(``IPC_queues``: forward, backward).  The reference moves every tensor through
the queue as a CUDA-IPC handle, one acknowledgement each, clones it on the
receiving side, and reshards over NCCL in the old world (scale-down) or the
new one (scale-up) (Suika/utils.py:325-406).

Here, with every old and new rank on the same GPU:

* the handshake on world sizes is the reference's (rank 0 of each side, over
  the queues, :1395-1405 / :1587-1598);
* each old rank packs its merged state (``merge_model_and_optimizer_state_dict``)
  into a few device allocations of its own with one gather launch, exports
  them (``sr_handoff_alloc``, at most 1 GiB each, always below 2 GiB), and the
  old world all-gathers the export records (handles, offsets, shapes: CPU
  objects);
* old rank ``i`` sends the source layout, the context and every old rank's
  record to new rank ``i`` over its forward queue; new ranks without an old
  counterpart read the launcher's placeholder (``dummy_migration_IPC_state_dict``),
  and the new world takes rank 0's message;
* each new rank maps the allocations of the old ranks its pieces come from
  (``sr_handoff_open``) and views the state there as tensors without copying;
* the new world sums its destination bytes.  When the device has room for
  them beside the old state and the hand-off (its 288 GiB of HBM hold all
  three for a 7B model's fp32 Adam state), every new rank takes that memory
  and new rank 0 sends ``ALLOCATED``; otherwise it sends ``WANT_RELEASED``
  and waits for ``RELEASED``;
* only then does each old rank free its state tensors, as the reference frees
  each sent tensor, and return the memory to the device (memory another
  process has just freed is slow to allocate); once all have, old rank 0
  sends ``RELEASED``;
* each new rank runs ``execute_param_transfer`` (one gather per launch group)
  straight from the mapped memory into one destination arena that the model
  adopts with ``load_state_dict(assign=True)``, beside the old state's
  release when the memory allowed it, and builds its optimizer;
* new rank 0, holding ``RELEASED``, acknowledges on rank 0's backward queue
  and the new world returns; the old world then frees the hand-off
  allocations and returns.

The packed allocations are the per-peer buffers of a pack -> unpack reshard:
the old side reads and writes P bytes, the new side reads P and writes D, and
nothing is cloned tensor by tensor.  The scale-up / scale-down distinction of
the reference only decides which world reshards; here the new world always
does, reading from the mapped memory.
"""
from __future__ import annotations

import ctypes
import threading
import time
from collections import OrderedDict
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple

import torch
import torch.distributed as dist
from torch import Tensor

from . import _lib

# Bytes per hand-off allocation the packer fills before it opens the next;
# a single larger tensor gets an allocation of its own (below 2 GiB).
CHUNK_BYTES = 1 << 30
ALIGN = 256

# What the launcher puts on a new guard's forward queue when no old process
# exists (Suika/migration.py:1314-1318, training.py:319-323): migration_load
# then finds no source layout and returns without state.
dummy_migration_IPC_state_dict = {
    "source_param_layout": None,
    "source_state_dict": {},
    "other_context_dict": {},
}

DONE = "suika_amd: handoff complete"
# New rank 0 to old rank 0 once every new rank has mapped the hand-off: either
# every new rank holds the memory for its destinations (ALLOCATED), or the
# device lacks room for them beside the old state (WANT_RELEASED).  The old
# ranks release their state only then, so memory they free is not what the
# new ranks allocate at once.
ALLOCATED = "suika_amd: destinations allocated"
WANT_RELEASED = "suika_amd: waiting for the old state's release"
# Old rank 0 to new rank 0, after either note: every old rank has released
# its state and returned the memory to the device.
RELEASED = "suika_amd: old state released"
# Device memory kept free per new rank beyond its destinations when they are
# allocated beside the old state (plan tables, allocator rounding).
HEADROOM_BYTES = 1 << 30
# Taken beyond a new rank's destination bytes when it reserves them.
ARENA_SLACK_BYTES = 64 << 20


def pack_layout(nbytes: Sequence[int], chunk_bytes: int = CHUNK_BYTES) -> Tuple[List[Tuple[int, int]], List[int]]:
    """(chunk, byte offset) of every tensor of ``nbytes`` bytes, in order, and
    the size of every chunk: tensors follow each other at 256-byte aligned
    offsets until the next would pass ``chunk_bytes``; a tensor larger than
    that gets a chunk of its own.  No chunk exceeds the hand-off limit."""
    where: List[Tuple[int, int]] = []
    sizes: List[int] = []
    for n in nbytes:
        assert 0 < n <= _lib.HANDOFF_MAX_BYTES, \
            f"a tensor of {n} bytes does not fit one hand-off allocation ({_lib.HANDOFF_MAX_BYTES} bytes)"
        off = (sizes[-1] + ALIGN - 1) // ALIGN * ALIGN if sizes else 0
        if sizes and off + n <= chunk_bytes:
            sizes[-1] = off + n
        else:
            sizes.append(n)
            off = 0
        where.append((len(sizes) - 1, off))
    return where, sizes


def _dtype_of(name: str) -> torch.dtype:
    dt = getattr(torch, name.replace("torch.", ""), None)
    assert isinstance(dt, torch.dtype), f"unknown dtype {name}"
    return dt


class Handoff:
    """An old rank's merged state packed into exported device allocations.

    ``state`` is ``{name: {field: tensor}}``.  Non-empty tensors on
    ``device`` are packed, in order, at 256-byte aligned offsets into
    allocations of at most ``chunk_bytes`` (a larger tensor gets one of its
    own); every other value (CPU tensors such as AdamW's ``step``, empty
    tensors) rides along in the record as a CPU tensor.  The copies are done
    when the constructor returns.
    """

    def __init__(self, state: Dict[str, Dict[str, Tensor]], device: torch.device, rank: int,
                 chunk_bytes: int = CHUNK_BYTES):
        L = self._L = _lib.lib()
        self.rank = rank
        self.device = device
        self._ptrs: List[int] = []
        moved: List[Tuple[str, str, Tensor]] = []
        self.tensors: Dict[str, Dict[str, tuple]] = {}
        self.host: Dict[str, Dict[str, Tensor]] = {}
        for name, entry in state.items():
            for f, t in entry.items():
                if not (isinstance(t, Tensor) and t.is_cuda and t.device == device and t.numel() > 0):
                    self.host.setdefault(name, {})[f] = t.detach().cpu() if isinstance(t, Tensor) else t
                    continue
                assert t.is_contiguous(), f"handoff: {name}/{f} is not contiguous"
                moved.append((name, f, t))
        where, sizes = pack_layout([t.numel() * t.element_size() for _, _, t in moved], chunk_bytes)
        packed = [(name, f, t, c, off) for (name, f, t), (c, off) in zip(moved, where)]
        for name, f, t, c, off in packed:
            self.tensors.setdefault(name, {})[f] = (c, off, tuple(t.shape), str(t.dtype))
        self.chunks: List[Tuple[bytes, int]] = []
        try:
            with torch.cuda.device(device):
                for n in sizes:
                    ptr, handle = ctypes.c_void_p(), _lib.SrIpcHandle()
                    _lib.check(L.sr_handoff_alloc(n, ctypes.byref(ptr), ctypes.byref(handle)), "sr_handoff_alloc", L)
                    self._ptrs.append(ptr.value)
                    self.chunks.append((bytes(handle.bytes), n))
                if packed:
                    self._pack(packed, sizes)
        except BaseException:
            self.release()
            raise
        self.bytes = sum(sizes)

    def _pack(self, packed, sizes) -> None:
        """One gather launch: every tensor, as bytes, to its chunk offset."""
        import numpy as np
        L = self._L
        src = np.zeros(len(packed), dtype=_lib.SR_TENSOR_DTYPE)
        dst = np.zeros(len(sizes), dtype=_lib.SR_TENSOR_DTYPE)
        pieces = np.zeros(len(packed), dtype=_lib.SR_PIECE_DTYPE)
        for i, (_, _, t, chunk, off) in enumerate(packed):
            nbytes = t.numel() * t.element_size()
            src[i] = (1, nbytes, _lib.SR_DT_U8, 0)
            pieces[i] = (_lib.SR_PIECE_COPY, 0, i, chunk, -1, 0, 1, nbytes, 0, 0, 0, off)
        for c, n in enumerate(sizes):
            dst[c] = (1, n, _lib.SR_DT_U8, 0)
        opts = _lib.SrPlanOptions(0, 0, _lib.SR_OPT_SKIP_COVERAGE, 0)
        plan = ctypes.c_void_p()
        _lib.check(L.sr_plan_create(_lib.as_tensors(src), len(src), _lib.as_tensors(dst), len(dst), 1,
                                    _lib.as_pieces(pieces), len(pieces), ctypes.byref(opts), ctypes.byref(plan)),
                   "handoff pack: sr_plan_create", L)
        try:
            vp = ctypes.c_void_p
            sp = (vp * len(packed))(*[t.data_ptr() for _, _, t, _, _ in packed])
            dp = (vp * len(sizes))(*self._ptrs)
            stream = torch.cuda.current_stream(self.device)
            _lib.check(L.sr_gather(plan, sp, dp, vp(stream.cuda_stream)), "handoff pack: sr_gather", L)
            stream.synchronize()
        finally:
            L.sr_plan_destroy(plan)

    def record(self) -> Dict[str, Any]:
        """What a new rank needs to map and view this state (CPU objects)."""
        return {"rank": self.rank, "device": self.device.index, "chunks": list(self.chunks),
                "tensors": self.tensors, "host": self.host}

    def release(self) -> None:
        """Free the allocations (after every new rank has closed them)."""
        L = self._L
        with torch.cuda.device(self.device):
            while self._ptrs:
                _lib.check(L.sr_handoff_free(ctypes.c_void_p(self._ptrs.pop())), "sr_handoff_free", L)


class MappedSources:
    """Old ranks' packed state mapped into this process: ``states`` is
    ``{old rank: {name: {field: tensor}}}``, tensors viewing the mapped
    allocations (no copy); CPU values of the records ride along.  ``close``
    unmaps them; the views must be dropped first."""

    def __init__(self, records: Sequence[Dict[str, Any]], ranks: Sequence[int], device: torch.device):
        L = self._L = _lib.lib()
        self.device = device
        self._opened: List[int] = []
        self.states: Dict[int, Dict[str, Dict[str, Tensor]]] = {}
        by_rank = {rec["rank"]: rec for rec in records}
        host = _lib.host()
        try:
            with torch.cuda.device(device):
                for r in ranks:
                    rec = by_rank[r]
                    assert rec["device"] == device.index, \
                        f"rank {r}'s state is on cuda:{rec['device']}, this rank runs on {device}"
                    bases = []
                    for handle, _ in rec["chunks"]:
                        h = _lib.SrIpcHandle()
                        ctypes.memmove(h.bytes, handle, len(handle))
                        ptr = ctypes.c_void_p()
                        _lib.check(L.sr_handoff_open(ctypes.byref(h), ctypes.byref(ptr)), "sr_handoff_open", L)
                        self._opened.append(ptr.value)
                        bases.append(ptr.value)
                    state: Dict[str, Dict[str, Tensor]] = {}
                    keys = [(n, f) for n, e in rec["tensors"].items() for f in e]
                    per_chunk: Dict[int, List[Tuple[str, str]]] = {}
                    for n, f in keys:
                        per_chunk.setdefault(rec["tensors"][n][f][0], []).append((n, f))
                    for c, members in per_chunk.items():
                        views = [(rec["tensors"][n][f][1], list(rec["tensors"][n][f][2]),
                                  _dtype_of(rec["tensors"][n][f][3])) for n, f in members]
                        for (n, f), t in zip(members, host.device_views(bases[c], views, device.index)):
                            state.setdefault(n, {})[f] = t
                    for n, e in rec["host"].items():
                        for f, v in e.items():
                            state.setdefault(n, {})[f] = v
                    self.states[r] = state
        except BaseException:
            self.states = {}
            self.close()
            raise

    def close(self) -> None:
        L = self._L
        self.states = {}
        with torch.cuda.device(self.device):
            while self._opened:
                _lib.check(L.sr_handoff_close(ctypes.c_void_p(self._opened.pop())), "sr_handoff_close", L)


def _broadcast_objects(*objs, group=None):
    """Rank 0's objects on every rank of ``group`` (Suika/utils.py:98-104)."""
    lst = list(objs)
    src = 0 if group is None else dist.get_global_rank(group, 0)
    dist.broadcast_object_list(lst, src=src, group=group)
    return lst[0] if len(lst) == 1 else lst


def live_save(IPC_queues, model, optimizer, other_context, device: torch.device, world,
              log_func: Callable[[str], None]) -> None:
    """The old side of a live migration (Suika/migration.py:1394-1486)."""
    from .meta import ParamLayout
    from .migration import forcefully_free_tensor, merge_model_and_optimizer_state_dict

    rank = dist.get_rank(world)
    # the library's first-use costs are paid while the new world starts
    warm = _WarmUp(device, optimizer=False)
    warm.start()
    if rank == 0:
        old_world_size = dist.get_world_size(world)
        IPC_queues[0].put(old_world_size)
        new_world_size = IPC_queues[1].get(block=True)
        is_scale_up = new_world_size >= old_world_size
    else:
        is_scale_up = new_world_size = None
    is_scale_up, new_world_size = _broadcast_objects(is_scale_up, new_world_size, group=world)
    log_func(f"migration_save: is_scale_up = {is_scale_up} (new world size {new_world_size})")
    warm.join()

    param_layout = ParamLayout()
    param_layout.gather(model, world)
    source_state_dict, other_context_dict = merge_model_and_optimizer_state_dict(model, optimizer, other_context)

    t0 = time.perf_counter()
    handoff = Handoff(source_state_dict, device, rank)
    t1 = time.perf_counter()
    log_func(f"migration_save: packed {handoff.bytes / 1e9:.3f} GB into {len(handoff.chunks)} hand-off "
             f"allocation(s) in {(t1 - t0) * 1e3:.2f} ms")
    try:
        records = [None] * dist.get_world_size(world)
        dist.all_gather_object(records, handoff.record(), group=world)
        log_func(f"migration_save: {len(records)} hand-off record(s) gathered")
        if rank < new_world_size:
            IPC_queues[0].put({"source_param_layout": param_layout, "source_state_dict": {},
                               "other_context_dict": other_context_dict, "handoff": records})
            log_func("migration_save: hand-off sent to the new rank")
        # The state now lives in the hand-off allocations: release it, as the
        # reference releases every tensor it has sent (utils.py:372-376), and
        # return the memory to the device for the new world, as its cuda_gc
        # does after sending (utils.py:248-253, 385) -- once the new world
        # has mapped the hand-off and either allocated its destinations
        # beside this state or asked for the memory.
        note = IPC_queues[1].get(block=True) if rank == 0 else None
        note = _broadcast_objects(note, group=world)
        assert note in (ALLOCATED, WANT_RELEASED), f"migration_save: unexpected message {note!r}"
        log_func("migration_save: the new world " + ("has allocated its destinations" if note == ALLOCATED
                                                     else "waits for this state's memory"))
        t2 = time.perf_counter()
        for entry in source_state_dict.values():
            for t in entry.values():
                if isinstance(t, Tensor) and t.is_cuda:
                    forcefully_free_tensor(t)
        del source_state_dict
        t3 = time.perf_counter()
        torch.cuda.empty_cache()
        t4 = time.perf_counter()
        log_func(f"migration_save: state released ({(t3 - t2) * 1e3:.2f} ms), device memory returned "
                 f"({(t4 - t3) * 1e3:.2f} ms)")
        dist.barrier(world)
        # the new world maps these allocations until it has resharded
        if rank == 0:
            IPC_queues[0].put(RELEASED)
            ack = IPC_queues[1].get(block=True)
            assert ack == DONE, f"migration_save: unexpected acknowledgement {ack!r}"
        dist.barrier(world)
        log_func("migration_save: the new world is done with the hand-off")
    finally:
        handoff.release()
    log_func("migration_save: end")


class _WarmUp(threading.Thread):
    """First-use costs of a fresh process of a migration, paid on a thread
    while it waits: in a live migration the old ranks for the new world's
    handshake and the new ranks for the old world's message; in
    ``checkpoint_load`` while the files are read:

    * the reshard library's: ``sr_prepare`` loads its GPU code and sets up
      its streams and the runtime's copy path, and one tiny gather warms
      the drop-in call's host side.  With twelve processes on one MI355X
      these took 30-57 ms per first launch, 40-54 ms per first table upload
      and 26 ms for the setup stream, inside the pack and the reshard;
    * with an optimizer to build, torch.optim's: a process's first optimizer
      imports torch's compiler front end (torch._dynamo, about 0.4 s).

    ``library_done`` is set once the library is no longer in use here; the
    caller waits for it before its own library calls and joins the thread
    before building its optimizer.  Failures are ignored: the real calls
    report their own."""

    def __init__(self, device: torch.device, optimizer: bool):
        super().__init__(name="suika-warm-up", daemon=True)
        self.device = device
        self.optimizer = optimizer
        self.library_done = threading.Event()

    def run(self) -> None:
        try:
            from .meta import TensorMeta, TransferOp
            from .migration import execute_param_transfer
            with torch.cuda.device(self.device):
                stream = torch.cuda.current_stream(self.device).cuda_stream
                _lib.lib().sr_prepare(ctypes.c_void_p(stream))
                meta = TensorMeta(name="warm-up", dtype=torch.float32, shape=(64,))
                src = {0: {"warm-up": {"param": torch.zeros(64, device=self.device)}}}
                execute_param_transfer([TransferOp("warm-up", 0, 0, meta, meta)], {}, self.device,
                                       [("param", "normal")], rank=0, fake_source_state_dicts=src)
                torch.cuda.synchronize(self.device)
        except Exception:
            pass
        finally:
            self.library_done.set()
        if self.optimizer:
            try:
                torch.optim.SGD([torch.nn.Parameter(torch.zeros(1))], lr=0.0)
            except Exception:
                pass


def _destination_bytes(ops, rank: int, records: Sequence[Dict[str, Any]]) -> int:
    """Device bytes of ``rank``'s destination tensors: per name, the elements
    of its shard on this rank times the item sizes of the fields the old
    ranks' hand-off records hold on the device, each tensor rounded up to
    256 bytes."""
    by_rank = {rec["rank"]: rec for rec in records}
    per_name: Dict[str, int] = {}
    for op in ops:
        if op.dst_rank != rank or op.param_name in per_name:
            continue
        numel = 1
        for d in op.dst_shard_meta.actual_shape():
            numel *= int(d)
        fields = by_rank[op.src_rank]["tensors"].get(op.param_name, {})
        per_name[op.param_name] = sum((numel * _dtype_of(f[3]).itemsize + ALIGN - 1) // ALIGN * ALIGN
                                      for f in fields.values())
    return sum(per_name.values())


def live_load(IPC_queues, model, optimizer_provider, optimizer, device: torch.device, world,
              log_func: Callable[[str], None], wait_for_release: Optional[bool] = None):
    """The new side of a live migration (Suika/migration.py:1586-1727).

    The destinations are allocated beside the old state when the device has
    room for every new rank's (``wait_for_release=None``), else after the old
    world has released its state; ``True`` always waits."""
    from .meta import ParamLayout, schedule_param_transfer
    from .migration import execute_param_transfer, split_model_and_optimizer_state_dict

    rank = dist.get_rank(world)
    # the process's first-use costs are paid while it waits for the old world
    warm = _WarmUp(device, optimizer_provider is not None)
    warm.start()
    if rank == 0:
        old_world_size = IPC_queues[0].get(block=True)
        new_world_size = dist.get_world_size(world)
        if old_world_size != 0:
            IPC_queues[1].put(new_world_size)
        is_scale_up = new_world_size >= old_world_size
    else:
        is_scale_up = None
    is_scale_up = _broadcast_objects(is_scale_up, group=world)
    log_func(f"migration_load: is_scale_up = {is_scale_up}")

    target_param_layout = ParamLayout()
    target_param_layout.gather(model, world)
    # old rank i's message, or the launcher's placeholder when there is none
    msg = IPC_queues[0].get(block=True)
    log_func("migration_load: hand-off message received")
    source_param_layout, other_context_dict, records = _broadcast_objects(
        msg.get("source_param_layout"), msg.get("other_context_dict"), msg.get("handoff"), group=world)
    del msg

    if source_param_layout is None:
        log_func("migration_load: no checkpoint received; skip loading")
        if hasattr(model, "instantiate") and getattr(model, "on_meta", False):
            model.instantiate()
        warm.join()
        return (optimizer_provider(), None) if optimizer_provider else None

    t0 = time.perf_counter()
    ops = schedule_param_transfer(source_param_layout, target_param_layout)
    needed = sorted({op.src_rank for op in ops if op.dst_rank == rank})
    t_sched = time.perf_counter()
    # Old state, hand-off and destinations side by side when the device has
    # room for all of them: each new rank takes its destinations' memory
    # before the old world frees anything.  Else the destinations wait for
    # the old world to return its state's memory.
    mine = _destination_bytes(ops, rank, records)
    need = torch.tensor([mine], dtype=torch.int64)
    dist.all_reduce(need, group=world)
    wait = None
    if rank == 0:
        free, _ = torch.cuda.mem_get_info(device)
        room = int(need.item()) + HEADROOM_BYTES * dist.get_world_size(world)
        wait = bool(wait_for_release) if wait_for_release is not None else free < room
    wait = _broadcast_objects(wait, group=world)
    if not wait:
        # the destination arena's memory, taken now and kept in this
        # process's allocator cache, where the arena finds it
        torch.empty(mine + ARENA_SLACK_BYTES, dtype=torch.uint8, device=device)
    t_alloc = time.perf_counter()
    # mapped before the old world frees anything: IPC opens beside other
    # processes' frees were 20-40x slower
    mapped = MappedSources(records, needed, device)
    t_map = time.perf_counter()
    log_func(f"migration_load: mapped the state of old rank(s) {needed}")
    try:
        dist.barrier(world)
        if rank == 0:
            IPC_queues[1].put(WANT_RELEASED if wait else ALLOCATED)
        warm.library_done.wait()
        if wait:
            if rank == 0:
                note = IPC_queues[0].get(block=True)
                assert note == RELEASED, f"migration_load: unexpected message {note!r}"
            dist.barrier(world)
        log_func(f"migration_load: destinations of {int(need.item()) / 1e9:.3f} GB "
                 + ("after the old world released its state" if wait else "beside the old state"))
        t1 = time.perf_counter()
        target_state_dict = execute_param_transfer(
            transfer_ops=ops, source_state_dict={}, device=device,
            expected_sub_fields=other_context_dict["expected_sub_fields"], world=world,
            fake_source_state_dicts=mapped.states, log_func=log_func, rank=rank, arena=True)
        torch.cuda.synchronize(device)
        t2 = time.perf_counter()
    finally:
        mapped.close()
    log_func(f"migration_load: scheduled in {(t_sched - t0) * 1e3:.2f} ms, "
             + ("" if wait else f"destinations' memory taken in {(t_alloc - t_sched) * 1e3:.2f} ms, ")
             + f"mapped {len(needed)} old rank(s) in {(t_map - t_alloc) * 1e3:.2f} ms, "
             f"resharded in {(t2 - t1) * 1e3:.2f} ms")
    dist.barrier(world)
    log_func("migration_load: every new rank has resharded")

    model_state_dict, optimizer_state_dict, other_context = split_model_and_optimizer_state_dict(
        model=model, merged_state_dict=target_state_dict, other_context_dict=other_context_dict)
    model_state_dict = OrderedDict(sorted(model_state_dict.items(), key=lambda x: x[0]))
    model.load_state_dict(model_state_dict, assign=True)
    log_func("migration_load: model state adopted")
    warm.join()
    if optimizer_provider:
        optimizer = optimizer_provider()
    if optimizer:
        # one parameter group, as the reference (migration.py:1712-1716)
        optimizer_state_dict["param_groups"][0]["params"] = optimizer.state_dict()["param_groups"][0]["params"]
        optimizer.load_state_dict(optimizer_state_dict)
    # the old world's state released (beside which the destinations may have
    # been allocated) before any new rank returns; then the old world may
    # free the hand-off
    if rank == 0:
        if not wait:
            note = IPC_queues[0].get(block=True)
            assert note == RELEASED, f"migration_load: unexpected message {note!r}"
        IPC_queues[1].put(DONE)
    dist.barrier(world)
    log_func("migration_load: end")
    return (optimizer, other_context) if optimizer_provider else other_context

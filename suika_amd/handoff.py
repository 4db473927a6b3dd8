"""Live state migration between processes on one GPU.

Suika's ``migration_save`` / ``migration_load`` (Suika/migration.py:1357-1727)
hand a job's model and optimizer state from the processes of its old plan to
the processes of its new plan.  The two sets of processes run side by side;
each guard process owns a pair of queues shared by its old and new rank
(``IPC_queues``: forward, backward).  The reference moves every tensor through
the queue as a CUDA-IPC handle, one acknowledgement each, clones it on the
receiving side, frees it on the sending side once acknowledged (collecting
the cache every 1 GiB sent), and reshards over NCCL in the old world
(scale-down) or the new one (scale-up) (Suika/utils.py:325-406).

Here, with every old and new rank on the same GPU, the handshake on world
sizes is the reference's (rank 0 of each side, over the queues, :1395-1405 /
:1587-1598).  Then the old world sums the bytes it holds on the device and
old rank 0 picks one of two orders from the device's free memory:

**Whole** (the hand-off fits beside the old state):

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
  sends ``RELEASED`` when the new world waits for it;
* each new rank runs ``execute_param_transfer`` (one gather per launch group)
  straight from the mapped memory into one destination arena that the model
  adopts with ``load_state_dict(assign=True)``, beside the old state's
  release when the memory allowed it; new rank 0 then sends ``DONE`` and the
  old world frees the hand-off allocations;
* the new world builds its optimizer and returns: by default once ``RELEASED``
  has come (the device is then the new world's alone), or at once with
  ``return_before_release`` (the reference's order: its new processes return
  after their own receive and reshard).

**Waves** (it does not: the device holds less than twice the state).  Names
are cut into waves of at most a third of the free memory, in the same order
on every old rank; a name's tensors on every old rank move in one wave, so a
wave is a self-contained reshard.  Each old rank allocates two hand-off
slots once (the ring), each as large as its largest wave needs, when every
rank's slots fit the room; else each wave gets allocations of its own.  For
each wave the old ranks pack its tensors into slot ``k mod 2``, free them and
return their memory (the reference's per-tensor free and periodic
``cuda_gc``), and only then does old rank 0 send the wave's records; the new
ranks map the slots (once each), reshard that wave into an arena of its own
and report it consumed.  The old world packs wave ``k + 1`` while the new
world reshards wave ``k``, so the device holds the state plus the ring (or
plus at most two waves without it).

Every step at which one rank may fail ends in an exchange of errors within
its world, so a failure raises on every rank of that world instead of
leaving the others in their next collective; the world that failed sends
``(ERROR, text)`` on the queue the other world reads next, and every queue
read has a time limit (``QUEUE_TIMEOUT_S``).  A world that sent records
releases their memory only after the other world has closed its mappings
(it reported the wave consumed, said ``DONE`` or failed).

The packed allocations are the per-peer buffers of a pack -> unpack reshard:
the old side reads and writes P bytes, the new side reads P and writes D, and
nothing is cloned tensor by tensor.  The scale-up / scale-down distinction of
the reference only decides which world reshards; here the new world always
does, reading from the mapped memory.
"""
from __future__ import annotations

import ctypes
import queue
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

# New rank 0 to old rank 0 once the new world has resharded: the hand-off
# allocations are no longer mapped.
DONE = "suika_amd: handoff complete"
# New rank 0 to old rank 0 once every new rank has mapped the hand-off (sent
# as {"note": ..., "await_release": bool}): either every new rank holds the
# memory for its destinations (ALLOCATED), or the device lacks room for them
# beside the old state (WANT_RELEASED).  The old ranks release their state
# only then, so memory they free is not what the new ranks allocate at once.
ALLOCATED = "suika_amd: destinations allocated"
WANT_RELEASED = "suika_amd: waiting for the old state's release"
# Old rank 0 to new rank 0, when the note asked for it: every old rank has
# released its state and returned the memory to the device.
RELEASED = "suika_amd: old state released"
# (ERROR, text) on either queue: the sending world failed; the reader raises.
ERROR = "suika_amd: handoff failed"
# Time limit of every queue read of the protocol, in seconds.
QUEUE_TIMEOUT_S = 600.0
# Device memory kept free per new rank beyond its destinations when they are
# allocated beside the old state: plan tables, allocator rounding, and the
# library's 64 MiB static scratch array, which its code object places on the
# device in every process that loads it (old and new ranks alike).
HEADROOM_BYTES = 1 << 30
# Taken beyond a new rank's destination bytes when it reserves them.
ARENA_SLACK_BYTES = 64 << 20
# Per process of either world, left out of the memory the waves may use:
# the same per-process costs at the granularity one wave adds them.
RESERVE_BYTES = 96 << 20
# Waves reuse two hand-off slots allocated once (the ring) when they fit;
# False gives every wave allocations of its own.
USE_RING = True


class HandoffError(RuntimeError):
    """A live migration failed; every process of the failing world raises
    it, and so does every process of the other world that was waiting on it.
    ``notify``: the other world has not been told yet."""

    def __init__(self, msg: str, notify: bool = True):
        super().__init__(msg)
        self.notify = notify


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


def _moved(state: Dict[str, Dict[str, Any]], device: torch.device):
    """(name, field, tensor) of every non-empty tensor on ``device``, in
    order, and every other value as (name, field, value)."""
    moved: List[Tuple[str, str, Tensor]] = []
    other: List[Tuple[str, str, Any]] = []
    for name, entry in state.items():
        for f, t in entry.items():
            if isinstance(t, Tensor) and t.is_cuda and t.device == device and t.numel() > 0:
                moved.append((name, f, t))
            else:
                other.append((name, f, t))
    return moved, other


def layout_of(state: Dict[str, Dict[str, Any]], device: torch.device,
              chunk_bytes: int = CHUNK_BYTES) -> List[int]:
    """The chunk sizes ``Handoff`` packs ``state`` into."""
    moved, _ = _moved(state, device)
    return pack_layout([t.numel() * t.element_size() for _, _, t in moved], chunk_bytes)[1]


class Slot:
    """Exported device allocations of given sizes that several hand-offs
    pack into one after the other (the waves' ring); ``free`` releases
    them."""

    def __init__(self, sizes: Sequence[int], device: torch.device):
        L = self._L = _lib.lib()
        self.device = device
        self.chunks: List[Tuple[bytes, int]] = []
        self.ptrs: List[int] = []
        try:
            with torch.cuda.device(device):
                for n in sizes:
                    ptr, handle = ctypes.c_void_p(), _lib.SrIpcHandle()
                    _lib.check(L.sr_handoff_alloc(n, ctypes.byref(ptr), ctypes.byref(handle)), "sr_handoff_alloc", L)
                    self.ptrs.append(ptr.value)
                    self.chunks.append((bytes(handle.bytes), n))
        except BaseException:
            self.free()
            raise

    def free(self) -> None:
        L = self._L
        with torch.cuda.device(self.device):
            while self.ptrs:
                _lib.check(L.sr_handoff_free(ctypes.c_void_p(self.ptrs.pop())), "sr_handoff_free", L)
        self.chunks = []


class Handoff:
    """An old rank's merged state packed into exported device allocations.

    ``state`` is ``{name: {field: tensor}}``.  Non-empty tensors on
    ``device`` are packed, in order, at 256-byte aligned offsets into
    allocations of at most ``chunk_bytes`` (a larger tensor gets one of its
    own); every other value (CPU tensors such as AdamW's ``step``, empty
    tensors) rides along in the record as a CPU tensor.  With ``slot`` the
    tensors go into that slot's allocations (each chunk at least as large as
    this state's layout needs), which the hand-off does not own; otherwise
    it allocates its own.  The copies are done when the constructor
    returns.
    """

    def __init__(self, state: Dict[str, Dict[str, Tensor]], device: torch.device, rank: int,
                 chunk_bytes: int = CHUNK_BYTES, slot: Optional[Slot] = None):
        L = self._L = _lib.lib()
        self.rank = rank
        self.device = device
        self._ptrs: List[int] = []
        self.tensors: Dict[str, Dict[str, tuple]] = {}
        self.host: Dict[str, Dict[str, Tensor]] = {}
        moved, other = _moved(state, device)
        for name, f, t in other:
            self.host.setdefault(name, {})[f] = t.detach().cpu() if isinstance(t, Tensor) else t
        for name, f, t in moved:
            assert t.is_contiguous(), f"handoff: {name}/{f} is not contiguous"
        where, sizes = pack_layout([t.numel() * t.element_size() for _, _, t in moved], chunk_bytes)
        packed = [(name, f, t, c, off) for (name, f, t), (c, off) in zip(moved, where)]
        for name, f, t, c, off in packed:
            self.tensors.setdefault(name, {})[f] = (c, off, tuple(t.shape), str(t.dtype))
        self.chunks: List[Tuple[bytes, int]] = []
        if slot is not None:
            assert len(sizes) <= len(slot.chunks) and all(n <= cap for n, (_, cap) in zip(sizes, slot.chunks)), \
                f"handoff: chunks of {sizes} bytes do not fit the slot's {[cap for _, cap in slot.chunks]}"
            self.chunks = list(slot.chunks)
            if packed:
                self._pack(packed, sizes, slot.ptrs)
            self.bytes = sum(sizes)
            return
        try:
            with torch.cuda.device(device):
                for n in sizes:
                    ptr, handle = ctypes.c_void_p(), _lib.SrIpcHandle()
                    _lib.check(L.sr_handoff_alloc(n, ctypes.byref(ptr), ctypes.byref(handle)), "sr_handoff_alloc", L)
                    self._ptrs.append(ptr.value)
                    self.chunks.append((bytes(handle.bytes), n))
                if packed:
                    self._pack(packed, sizes, self._ptrs)
        except BaseException:
            self.release()
            raise
        self.bytes = sum(sizes)

    def _pack(self, packed, sizes, ptrs) -> None:
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
            dp = (vp * len(sizes))(*ptrs[:len(sizes)])
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
        """Free the allocations it owns (after every new rank has closed
        them); a slot's are the slot's to free."""
        L = self._L
        with torch.cuda.device(self.device):
            while self._ptrs:
                _lib.check(L.sr_handoff_free(ctypes.c_void_p(self._ptrs.pop())), "sr_handoff_free", L)


def _open(L, handle: bytes) -> int:
    h = _lib.SrIpcHandle()
    ctypes.memmove(h.bytes, handle, len(handle))
    ptr = ctypes.c_void_p()
    _lib.check(L.sr_handoff_open(ctypes.byref(h), ctypes.byref(ptr)), "sr_handoff_open", L)
    return ptr.value


class Mappings:
    """Hand-off allocations mapped into this process once each, by handle,
    for the waves' ring (its slots come back wave after wave); ``close``
    unmaps them all once no view of them is left."""

    def __init__(self, device: torch.device):
        self._L = _lib.lib()
        self.device = device
        self._bases: Dict[bytes, int] = {}

    def open(self, handle: bytes) -> int:
        base = self._bases.get(handle)
        if base is None:
            base = self._bases[handle] = _open(self._L, handle)
        return base

    def close(self) -> None:
        L = self._L
        with torch.cuda.device(self.device):
            while self._bases:
                _, base = self._bases.popitem()
                _lib.check(L.sr_handoff_close(ctypes.c_void_p(base)), "sr_handoff_close", L)


class MappedSources:
    """Old ranks' packed state mapped into this process: ``states`` is
    ``{old rank: {name: {field: tensor}}}``, tensors viewing the mapped
    allocations (no copy); CPU values of the records ride along.  Only the
    chunks a tensor lies in are mapped, through ``cache`` when given (which
    then keeps them mapped).  ``close`` drops the views and unmaps what it
    mapped itself."""

    def __init__(self, records: Sequence[Dict[str, Any]], ranks: Sequence[int], device: torch.device,
                 cache: Optional["Mappings"] = None):
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
                    keys = [(n, f) for n, e in rec["tensors"].items() for f in e]
                    used = {rec["tensors"][n][f][0] for n, f in keys}
                    for c, (handle, _) in enumerate(rec["chunks"]):
                        if c not in used:
                            bases.append(None)
                        elif cache is not None:
                            bases.append(cache.open(handle))
                        else:
                            bases.append(_open(L, handle))
                            self._opened.append(bases[-1])
                    state: Dict[str, Dict[str, Tensor]] = {}
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


def device_bytes(entry: Dict[str, Any], device: torch.device) -> int:
    """Bytes a name's fields take in the hand-off: its non-empty tensors on
    ``device``, each rounded up to 256 bytes."""
    return sum((t.numel() * t.element_size() + ALIGN - 1) // ALIGN * ALIGN for t in entry.values()
               if isinstance(t, Tensor) and t.is_cuda and t.device == device and t.numel() > 0)


def plan_waves(per_rank: Sequence[Sequence[Tuple[str, int]]], wave_bytes: int) -> List[List[str]]:
    """Names cut into waves for a hand-off in waves.

    ``per_rank[r]`` lists old rank ``r``'s names in its own order with the
    bytes each takes there.  Names are taken round-robin over the ranks'
    lists (the first name of every rank, then the second, ...; each name
    once), so pipeline stages holding different layers share every wave;
    a wave closes before the name that would take its bytes, summed over all
    ranks, past ``wave_bytes``.  A name larger than that is a wave alone.
    Every rank computes the same waves from the same lists."""
    total: Dict[str, int] = {}
    for names in per_rank:
        for name, n in names:
            total[name] = total.get(name, 0) + int(n)
    order: List[str] = []
    seen = set()
    for i in range(max((len(names) for names in per_rank), default=0)):
        for names in per_rank:
            if i < len(names) and names[i][0] not in seen:
                seen.add(names[i][0])
                order.append(names[i][0])
    waves: List[List[str]] = []
    acc = 0
    for name in order:
        if not waves or (acc + total[name] > wave_bytes and waves[-1]):
            waves.append([])
            acc = 0
        waves[-1].append(name)
        acc += total[name]
    return waves


def choose_order(state_bytes: int, largest_name_bytes: int, free_bytes: int, processes: int,
                 mode: Optional[str] = None, wave_bytes: Optional[int] = None) -> Tuple[str, int]:
    """``("whole", 0)`` or ``("waves", W)`` for a hand-off of ``state_bytes``
    (the old world's device bytes) with ``free_bytes`` free on the device and
    ``processes`` processes of both worlds on it.

    The room is the free memory less ``RESERVE_BYTES`` per process.  Whole
    needs the hand-off beside the old state (``state_bytes`` of room); the
    new world's destinations, about as large, then fit beside the hand-off
    once the old state is released.  Waves need two waves of room: the one
    the new world reshards and the next being packed (each wave's sources are
    freed once packed, and its destinations take what they held).  ``W`` is
    ``wave_bytes`` or a third of the room, and at least the largest name's
    bytes.  ``mode`` forces an order; ``None`` takes whole when it fits.
    Raises ``HandoffError`` when the chosen order does not fit."""
    if mode not in (None, "whole", "waves"):
        raise ValueError(f"hand-off mode {mode!r}: expected None, 'whole' or 'waves'")
    room = free_bytes - RESERVE_BYTES * processes
    if mode == "whole" or (mode is None and state_bytes <= room):
        if state_bytes > room:
            raise HandoffError(f"a whole hand-off of {state_bytes / 1e9:.3f} GB does not fit beside the old "
                               f"state: {free_bytes / 1e9:.3f} GB free on the device, "
                               f"{RESERVE_BYTES * processes / 1e9:.3f} GB kept for {processes} processes")
        return "whole", 0
    w = int(wave_bytes) if wave_bytes else room // 3
    w = max(w, int(largest_name_bytes), 1)
    if 2 * w > room:
        raise HandoffError(f"the device lacks memory for a hand-off in waves: {free_bytes / 1e9:.3f} GB free, "
                           f"{RESERVE_BYTES * processes / 1e9:.3f} GB kept for {processes} processes, and two "
                           f"waves of {w / 1e9:.3f} GB (the largest name takes "
                           f"{largest_name_bytes / 1e9:.3f} GB) need {2 * w / 1e9:.3f} GB")
    return "waves", w


def _broadcast_objects(*objs, group=None):
    """Rank 0's objects on every rank of ``group`` (Suika/utils.py:98-104)."""
    lst = list(objs)
    src = 0 if group is None else dist.get_global_rank(group, 0)
    dist.broadcast_object_list(lst, src=src, group=group)
    return lst[0] if len(lst) == 1 else lst


def _error_note(text: str) -> Tuple[str, str]:
    return (ERROR, text)


def _is_error(msg: Any) -> bool:
    return isinstance(msg, tuple) and len(msg) == 2 and msg[0] == ERROR


def _recv(q, what: str) -> Any:
    """The next message on ``q``; an error note when none comes in time."""
    try:
        return q.get(block=True, timeout=QUEUE_TIMEOUT_S)
    except queue.Empty:
        return _error_note(f"no {what} from the other world within {QUEUE_TIMEOUT_S:.0f} s")


def _recv_on_rank0(q, what: str, world) -> Any:
    """Rank 0 reads ``q``; every rank gets the message.  An error note from
    the other world (or none in time) raises on every rank."""
    msg = _recv(q, what) if dist.get_rank(world) == 0 else None
    msg = _broadcast_objects(msg, group=world)
    if _is_error(msg):
        raise HandoffError(f"waiting for {what}: {msg[1]}", notify=False)
    return msg


def _attempt(fn: Callable[[], Any]) -> Tuple[Any, Optional[str]]:
    """``fn()``, or its failure as text."""
    try:
        return fn(), None
    except Exception as e:  # reported to every rank by _agree
        return None, f"{type(e).__name__}: {e}"


def _agree(world, err: Optional[str], what: str, notify: bool = True) -> None:
    """Every rank's error (or None) to every rank; raise on all when any
    failed (``notify``: the other world is still to be told)."""
    errs: List[Optional[str]] = [None] * dist.get_world_size(world)
    dist.all_gather_object(errs, err, group=world)
    bad = [f"rank {r}: {e}" for r, e in enumerate(errs) if e is not None]
    if bad:
        raise HandoffError(f"{what} failed on " + "; ".join(bad), notify=notify)


class _LowWater:
    """The least free device memory seen at this rank's samples (taken where
    the hand-off holds the most)."""

    def __init__(self, device: torch.device):
        self.device = device
        self.free: Optional[int] = None

    def sample(self) -> None:
        free, _ = torch.cuda.mem_get_info(self.device)
        self.free = free if self.free is None else min(self.free, free)

    def line(self, side: str) -> str:
        return f"{side}: low-water free device memory {(self.free or 0) / 1e9:.3f} GB"


def _release_state(state: Dict[str, Dict[str, Any]], names) -> None:
    """Free the device tensors of ``names`` in ``state`` (as the reference
    frees every tensor it has sent, utils.py:372-376), drop them from
    ``state``, and return the freed memory to the device (its ``cuda_gc``,
    utils.py:248-253, 379-386)."""
    from .migration import forcefully_free_tensor
    for name in names:
        for t in state.pop(name, {}).values():
            if isinstance(t, Tensor) and t.is_cuda:
                forcefully_free_tensor(t)
    torch.cuda.empty_cache()



class _OldWorld:
    """The old side's half of the protocol after the handshake."""

    def __init__(self, queues, world, device: torch.device, new_world_size: int,
                 log_func: Callable[[str], None]):
        self.q = queues
        self.world = world
        self.rank = dist.get_rank(world)
        self.device = device
        self.new_world_size = new_world_size
        self.log = log_func
        self.low = _LowWater(device)
        self.sent_first = False

    def notify(self, text: str) -> None:
        """Tell the new world that this one failed, where it reads next: each
        new rank its own forward queue before the first message, new rank 0
        the forward queue after it."""
        if not self.sent_first:
            if self.rank < self.new_world_size:
                self.q[0].put(_error_note(text))
        elif self.rank == 0:
            self.q[0].put(_error_note(text))

    def send_first(self, param_layout, other_context_dict, order) -> None:
        """Old rank i's message to new rank i: the layout, the context and the
        order (``"whole"`` or the number of waves); the records follow on
        rank 0's forward queue."""
        if self.rank < self.new_world_size:
            self.q[0].put({"source_param_layout": param_layout, "source_state_dict": {},
                           "other_context_dict": other_context_dict, "order": order})
        self.sent_first = True

    def _records(self, handoff: "Handoff") -> List[Dict[str, Any]]:
        records: List[Any] = [None] * dist.get_world_size(self.world)
        dist.all_gather_object(records, handoff.record(), group=self.world)
        return records

    def whole(self, state, param_layout, other_context_dict) -> None:
        self.send_first(param_layout, other_context_dict, "whole")
        t0 = time.perf_counter()
        handoff, err = _attempt(lambda: Handoff(state, self.device, self.rank))
        t1 = time.perf_counter()
        self.low.sample()
        try:
            _agree(self.world, err, "packing the hand-off")
            self.log(f"migration_save: packed {handoff.bytes / 1e9:.3f} GB into {len(handoff.chunks)} hand-off "
                     f"allocation(s) in {(t1 - t0) * 1e3:.2f} ms")
            records = self._records(handoff)
            if self.rank == 0:
                self.q[0].put(("records", records))
            self.log(f"migration_save: {len(records)} hand-off record(s) sent")
            # The state now lives in the hand-off allocations: it is released
            # once the new world has mapped them and either allocated its
            # destinations beside this state or asked for the memory.
            note = _recv_on_rank0(self.q[1], "the new world's allocation note", self.world)
            assert isinstance(note, dict) and note.get("note") in (ALLOCATED, WANT_RELEASED), \
                f"migration_save: unexpected message {note!r}"
            self.log("migration_save: the new world " + ("has allocated its destinations"
                                                         if note["note"] == ALLOCATED
                                                         else "waits for this state's memory"))
            t2 = time.perf_counter()
            _, rel_err = _attempt(lambda: _release_state(state, list(state)))
            t3 = time.perf_counter()
            self.log(f"migration_save: state released and device memory returned ({(t3 - t2) * 1e3:.2f} ms)")
            dist.barrier(self.world)
            if note["await_release"] and self.rank == 0:
                self.q[0].put(RELEASED)
            done = _recv_on_rank0(self.q[1], "the new world's DONE", self.world)
            assert done == DONE, f"migration_save: unexpected acknowledgement {done!r}"
            self.log("migration_save: the new world is done with the hand-off")
            # the new world has its state; a failure to release ours is this
            # world's alone
            _agree(self.world, rel_err, "releasing the old state", notify=False)
        finally:
            if handoff is not None:
                handoff.release()

    def _ring(self, state, waves: List[List[str]], budget: int) -> List[Slot]:
        """The waves' two hand-off slots, each chunk as large as this rank's
        largest wave needs it, allocated once -- when every old rank's slots
        together fit in ``budget`` bytes; else none (each wave then
        allocates its own hand-off).  Allocations of memory another process
        has just freed are slow, and so is mapping them: the new ranks map
        the two slots once instead of every wave's allocations."""
        if not USE_RING:
            return []
        layouts = [layout_of({n: state[n] for n in names if n in state}, self.device) for names in waves]
        width = max((len(lay) for lay in layouts), default=0)
        sizes = [max(lay[c] for lay in layouts if c < len(lay)) for c in range(width)]
        totals: List[Any] = [None] * dist.get_world_size(self.world)
        dist.all_gather_object(totals, 2 * sum(sizes), group=self.world)
        if sum(totals) > budget:
            self.log(f"migration_save: a ring of {sum(totals) / 1e9:.3f} GB does not fit "
                     f"{budget / 1e9:.3f} GB: one hand-off per wave")
            return []
        ring: List[Slot] = []

        def make():
            for _ in range(2):
                ring.append(Slot(sizes, self.device))
        _, err = _attempt(make)
        try:
            _agree(self.world, err, "allocating the waves' ring")
        except HandoffError:
            for slot in ring:
                slot.free()
            raise
        self.log(f"migration_save: ring of 2 x {sum(sizes) / 1e9:.3f} GB on this rank, "
                 f"{sum(totals) / 1e9:.3f} GB in all")
        return ring

    def waves(self, state, param_layout, other_context_dict, waves: List[List[str]], ring_budget: int) -> None:
        self.send_first(param_layout, other_context_dict, len(waves))
        ring = self._ring(state, waves, ring_budget)
        held: List[Tuple[int, Handoff]] = []     # sent, not yet reported consumed
        pending_err: Optional[str] = None
        t_start = time.perf_counter()
        packed = 0

        def consumed(k: int) -> None:
            msg = _recv_on_rank0(self.q[1], f"the new world's report on wave {k}", self.world)
            assert msg == ("consumed", k), f"migration_save: unexpected message {msg!r}"

        try:
            for k, names in enumerate(waves):
                part = {n: state[n] for n in names if n in state}
                # ring slot k % 2 is free again: the wave that used it (k - 2)
                # was reported consumed in the previous iteration
                slot = ring[k % 2] if ring else None
                t0 = time.perf_counter()
                handoff, err = _attempt(lambda: Handoff(part, self.device, self.rank, slot=slot))
                t1 = time.perf_counter()
                self.low.sample()
                if handoff is not None:
                    packed += handoff.bytes
                try:
                    _agree(self.world, err or pending_err, f"packing wave {k}")
                except HandoffError:
                    if handoff is not None:
                        handoff.release()     # never sent
                    raise
                records = self._records(handoff)
                held.append((k, handoff))
                # the wave's sources are in the hand-off: their memory goes back
                # to the device for the next wave and the new world's arenas,
                # before the new world hears of the wave (so its arena never
                # sits beside these sources)
                del part
                t2 = time.perf_counter()
                _, pending_err = _attempt(lambda: _release_state(state, names))
                t3 = time.perf_counter()
                if self.rank == 0:
                    self.q[0].put(("wave", k, list(names), records, bool(ring)))
                if len(held) > 1:
                    consumed(held[0][0])
                    held.pop(0)[1].release()
                self.log(f"migration_save: wave {k}: {handoff.bytes / 1e9:.3f} GB packed in {(t1 - t0) * 1e3:.2f} ms, "
                         f"sources released in {(t3 - t2) * 1e3:.2f} ms and the wave sent, "
                         f"then {(time.perf_counter() - t3) * 1e3:.2f} ms for the previous wave's report")
            while held:
                consumed(held[0][0])
                held.pop(0)[1].release()
            _agree(self.world, pending_err, "releasing the old state", notify=False)
        except HandoffError as e:
            if e.notify:
                self.notify(str(e))
                e.notify = False
                # the new world stops at this note; the waves it was sent stay
                # mapped until it reports them consumed (or fails)
                try:
                    for k, _ in held:
                        consumed(k)
                except HandoffError:
                    pass
            raise
        finally:
            for _, h in held:
                h.release()
            for slot in ring:
                slot.free()
        self.log(f"migration_save: {packed / 1e9:.3f} GB handed off in {len(waves)} wave(s) in "
                 f"{(time.perf_counter() - t_start) * 1e3:.2f} ms")


def live_save(IPC_queues, model, optimizer, other_context, device: torch.device, world,
              log_func: Callable[[str], None], mode: Optional[str] = None,
              wave_bytes: Optional[int] = None) -> None:
    """The old side of a live migration (Suika/migration.py:1394-1486).

    ``mode`` forces the hand-off's order (``"whole"``, or ``"waves"`` with
    ``wave_bytes`` per wave); ``None`` takes whole when it fits beside the
    old state.  Raises ``HandoffError`` on every old rank when the hand-off
    fails on any rank of either world."""
    from .meta import ParamLayout
    from .migration import merge_model_and_optimizer_state_dict

    rank = dist.get_rank(world)
    # the library's first-use costs are paid while the new world starts
    warm = _WarmUp(device, optimizer=False)
    warm.start()
    if rank == 0:
        IPC_queues[0].put(dist.get_world_size(world))
        reply = _recv(IPC_queues[1], "world size")
    else:
        reply = None
    reply = _broadcast_objects(reply, group=world)
    warm.join()
    if _is_error(reply):
        raise HandoffError(f"migration_save: handshake: {reply[1]}", notify=False)
    new_world_size = int(reply)
    is_scale_up = new_world_size >= dist.get_world_size(world)
    log_func(f"migration_save: is_scale_up = {is_scale_up} (new world size {new_world_size})")

    param_layout = ParamLayout()
    param_layout.gather(model, world)
    side = _OldWorld(IPC_queues, world, device, new_world_size, log_func)
    try:
        # every rank's device bytes per name, checked before anything is
        # allocated: a tensor a hand-off allocation cannot hold fails here
        def survey():
            state, ctx = merge_model_and_optimizer_state_dict(model, optimizer, other_context)
            for name, entry in state.items():
                for f, t in entry.items():
                    if isinstance(t, Tensor) and t.is_cuda and t.device == device and t.numel() > 0:
                        n = t.numel() * t.element_size()
                        if n > _lib.HANDOFF_MAX_BYTES:
                            raise ValueError(f"{name}/{f} takes {n} bytes, more than one hand-off "
                                             f"allocation holds ({_lib.HANDOFF_MAX_BYTES} bytes)")
                        if not t.is_contiguous():
                            raise ValueError(f"{name}/{f} is not contiguous")
            return state, ctx, [(name, device_bytes(entry, device)) for name, entry in state.items()]

        got, err = _attempt(survey)
        info: List[Any] = [None] * dist.get_world_size(world)
        dist.all_gather_object(info, (err, got[2] if got else None), group=world)
        bad = [f"rank {r}: {e}" for r, (e, _) in enumerate(info) if e is not None]
        if bad:
            raise HandoffError("migration_save: " + "; ".join(bad))
        source_state_dict, other_context_dict, _ = got
        per_rank = [names for _, names in info]
        totals: Dict[str, int] = {}
        for names in per_rank:
            for name, n in names:
                totals[name] = totals.get(name, 0) + n
        state_bytes = sum(totals.values())
        choice = None
        if rank == 0:
            free, _ = torch.cuda.mem_get_info(device)
            order, err = _attempt(lambda: choose_order(
                state_bytes, max(totals.values(), default=0), free,
                dist.get_world_size(world) + new_world_size, mode, wave_bytes))
            choice = (order, err, free)
        order, err, free = _broadcast_objects(choice, group=world)
        if err is not None:
            raise HandoffError(f"migration_save: {err}")
        how, w = order
        room = free - RESERVE_BYTES * (dist.get_world_size(world) + new_world_size)
        log_func(f"migration_save: {state_bytes / 1e9:.3f} GB on the device, {free / 1e9:.3f} GB free: hand-off "
                 + ("whole" if how == "whole" else f"in waves of at most {w / 1e9:.3f} GB"))
        if how == "whole":
            side.whole(source_state_dict, param_layout, other_context_dict)
        else:
            # Each wave's sources are freed before the new world hears of the
            # wave, so the device holds the state plus the hand-off memory:
            # the ring may take all the room
            side.waves(source_state_dict, param_layout, other_context_dict, plan_waves(per_rank, w),
                       ring_budget=max(2 * w, room))
    except HandoffError as e:
        if e.notify:
            side.notify(str(e))
        log_func(f"migration_save: failed: {e}")
        raise
    log_func(side.low.line("migration_save"))
    log_func("migration_save: end")


class _WarmUp:
    """First-use costs of a fresh process of a migration, paid on threads
    while it waits: in a live migration the old ranks for the new world's
    handshake and the new ranks for the old world's message; in
    ``checkpoint_load`` while the files are read:

    * the reshard library's: ``sr_prepare`` loads its GPU code and sets up
      its streams and the runtime's copy path, and one tiny gather warms
      the drop-in call's host side.  With twelve processes on one MI355X
      these took 30-57 ms per first launch, 40-54 ms per first table upload
      and 26 ms for the setup stream, inside the pack and the reshard;
    * with an optimizer to build, torch.optim's, on a thread of its own (it
      needs no device): a process's first optimizer imports torch's compiler
      front end (torch._dynamo, about 0.4 s).

    ``start`` runs both beside the caller, ``run`` one after the other on the
    calling thread.  ``library_done`` is set once the library is no longer
    in use here; the caller waits for it before its own library calls and
    joins before building its optimizer.  Failures are ignored: the real
    calls report their own."""

    def __init__(self, device: torch.device, optimizer: bool):
        self.device = device
        self.optimizer = optimizer
        self.library_done = threading.Event()
        self._threads: List[threading.Thread] = []

    def start(self) -> None:
        self._threads = [threading.Thread(target=self._library, name="suika-warm-up", daemon=True)]
        if self.optimizer:
            self._threads.append(threading.Thread(target=self._optimizer, name="suika-warm-up-optim",
                                                  daemon=True))
        for t in self._threads:
            t.start()

    def join(self) -> None:
        for t in self._threads:
            t.join()

    def run(self) -> None:
        self._library()
        if self.optimizer:
            self._optimizer()

    def _library(self) -> None:
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

    @staticmethod
    def _optimizer() -> None:
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


class _Closing:
    """A whole hand-off's mappings, closed on a thread while the new rank
    adopts its state; ``finish`` joins it, agrees on every rank's errors
    (reshard, close, adoption) and has new rank 0 send ``DONE``."""

    def __init__(self, side: "_NewWorld", mapped: "MappedSources", err: Optional[str]):
        self.side = side
        self.err = err
        self.t0 = time.perf_counter()
        self.t_closed = self.t0

        def close():
            try:
                mapped.close()
            except Exception as e:
                self.err = self.err or f"closing the hand-off: {type(e).__name__}: {e}"
            self.t_closed = time.perf_counter()
        self.thread = threading.Thread(target=close, name="suika-handoff-close", daemon=True)
        self.thread.start()

    def finish(self, err: Optional[str]) -> None:
        self.thread.join()
        t = time.perf_counter()
        _agree(self.side.world, self.err or err, "resharding from the hand-off and adopting the state")
        if self.side.rank == 0:
            self.side.q[1].put(DONE)
        self.side.log(f"migration_load: mappings closed in {(self.t_closed - self.t0) * 1e3:.2f} ms, "
                      f"every new rank done {(time.perf_counter() - t) * 1e3:.2f} ms after this one")


class _NewWorld:
    """The new side's half of the protocol once the first message is in."""

    def __init__(self, queues, world, device: torch.device, ops, other_context_dict,
                 warm: "_WarmUp", log_func: Callable[[str], None]):
        self.q = queues
        self.world = world
        self.rank = dist.get_rank(world)
        self.device = device
        self.ops = ops
        self.fields = other_context_dict["expected_sub_fields"]
        self.warm = warm
        self.log = log_func
        self.low = _LowWater(device)
        self.phases = (0.0, 0.0, 0.0)

    def _reshard(self, ops, records, needed, cache: Optional[Mappings] = None) -> Dict[str, Dict[str, Tensor]]:
        """``ops``' pieces for this rank, gathered from the mapped records of
        the old ranks ``needed`` into one arena; the mappings are closed
        (or, through ``cache``, kept for the next wave) before it returns or
        raises."""
        from .migration import execute_param_transfer
        t0 = time.perf_counter()
        mapped = MappedSources(records, needed, self.device, cache=cache)
        t1 = time.perf_counter()
        try:
            out = execute_param_transfer(
                transfer_ops=ops, source_state_dict={}, device=self.device, expected_sub_fields=self.fields,
                world=self.world, fake_source_state_dicts=mapped.states, log_func=self.log, rank=self.rank,
                arena=True)
            torch.cuda.synchronize(self.device)
            self.low.sample()
        finally:
            t2 = time.perf_counter()
            mapped.close()
            self.phases = (t1 - t0, t2 - t1, time.perf_counter() - t2)
        return out

    def whole(self, wait_for_release: Optional[bool], return_before_release: bool):
        """Returns the target state and whether the caller still waits for
        ``RELEASED`` before returning."""
        msg = _recv_on_rank0(self.q[0], "the hand-off records", self.world)
        assert isinstance(msg, tuple) and msg[0] == "records", f"migration_load: unexpected message {msg!r}"
        records = msg[1]
        rank = self.rank
        t0 = time.perf_counter()
        needed = sorted({op.src_rank for op in self.ops if op.dst_rank == rank})
        # Old state, hand-off and destinations side by side when the device
        # has room for all of them: each new rank takes its destinations'
        # memory before the old world frees anything.  Else the destinations
        # wait for the old world to return its state's memory.
        mine = _destination_bytes(self.ops, rank, records)
        need = torch.tensor([mine], dtype=torch.int64)
        dist.all_reduce(need, group=self.world)
        wait = None
        if rank == 0:
            free, _ = torch.cuda.mem_get_info(self.device)
            room = int(need.item()) + HEADROOM_BYTES * dist.get_world_size(self.world)
            wait = bool(wait_for_release) if wait_for_release is not None else free < room
        wait = _broadcast_objects(wait, group=self.world)
        await_release = wait or not return_before_release

        def reserve_and_map():
            if not wait:
                # the destination arena's memory, taken now and kept in this
                # process's allocator cache, where the arena finds it
                torch.empty(mine + ARENA_SLACK_BYTES, dtype=torch.uint8, device=self.device)
            t_alloc = time.perf_counter()
            # mapped before the old world frees anything: IPC opens beside
            # other processes' frees were 20-40x slower
            return t_alloc, MappedSources(records, needed, self.device)

        got, err = _attempt(reserve_and_map)
        self.low.sample()
        mapped = got[1] if got else None
        try:
            _agree(self.world, err, "taking the destinations' memory and mapping the hand-off")
            t_alloc, t_map = got[0], time.perf_counter()
            self.log(f"migration_load: mapped the state of old rank(s) {needed}")
            if rank == 0:
                self.q[1].put({"note": WANT_RELEASED if wait else ALLOCATED, "await_release": await_release})
            self.warm.library_done.wait()
            if wait:
                _recv_on_rank0(self.q[0], "the old world's release", self.world)
            self.log(f"migration_load: destinations of {int(need.item()) / 1e9:.3f} GB "
                     + ("after the old world released its state" if wait else "beside the old state"))
            t1 = time.perf_counter()

            def reshard():
                from .migration import execute_param_transfer
                out = execute_param_transfer(
                    transfer_ops=self.ops, source_state_dict={}, device=self.device,
                    expected_sub_fields=self.fields, world=self.world,
                    fake_source_state_dicts=mapped.states, log_func=self.log, rank=rank, arena=True)
                torch.cuda.synchronize(self.device)
                self.low.sample()
                return out
            target, err = _attempt(reshard)
            t2 = time.perf_counter()
        except BaseException:
            if mapped is not None:
                mapped.close()
            raise
        self.log("migration_load: "
                 + ("" if wait else f"destinations' memory taken in {(t_alloc - t0) * 1e3:.2f} ms, ")
                 + f"mapped {len(needed)} old rank(s) in {(t_map - t_alloc) * 1e3:.2f} ms, "
                 f"resharded in {(t2 - t1) * 1e3:.2f} ms")
        # The mappings are closed beside the adoption; the old world hears
        # DONE once every new rank has closed them (``finish``).
        return target, await_release and not wait, _Closing(self, mapped, err)

    def waves(self, n: int):
        target: Dict[str, Dict[str, Tensor]] = {}
        rank = self.rank
        t_start = time.perf_counter()
        gather_ms = 0.0
        # the old ranks' ring slots, mapped once each and closed before the
        # last wave is reported consumed (or before an error is reported)
        cache = Mappings(self.device)
        try:
            for k in range(n):
                msg = _recv_on_rank0(self.q[0], f"wave {k}", self.world)
                assert isinstance(msg, tuple) and msg[:2] == ("wave", k), \
                    f"migration_load: unexpected message {msg!r}"
                names, records, ring = set(msg[2]), msg[3], msg[4]
                ops = [op for op in self.ops if op.param_name in names]
                mine = [op for op in ops if op.dst_rank == rank]
                needed = sorted({op.src_rank for op in mine})
                if k == 0:
                    self.warm.library_done.wait()
                t0 = time.perf_counter()
                out, err = _attempt(lambda: self._reshard(ops, records, needed, cache if ring else None)
                                    if mine else {})
                t1 = time.perf_counter()
                gather_ms += (t1 - t0) * 1e3
                if k == n - 1:
                    _, close_err = _attempt(cache.close)
                    err = err or close_err
                _agree(self.world, err, f"resharding wave {k}")
                self.log(f"migration_load: wave {k}: mapped, resharded and closed in {(t1 - t0) * 1e3:.2f} ms "
                         f"({' / '.join(f'{x * 1e3:.2f}' for x in self.phases)}), "
                         f"every new rank done {(time.perf_counter() - t1) * 1e3:.2f} ms later")
                target.update(out)
                if rank == 0:
                    self.q[1].put(("consumed", k))
        finally:
            _attempt(cache.close)   # a no-op once closed; on a failure the caller reports it
        self.log(f"migration_load: destinations of {n} wave(s) resharded in {gather_ms:.2f} ms of "
                 f"{(time.perf_counter() - t_start) * 1e3:.2f} ms")
        return target


def live_load(IPC_queues, model, optimizer_provider, optimizer, device: torch.device, world,
              log_func: Callable[[str], None], wait_for_release: Optional[bool] = None,
              return_before_release: bool = False):
    """The new side of a live migration (Suika/migration.py:1586-1727).

    In a whole hand-off the destinations are allocated beside the old state
    when the device has room for every new rank's (``wait_for_release=None``),
    else after the old world has released its state; ``True`` always waits.
    The new world returns once the old world has released its state, or with
    ``return_before_release`` as soon as its own state is adopted and its
    optimizer built.  A hand-off in waves (the old world's choice when the
    device lacks room for the whole) reshards wave by wave as the old world
    releases its state.  Raises ``HandoffError`` on every new rank when the
    hand-off fails on any rank of either world."""
    from .meta import ParamLayout, schedule_param_transfer
    from .migration import split_model_and_optimizer_state_dict

    rank = dist.get_rank(world)
    # the process's first-use costs are paid while it waits for the old world
    warm = _WarmUp(device, optimizer_provider is not None)
    warm.start()
    if rank == 0:
        old_world_size = _recv(IPC_queues[0], "world size")
        if not _is_error(old_world_size) and old_world_size != 0:
            IPC_queues[1].put(dist.get_world_size(world))
    else:
        old_world_size = None
    old_world_size = _broadcast_objects(old_world_size, group=world)
    if _is_error(old_world_size):
        warm.join()
        raise HandoffError(f"migration_load: handshake: {old_world_size[1]}", notify=False)
    is_scale_up = dist.get_world_size(world) >= old_world_size
    log_func(f"migration_load: is_scale_up = {is_scale_up}")

    target_param_layout = ParamLayout()
    target_param_layout.gather(model, world)
    # old rank i's message, or the launcher's placeholder when there is none
    own = _recv(IPC_queues[0], "hand-off message")
    log_func("migration_load: hand-off message received")
    first = _broadcast_objects(own, group=world)
    err = own[1] if _is_error(own) else (first[1] if _is_error(first) else None)
    try:
        _agree(world, err, "receiving the old world's first message", notify=False)
    except HandoffError:
        warm.join()
        raise
    del own
    source_param_layout, other_context_dict = first.get("source_param_layout"), first.get("other_context_dict")
    order = first.get("order")
    del first

    if source_param_layout is None:
        log_func("migration_load: no checkpoint received; skip loading")
        if hasattr(model, "instantiate") and getattr(model, "on_meta", False):
            model.instantiate()
        warm.join()
        return (optimizer_provider(), None) if optimizer_provider else None

    t0 = time.perf_counter()
    ops = schedule_param_transfer(source_param_layout, target_param_layout)
    log_func(f"migration_load: scheduled in {(time.perf_counter() - t0) * 1e3:.2f} ms")
    side = _NewWorld(IPC_queues, world, device, ops, other_context_dict, warm, log_func)
    try:
        closing = None
        if order == "whole":
            target_state_dict, await_release, closing = side.whole(wait_for_release, return_before_release)
        else:
            target_state_dict, await_release = side.waves(int(order)), False

        def adopt():
            model_state_dict, optimizer_state_dict, other_context = split_model_and_optimizer_state_dict(
                model=model, merged_state_dict=target_state_dict, other_context_dict=other_context_dict)
            model_state_dict = OrderedDict(sorted(model_state_dict.items(), key=lambda x: x[0]))
            model.load_state_dict(model_state_dict, assign=True)
            log_func("migration_load: model state adopted")
            warm.join()
            log_func("migration_load: first-use warm-up joined")
            opt = optimizer_provider() if optimizer_provider else optimizer
            if opt:
                # one parameter group, as the reference (migration.py:1712-1716)
                optimizer_state_dict["param_groups"][0]["params"] = opt.state_dict()["param_groups"][0]["params"]
                opt.load_state_dict(optimizer_state_dict)
                log_func("migration_load: optimizer state loaded")
            return opt, other_context
        if closing is not None:
            got, err = _attempt(adopt) if closing.err is None else (None, None)
            closing.finish(err)
        else:
            got, err = _attempt(adopt)
            # every wave is consumed: failures from here on are this world's alone
            _agree(world, err, "adopting the new state", notify=False)
        optimizer, other_context = got
        if await_release:
            # the old world's state released (beside which the destinations
            # may have been allocated) before any new rank returns
            _recv_on_rank0(IPC_queues[0], "the old world's release", world)
            log_func("migration_load: the old world has released its state")
    except HandoffError as e:
        if e.notify and rank == 0:
            IPC_queues[1].put(_error_note(str(e)))
        log_func(f"migration_load: failed: {e}")
        raise
    log_func(side.low.line("migration_load"))
    log_func("migration_load: end")
    return (optimizer, other_context) if optimizer_provider else other_context

"""Layout metadata and the transfer schedule of Suika's state migration.

Host-side mirror of the reference's plan types, same names and semantics:

* ``TensorMeta``            -- Suika/migration.py:29-131
* ``get_named_parameters_and_persistent_buffers`` / ``get_param_tensor_meta``
                            -- Suika/migration.py:135-151
* ``ParamLayout``           -- Suika/migration.py:161-254
* ``TransferOp``            -- Suika/migration.py:257-312 (geometry only: the
                               bytes are moved by the HIP pack/unpack kernels)
* ``schedule_param_transfer`` -- Suika/migration.py:322-381 (same greedy,
                               run by the library's ``sr_schedule``)

Two shard kinds extend the reference's ``torch.chunk`` layout; both are
declared on a tensor through extra attributes next to the reference's
``slice_dim`` / ``tp_index`` / ``tp_deg`` (tensor_parallel.py:255-261):

* ``vocab_pad`` (vocabulary-parallel embedding): the table is zero-padded to
  ``Vpad = ceil(V / (m * tp)) * m * tp`` rows (``m`` = ``pad_multiple``) and
  rank ``r`` holds rows ``[r * Vpad/tp, (r+1) * Vpad/tp)``.  ``shape`` keeps
  the unpadded ``[V, H]``.
* ``qkv_heads`` (fused QKV split at head granularity): the global tensor is
  ``[Q; K; V]`` with ``n_q`` / ``n_kv`` heads of ``head_dim`` rows and shard
  ``r`` is ``[Q_r; K_r; V_r]`` -- the concatenation of the three per-projection
  chunks.  It nests across degrees exactly like ``chunk`` does.
"""
from __future__ import annotations

import ctypes
import os
import re
from itertools import chain
from typing import Any, Callable, Dict, List, Optional, Tuple, Union

import numpy as np
import torch
import torch.distributed as dist
from torch import Tensor
from torch.nn import Module

TPMeta = Tuple[int, int, int]  # slice_dim, tp_index, tp_deg

CHUNK = "chunk"
VOCAB_PAD = "vocab_pad"
QKV_HEADS = "qkv_heads"
SHARD_KINDS = (CHUNK, VOCAB_PAD, QKV_HEADS)


def vocab_padded(vocab: int, tp_deg: int, multiple: int) -> int:
    """Padded vocabulary rows for ``tp_deg`` ranks: a multiple of multiple*tp."""
    step = multiple * tp_deg
    return -(-vocab // step) * step


def is_ib_enabled() -> bool:
    """Mirror of Suika/utils.py:209-210 (steers the schedule's peer reuse)."""
    return not (os.getenv("NCCL_IB_DISABLE", "False") in ["1", "true"])


class TensorMeta:
    """Global dtype/shape of a (possibly TP-sharded) tensor plus its shard.

    Mirrors Suika/migration.py:29-131.  ``kind``/``kind_args`` carry the
    ``vocab_pad`` / ``qkv_heads`` extensions; ``rows`` marks a vocab piece
    (a global row interval) produced by ``schedule_param_transfer``.
    """

    def __init__(self, tensor: Optional[Tensor] = None, name: Optional[str] = None,
                 dtype: Optional[torch.dtype] = None, shape=None,
                 tp_meta: Optional[TPMeta] = None, kind: Optional[str] = None,
                 kind_args: Optional[Tuple[int, ...]] = None,
                 rows: Optional[Tuple[int, int]] = None):
        self.tp_meta = None
        self.kind = CHUNK
        self.kind_args: Tuple[int, ...] = ()
        self.rows = rows
        if tensor is not None:
            self.dtype = tensor.dtype
            if hasattr(tensor, "slice_dim"):
                t_kind = getattr(tensor, "shard_kind", CHUNK)
                gshape = list(tensor.shape)
                if t_kind == VOCAB_PAD:
                    gshape[0] = int(tensor.vocab_size)
                    self.kind_args = (int(getattr(tensor, "pad_multiple", 128)),)
                else:
                    gshape[tensor.slice_dim] *= tensor.tp_deg
                    if t_kind == QKV_HEADS:
                        self.kind_args = tuple(int(v) for v in tensor.qkv_heads)
                self.kind = t_kind
                self.shape = torch.Size(gshape)
                self.tp_meta = (tensor.slice_dim, tensor.tp_index, tensor.tp_deg)
            else:
                self.shape = tensor.shape
        else:
            assert dtype is not None and shape is not None, \
                "Either tensor or (dtype, shape) should be provided"
        self.name = name
        if dtype is not None:
            self.dtype = dtype if isinstance(dtype, torch.dtype) else torch.dtype(dtype)
        if shape is not None:
            self.shape = torch.Size(shape)
        if tp_meta is not None:
            self.tp_meta = tuple(tp_meta)
        if kind is not None:
            assert kind in SHARD_KINDS, f"unknown shard kind {kind}"
            self.kind = kind
        if kind_args is not None:
            self.kind_args = tuple(kind_args)
        if self.kind == VOCAB_PAD:
            assert len(self.kind_args) == 1, "vocab_pad takes (pad_multiple,)"
            assert self.tp_meta is not None and self.tp_meta[0] in (0, -len(self.shape)), \
                "vocab_pad is a TP layout sharded along dim 0"
        if self.kind == QKV_HEADS:
            assert len(self.kind_args) == 3, "qkv_heads takes (n_q, n_kv, head_dim)"
            n_q, n_kv, hd = self.kind_args
            assert self.shape[0] == (n_q + 2 * n_kv) * hd, \
                f"qkv_heads: rows {self.shape[0]} != (n_q + 2 n_kv) * head_dim"

    # -- reference accessors (migration.py:62-98) --------------------------
    def numel(self) -> int:
        if self.kind == CHUNK and self.rows is None:
            n = 1
            for s in self.shape:
                n *= int(s)
            return n // self.tp_deg()
        n = 1
        for s in self.actual_shape():
            n *= int(s)
        return n

    def volumn(self) -> float:
        return self.numel() * self.dtype.itemsize

    def is_tp(self) -> bool:
        return self.tp_meta is not None

    def slice_dim(self) -> Optional[int]:
        return self.tp_meta[0] if self.is_tp() else None

    def tp_index(self) -> int:
        return self.tp_meta[1] if self.is_tp() else 0

    def tp_deg(self) -> int:
        return self.tp_meta[2] if self.is_tp() else 1

    def padded_rows(self) -> int:
        """Rows of the padded table at this meta's degree (vocab_pad only)."""
        assert self.kind == VOCAB_PAD
        return vocab_padded(int(self.shape[0]), self.tp_deg(), self.kind_args[0])

    def actual_shape(self) -> torch.Size:
        if self.rows is not None:
            shape = list(self.shape)
            shape[0] = self.rows[1] - self.rows[0]
            return torch.Size(shape)
        if not self.is_tp():
            return self.shape
        shape = list(self.shape)
        if self.kind == VOCAB_PAD:
            shape[0] = self.padded_rows() // self.tp_deg()
        else:
            shape[self.slice_dim()] //= self.tp_deg()
        return torch.Size(shape)

    def scale_to_tp(self, target_tp_deg: int) -> List["TensorMeta"]:
        """Split into ``target/tp_deg`` finer pieces, ascending (migration.py:103-118).

        ``vocab_pad`` metas do not nest across degrees; they are split by row
        intervals inside ``schedule_param_transfer`` instead.
        """
        if self.is_tp() and target_tp_deg > self.tp_deg() and self.kind != VOCAB_PAD:
            slice_dim, tp_index, deg = self.tp_meta
            assert target_tp_deg % deg == 0, \
                f"scale_to_tp: target degree {target_tp_deg} is not a multiple of {deg} ({self.name})"
            scale = target_tp_deg // deg
            return [TensorMeta(name=self.name, dtype=self.dtype, shape=self.shape,
                               tp_meta=(slice_dim, scale * tp_index + i, target_tp_deg),
                               kind=self.kind, kind_args=self.kind_args)
                    for i in range(scale)]
        return [self]

    def with_rows(self, g0: int, g1: int) -> "TensorMeta":
        """A vocab piece: global rows [g0, g1) of this shard's layout."""
        return TensorMeta(name=self.name, dtype=self.dtype, shape=self.shape,
                          tp_meta=self.tp_meta, kind=self.kind, kind_args=self.kind_args,
                          rows=(g0, g1))

    def valid_rows(self) -> Tuple[int, int]:
        """Global rows held with data (vocab_pad: excludes the pad rows)."""
        if self.rows is not None:
            return self.rows
        assert self.kind == VOCAB_PAD
        n = self.padded_rows() // self.tp_deg()
        lo = self.tp_index() * n
        hi = min(lo + n, int(self.shape[0]))
        return lo, max(lo, hi)

    def __eq__(self, other: Any) -> bool:
        if not isinstance(other, TensorMeta):
            return False
        tp_meta_same = self.is_tp() == other.is_tp() and self.slice_dim() == other.slice_dim()
        return (tp_meta_same and self.dtype == other.dtype and self.shape == other.shape
                and self.kind == other.kind and self.kind_args == other.kind_args)

    __hash__ = None

    def __str__(self):
        extra = "" if self.kind == CHUNK else f", {self.kind}{self.kind_args}"
        if self.rows is not None:
            extra += f", rows={self.rows}"
        return f"TensorMeta(name={self.name}, {self.dtype}, {self.shape}, {self.tp_meta}{extra})"

    __repr__ = __str__


def get_named_parameters_and_persistent_buffers(model: Module):
    """Parameters then persistent buffers, as Suika/migration.py:135-141."""
    state_dict = model.state_dict()
    for name, param in chain(model.named_parameters(), model.named_buffers()):
        if name in state_dict:
            yield name, param


def get_param_tensor_meta(model: Module) -> Dict[str, TensorMeta]:
    """name -> TensorMeta of a module's state (Suika/migration.py:147-151)."""
    return {name: TensorMeta(tensor=param, name=name)
            for name, param in get_named_parameters_and_persistent_buffers(model)}


class ParamLayout:
    """rank -> name -> TensorMeta (Suika/migration.py:161-254)."""

    def __init__(self):
        self.layout: Dict[int, Dict[str, TensorMeta]] = {}

    @classmethod
    def from_metas(cls, metas: Dict[int, Dict[str, TensorMeta]]) -> "ParamLayout":
        pl = cls()
        for rank in sorted(metas):
            pl.layout[rank] = metas[rank]
        return pl

    def gather(self, self_param_meta_or_module: Union[Dict[str, TensorMeta], Module],
               world: Optional[dist.ProcessGroup] = None):
        if isinstance(self_param_meta_or_module, Module):
            self_param_meta = get_param_tensor_meta(self_param_meta_or_module)
        else:
            self_param_meta = self_param_meta_or_module
        param_meta_list = [None] * dist.get_world_size(world)
        dist.all_gather_object(param_meta_list, self_param_meta, group=world)
        for rank, param_meta in enumerate(param_meta_list):
            self.layout[rank] = param_meta

    def is_owned(self, rank: int, param: Union[str, TensorMeta]) -> bool:
        if isinstance(param, str):
            return param in self.layout[rank]
        name = param.name
        return name in self.layout[rank] and \
            self.is_tensor_tp_owned(meta_src=self.layout[rank][name], meta_tgt=param)

    def owners(self, param: Union[str, TensorMeta]) -> List[int]:
        return [rank for rank in self.layout if self.is_owned(rank, param)]

    def __str__(self):
        return f"ParamLayout(\n  {self.layout}\n)"

    __repr__ = __str__

    @staticmethod
    def is_tensor_tp_overlap(meta1: Union[TensorMeta, TPMeta, None],
                             meta2: Union[TensorMeta, TPMeta, None]) -> bool:
        if isinstance(meta1, TensorMeta):
            meta1 = meta1.tp_meta
        if isinstance(meta2, TensorMeta):
            meta2 = meta2.tp_meta
        if meta1 is None or meta2 is None:
            return True
        slice_dim1, tp_index1, tp_deg1 = meta1
        slice_dim2, tp_index2, tp_deg2 = meta2
        assert slice_dim1 == slice_dim2, f"slice dim mismatch {slice_dim1} vs {slice_dim2}"
        if tp_deg1 > tp_deg2:
            tp_index1, tp_index2 = tp_index2, tp_index1
            tp_deg1, tp_deg2 = tp_deg2, tp_deg1
        scale = tp_deg2 // tp_deg1
        return tp_index2 // scale == tp_index1

    @staticmethod
    def is_tensor_tp_owned(meta_src: Union[TensorMeta, TPMeta, None],
                           meta_tgt: Union[TensorMeta, TPMeta, None]) -> bool:
        if isinstance(meta_src, TensorMeta) and isinstance(meta_tgt, TensorMeta) \
                and meta_tgt.kind == VOCAB_PAD:
            # vocab pieces: the source shard must hold the piece's rows
            assert meta_src.kind == VOCAB_PAD, f"shard kind mismatch for {meta_tgt.name}"
            lo, hi = meta_tgt.valid_rows()
            if lo == hi:
                return True   # an empty piece (a shard of padding only)
            slo, shi = meta_src.valid_rows()
            return slo <= lo and hi <= shi
        if isinstance(meta_src, TensorMeta):
            meta_src = meta_src.tp_meta
        if isinstance(meta_tgt, TensorMeta):
            meta_tgt = meta_tgt.tp_meta
        src_tp_deg = meta_src[2] if meta_src is not None else 1
        tgt_tp_deg = meta_tgt[2] if meta_tgt is not None else 1
        return src_tp_deg <= tgt_tp_deg and ParamLayout.is_tensor_tp_overlap(meta_src, meta_tgt)


class TransferOp:
    """One scheduled piece: ``src_rank`` sends ``dst_meta`` of ``param_name``.

    Mirrors Suika/migration.py:257-312.  ``dst_shard_meta`` (an extension) is
    the full destination shard the piece lands in; ``schedule_param_transfer``
    sets it, and ``execute_param_transfer`` infers it when absent.
    """

    def __init__(self, param_name: str, src_rank: int, dst_rank: int,
                 src_meta: Union[TensorMeta, Tensor],
                 dst_meta: Optional[Union[TensorMeta, Tensor]] = None,
                 dst_shard_meta: Optional[TensorMeta] = None):
        self.param_name = param_name
        self.src_meta = src_meta if isinstance(src_meta, TensorMeta) else TensorMeta(tensor=src_meta)
        if dst_meta is None:
            self.dst_meta = self.src_meta
        else:
            self.dst_meta = dst_meta if isinstance(dst_meta, TensorMeta) else TensorMeta(tensor=dst_meta)
        self.src_rank = src_rank
        self.dst_rank = dst_rank
        self.dst_shard_meta = dst_shard_meta

    def __str__(self):
        return (f"TransferOp({self.param_name}, src={self.src_rank}, dst={self.dst_rank}, "
                f"{self.src_meta} -> {self.dst_meta})")

    __repr__ = __str__

    def get_recv_tensor(self, device: torch.device) -> Tensor:
        """Receive buffer of the piece's shape (Suika/migration.py:285-287)."""
        return torch.empty(self.dst_meta.actual_shape(), dtype=self.dst_meta.dtype, device=device)

    def get_send_tensor(self, src_tensor: Tensor) -> Tensor:
        """The contiguous part of ``src_tensor`` this op sends (migration.py:290-312).

        A source shard at least as fine as the piece is sent whole (the tensor
        itself); otherwise the piece -- the reference's
        ``chunk(dst_deg / src_deg, slice_dim)[k].contiguous()``, or the rows
        of a vocab_pad piece -- is cut into a new tensor by the reshard
        engine on the tensor's GPU.  The copy is complete when this returns.
        """
        self.check_send(src_tensor.shape)
        src, piece = self.src_meta, self.dst_meta
        if piece.rows is None and src.tp_deg() >= piece.tp_deg():
            return src_tensor
        assert src_tensor.is_cuda, \
            (f"get_send_tensor: param {self.param_name} - the reshard engine runs on the GPU; "
             f"src_tensor is on {src_tensor.device}")
        from .plan import ReshardPlan
        name = self.param_name
        op = TransferOp(name, self.src_rank, self.dst_rank, src, piece, dst_shard_meta=piece)
        device = src_tensor.device
        with torch.cuda.device(device):
            plan, src_ptrs = ReshardPlan.from_sources([op], lambda r: {name: {"x": src_tensor}}, ["x"], device)
            try:
                out, dst_ptrs = plan.alloc_dst_ptrs(device)
                if len(dst_ptrs):
                    plan.gather_ptrs(src_ptrs, dst_ptrs)
            finally:
                plan.close()   # waits for the launch
        send = out[name]["x"]
        assert send.shape == piece.actual_shape(), \
            (f"get_send_tensor: param {name} - send_tensor shape {send.shape} mismatch with dst_meta "
             f"{piece.actual_shape()}")
        return send

    def check_send(self, src_shape) -> None:
        """The reference's preconditions of get_send_tensor (migration.py:293-294)."""
        assert torch.Size(src_shape) == self.src_meta.actual_shape(), \
            (f"get_send_tensor: param {self.param_name} - src_tensor shape {tuple(src_shape)} "
             f"mismatch with src_meta {self.src_meta.actual_shape()}")
        assert self.src_meta.slice_dim() == self.dst_meta.slice_dim() or \
            not self.src_meta.is_tp() or not self.dst_meta.is_tp(), \
            (f"get_send_tensor: param {self.param_name} - slice dim mismatch btw src "
             f"{self.src_meta.slice_dim()} and dst {self.dst_meta.slice_dim()}")


_SHAPE_PAD = [(0,) * (8 - n) for n in range(9)]


def _encode_layout(pl: ParamLayout, names: Dict[str, int], objs: List[TensorMeta]):
    """A layout as an [n, 21] int64 sr_meta table, rank by rank in the
    layout's order; ``names`` maps tensor names to ids and ``objs`` receives
    the TensorMeta of every row (the host extension walks the dicts)."""
    from . import _lib
    return _lib.host().encode_layout(pl.layout, names, objs)


class Schedule(list):
    """The ops ``schedule_param_transfer`` returns: a list, which also keeps
    each op's destination rank as an array, so that the drop-in call takes a
    rank's ops without reading every op's attributes, and the tables its ops
    were made from (the sr_op table, both layouts' sr_meta tables and meta
    objects, each op's piece meta), so that the call encodes them without
    walking their metas' attributes.  Any change to the list drops both (the
    call then scans it and walks the metas)."""

    def __init__(self, ops=(), dst_ranks=None, tables=None):
        super().__init__(ops)
        n = len(self)
        self._dst_ranks = dst_ranks if dst_ranks is not None and len(dst_ranks) == n else None
        self._positions: Dict[int, np.ndarray] = {}
        self._tables = tables if tables is not None and len(tables[0]) == n else None

    def positions_of(self, rank: int) -> Optional[np.ndarray]:
        """Positions of ``rank``'s ops in schedule order, or None when the
        list has changed since it was scheduled."""
        if self._dst_ranks is None:
            return None
        rank = int(rank)
        found = self._positions.get(rank)
        if found is None:
            found = self._positions[rank] = np.flatnonzero(self._dst_ranks == rank)
        return found

    def encoding(self):
        """The host extension's view of the tables (a ScheduleEncoding), or
        None when the list has changed since it was scheduled."""
        if self._tables is None:
            return None
        from . import _lib
        return _lib.host().ScheduleEncoding(self, self._tables)

    def _changed(self) -> None:
        self._dst_ranks = None
        self._positions = {}
        self._tables = None


def _dropping_tables(name):
    method = getattr(list, name)

    def change(self, *args, **kwargs):
        self._changed()
        return method(self, *args, **kwargs)
    change.__name__ = name
    return change


for _name in ("__setitem__", "__delitem__", "__iadd__", "__imul__", "append", "extend", "insert", "pop",
              "remove", "sort", "reverse", "clear"):
    setattr(Schedule, _name, _dropping_tables(_name))


def schedule_param_transfer(source_param_layout: ParamLayout, target_param_layout: ParamLayout,
                            log_func: Optional[Callable] = None,
                            minimum_est_peers: Optional[int] = None) -> Schedule:
    """Greedy piece -> source assignment of Suika/migration.py:322-381.

    Every target tensor is cut into pieces at the largest source TP degree
    (``vocab_pad`` tensors: at the source shard boundaries); each piece goes
    to its own rank when owned there, otherwise to the owner with the
    smallest accumulated volume, preferring already-connected peers once
    ``minimum_est_peers`` are connected (1 with InfiniBand, else 2).  The
    greedy runs in the library (``sr_schedule``) on the layouts encoded as
    tables; the TransferOps reference the layouts' own TensorMeta objects.
    """
    import numpy as np
    from . import _lib
    spl, tpl = source_param_layout, target_param_layout
    if minimum_est_peers is None:
        minimum_est_peers = 1 if is_ib_enabled() else 2
    names: Dict[str, int] = {}
    src_objs: List[TensorMeta] = []
    dst_objs: List[TensorMeta] = []
    src = _encode_layout(spl, names, src_objs)
    dst = _encode_layout(tpl, names, dst_objs)
    if not src_objs:
        max([])   # the reference's max_tp_degree over an empty layout: ValueError
    n_ranks = len(spl.layout)
    max_tp = max(1, int(src[:, 14].max()))     # column 14: tp_deg
    cap = len(dst_objs) * max(max_tp, 2 * n_ranks + 1)
    ops = np.empty((max(cap, 1), _lib.SR_OP_WORDS), dtype=np.int64)
    n_ops = ctypes.c_int64()
    L = _lib.lib()
    rc = L.sr_schedule(_lib.as_int64_ptr(src), len(src_objs), n_ranks, _lib.as_int64_ptr(dst),
                       len(dst_objs), len(names), int(minimum_est_peers), _lib.as_int64_ptr(ops),
                       cap, ctypes.byref(n_ops))
    if rc != _lib.SR_OK:
        by_id = list(names)
        msg = re.sub(r"#(\d+)", lambda g: by_id[int(g.group(1))], _lib.last_error(L))
        raise _lib.PlanError(f"schedule_param_transfer: {msg}")

    # TransferOps over the layouts' own metas; a piece is its shard with
    # another tp meta (scale_to_tp) or a row interval (vocab_pad)
    table = ops[:n_ops.value]
    pieces: List[TensorMeta] = []
    schedule = Schedule(_lib.host().make_ops(table, list(names), src_objs, dst_objs, TransferOp, TensorMeta, pieces),
                        table[:, 2],   # column 2: dst_rank
                        (table, src, dst, src_objs, dst_objs, pieces))
    if log_func is not None:
        for op in schedule:
            if op.src_rank != op.dst_rank:
                log_func(f"schedule_param_transfer: {op.src_rank} > {op.dst_rank} transfer {op.param_name}")
    return schedule

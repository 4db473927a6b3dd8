"""Compile a destination rank's TransferOps into a library plan and run it.

``ReshardPlan`` is the bridge between the reference-shaped host API
(``TransferOp`` lists and ``{name: {field: Tensor}}`` state dicts, as used by
Suika/migration.py:397-556) and the C ABI of ``libsuika_reshard.so``:

* every (source rank, name, field) tensor becomes a source slot, every
  (name, field) of the destination a destination slot;
* every source rank becomes a peer with one contiguous buffer;
* every TransferOp x region x normal field becomes one ``sr_piece`` (in
  schedule order, fields in ``fields`` order), pad rows of vocab-parallel
  shards become ZERO pieces, and a ``recast`` target field (bf16) is written by
  the unpack of its f32 source field.

The lowering itself (regions, slots, pieces) runs in the library
(``sr_lower``); this class encodes the ops, metas and source shapes as int64
tables and maps the slots back to (rank, name, field) keys.

The plan is built once from shapes and dtypes and can then be executed on any
tensors of those shapes: ``pack`` and ``unpack`` are asynchronous on the
current HIP stream.
"""
from __future__ import annotations

import ctypes
import functools
import re
from dataclasses import dataclass
from typing import Callable, Dict, List, Mapping, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib
from .geometry import infer_dst_shard
from .meta import _SHAPE_PAD, TensorMeta, TransferOp

SrcKey = Tuple[int, str, str]   # (source rank, name, field)
DstKey = Tuple[str, str]        # (name, field)

_DTYPES = {
    torch.uint8: _lib.SR_DT_U8,
    torch.int8: _lib.SR_DT_U8,
    torch.bool: _lib.SR_DT_U8,
    torch.bfloat16: _lib.SR_DT_BF16,
    torch.float16: _lib.SR_DT_F16,
    torch.float32: _lib.SR_DT_F32,
    torch.float64: _lib.SR_DT_F64,
    torch.int32: _lib.SR_DT_I32,
    torch.int64: _lib.SR_DT_I64,
}
for _name in ("float8_e4m3fn", "float8_e5m2", "float8_e4m3fnuz", "float8_e5m2fnuz"):
    if hasattr(torch, _name):
        _DTYPES[getattr(torch, _name)] = _lib.SR_DT_U8


def sr_dtype(dtype: torch.dtype) -> int:
    assert dtype in _DTYPES, f"dtype {dtype} is not supported by the reshard engine"
    return _DTYPES[dtype]


@dataclass(frozen=True)
class PlanOptions:
    tile_bytes: int = 0          # 0 = library default
    max_blocks: int = 0          # 0 = one workgroup per tile
    nontemporal: bool = True     # streaming loads/stores (library default)
    skip_coverage: bool = False
    address_order: bool = True   # tiles ordered by tensor address (library default)
    xcd_order: bool = True       # tiles interleaved 8 ways, one eighth per XCD (default)
    row_groups: bool = True      # side-by-side strided pieces dealt out by row block (default)
    gather_only: bool = False    # build only the gather phase (no pack / unpack)

    @functools.cached_property
    def flags(self) -> int:
        """The SR_OPT_* flags of these options (computed once)."""
        return (0 if self.nontemporal else _lib.SR_OPT_TEMPORAL) | \
            (_lib.SR_OPT_SKIP_COVERAGE if self.skip_coverage else 0) | \
            (0 if self.address_order else _lib.SR_OPT_PIECE_ORDER) | \
            (0 if self.xcd_order else _lib.SR_OPT_NO_XCD_INTERLEAVE) | \
            (0 if self.row_groups else _lib.SR_OPT_NO_ROW_GROUPS) | \
            (_lib.SR_OPT_GATHER_ONLY if self.gather_only else 0)

    def to_c(self) -> _lib.SrPlanOptions:
        return _lib.SrPlanOptions(self.tile_bytes, self.max_blocks, self.flags, 0)


@dataclass(frozen=True)
class SlotSpec:
    shape: Tuple[int, ...]
    dtype: torch.dtype


def _spec_words(out: List[int], shape: Tuple[int, ...], dtype: torch.dtype, name: str, field: str) -> None:
    """Append one sr_src_spec row (dtype, ndim, shape[8])."""
    nd = len(shape)
    assert nd <= _lib.SR_MAX_DIMS, f"{name}/{field}: {nd}-D source"
    out.extend((sr_dtype(dtype), nd, *shape, *_SHAPE_PAD[nd]))


def _numel(shape: Sequence[int]) -> int:
    n = 1
    for s in shape:
        n *= int(s)
    return n


def _stream_handle(stream) -> ctypes.c_void_p:
    if stream is None:
        # the current stream's handle, without building a Stream object
        return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(torch.cuda.current_device()))
    if isinstance(stream, torch.cuda.Stream):
        return ctypes.c_void_p(stream.cuda_stream)
    return ctypes.c_void_p(int(stream))


def download(pairs: Sequence[Tuple[torch.Tensor, torch.Tensor]], stream=None) -> None:
    """Copy each device tensor of ``pairs`` (device, host) into its host
    tensor (``sr_download``: through the library's pinned windows, on
    ``stream`` after the work queued there); returns when the host tensors
    hold the bytes."""
    dev, host, nbytes = [], [], []
    cur = torch.cuda.current_device()
    for d, h in pairs:
        n = d.numel() * d.element_size()
        assert d.is_cuda and d.get_device() == cur and d.is_contiguous(), "download: source must be on the device"
        assert h.is_cpu and h.is_contiguous() and h.numel() * h.element_size() == n, \
            "download: destination must be a contiguous host tensor of the same size"
        if n:
            dev.append(d.data_ptr())
            host.append(h.data_ptr())
            nbytes.append(n)
    if not nbytes:
        return
    L = _lib.lib()
    k = len(nbytes)
    rc = L.sr_download((ctypes.c_void_p * k)(*dev), (ctypes.c_void_p * k)(*host), (ctypes.c_uint64 * k)(*nbytes),
                       k, _stream_handle(stream))
    _lib.check(rc, "sr_download", L)


class ReshardPlan:
    """Pack/unpack plan of one destination rank's share of a reshard."""

    def __init__(self, ops: Sequence[TransferOp],
                 src_specs: Mapping[SrcKey, SlotSpec],
                 fields: Sequence[str],
                 recast: Optional[Mapping[str, str]] = None,
                 options: Optional[PlanOptions] = None):
        """``src_specs`` gives the shape/dtype of every source (rank, name,
        field) the ops read; ``fields`` are the normal sub-fields moved;
        ``recast`` maps a bf16 destination field to the f32 field it is
        rounded from (e.g. ``{"param": "master"}``)."""
        self._setup(ops, fields, recast, options)
        spec_words: List[int] = []
        dtypes: List[torch.dtype] = []
        for op in self._ops:
            name = op.param_name
            for f in self.fields:
                spec = src_specs.get((op.src_rank, name, f))
                assert spec is not None, f"[{op.src_rank}]: param missing in source {name}/{f}"
                _spec_words(spec_words, tuple(spec.shape), spec.dtype, name, f)
                dtypes.append(spec.dtype)
        self._build(np.array(spec_words, dtype=np.int64), dtypes)

    @classmethod
    def from_sources(cls, ops: Sequence[TransferOp], source: Callable[[int], Mapping],
                     fields: Sequence[str], device: torch.device,
                     recast: Optional[Mapping[str, str]] = None,
                     options: Optional[PlanOptions] = None,
                     rank: Optional[int] = None,
                     host_ok: bool = False) -> Tuple["ReshardPlan", List[int]]:
        """The plan of ``ops`` with shapes and dtypes read from the source
        tensors themselves, and the address of every source slot (a uint64
        array).

        ``source(r)`` is rank ``r``'s state dict ``{name: {field: Tensor}}``.
        Each tensor is read once: it must be a contiguous CUDA tensor on
        ``device`` -- or, with ``host_ok``, a contiguous tensor in host
        memory, whose address is then a host address that only
        ``stage_pack_ptrs`` may be given (a source in host memory without
        ``host_ok`` raises ``_lib.HostSourceError``).  ``rank`` (the
        executing rank) only prefixes messages.
        """
        plan, src_ptrs, _ = cls._native(ops, source, fields, device, recast, options, rank, host_ok=host_ok)
        return plan, src_ptrs

    @classmethod
    def gather_sources(cls, ops: Sequence[TransferOp], source: Callable[[int], Mapping],
                       fields: Sequence[str], device: torch.device,
                       recast: Optional[Mapping[str, str]] = None,
                       options: Optional[PlanOptions] = None,
                       rank: Optional[int] = None,
                       stream=None, dst=None, ahead=None) -> Tuple["ReshardPlan", Dict[str, Dict[str, torch.Tensor]]]:
        """``from_sources``, the destination tensors and the gather into them
        on ``stream`` (default: the current stream), in one native call: the
        drop-in call's direct route.  The destinations are fresh tensors (as
        ``alloc_dst``), or ``dst`` ``{name: {field: tensor}}``, each checked
        against its slot (as ``bind_dst_ptrs``).  With ``ahead`` = ({name:
        tensor index}, blocks) -- blocks from the host extension's
        ``start_blocks``, which a helper thread is allocating --, the fresh
        tensors are built on those blocks where their sizes match.  Returns
        the plan (its kernels possibly still running: ``close`` waits for
        them) and the destinations."""
        plan, _, part = cls._native(ops, source, fields, device, recast, options, rank, gather=True,
                                    stream=_stream_handle(stream).value or 0, dst=dst, ahead=ahead)
        return plan, part

    @classmethod
    def _native(cls, ops, source, fields, device, recast, options, rank, gather=False, stream=0, dst=None,
                ahead=None, host_ok=False):
        self = cls.__new__(cls)
        self._configure(ops, fields, recast, options)
        dev_index = device.index if device.index is not None else torch.cuda.current_device()
        who = f"[{rank}]" if rank is not None else ""
        opt = self.options
        self._L = _lib.lib()
        # grouping, shards, tables, source checks, sr_lower and sr_plan_create
        # (and with `gather` the destinations and the launch) in one native call
        src_ptrs, part = self._adopt(_lib.host().plan_sources(
            self._ops, source, self.fields, [self._recast_of.get(f) for f in self.fields],
            infer_dst_shard, dev_index, who, opt.tile_bytes, opt.max_blocks, opt.flags,
            _lib.SR_TENSOR_DTYPE, _lib.SR_PIECE_DTYPE, gather, stream, dst, ahead, host_ok))
        return self, src_ptrs, part

    def _adopt(self, made):
        """The plan's state from plan_sources' result; returns the source
        addresses and the destinations."""
        (handle, self._names, self.dst_metas, self._op_names, self.dst_rank, self._dtypes, src_ptrs,
         self._src_arr, self._dst_arr, self._piece_arr, self.peers, self._src_rows, self._dst_rows,
         self._empty_rows, self.peer_bytes, info, part) = made
        self._handle = ctypes.c_void_p(handle)
        self.info = _lib.SrPlanInfo.from_buffer_copy(info)
        self.n_pieces = len(self._piece_arr)
        self._views = self._pieces_view = self._c_src_view = self._c_dst_view = None
        return src_ptrs, part

    @classmethod
    def gatherer(cls, source: Callable[[int], Mapping], fields: Sequence[str], device: torch.device,
                 recast: Optional[Mapping[str, str]] = None, options: Optional[PlanOptions] = None,
                 rank: Optional[int] = None, stream=None, encoding=None):
        """``gather_sources`` for many groups of ops with the same sources,
        fields, device, options and stream: what the groups share is checked
        and converted once.  ``encoding`` (the schedule's ``encoding()``)
        encodes the ops of that schedule from its tables.  Returns
        ``gather(ops, dst=None, ahead=None) -> (plan, destinations)``."""
        proto = cls.__new__(cls)
        proto._configure((), fields, recast, options)
        fields, recast, options, recast_of = proto.fields, proto.recast, proto.options, proto._recast_of
        recast_names = [recast_of.get(f) for f in fields]
        dev_index = device.index if device.index is not None else torch.cuda.current_device()
        who = f"[{rank}]" if rank is not None else ""
        # the stream: `stream`, else the device's current stream
        handle = torch._C._cuda_getCurrentRawStream(dev_index) if stream is None else _stream_handle(stream).value
        args = (infer_dst_shard, dev_index, who, options.tile_bytes, options.max_blocks, options.flags,
                _lib.SR_TENSOR_DTYPE, _lib.SR_PIECE_DTYPE, True, handle or 0)
        L, plan_sources = _lib.lib(), _lib.host().plan_sources

        def gather(ops, dst=None, ahead=None):
            self = cls.__new__(cls)
            self.fields, self.recast, self.options, self._recast_of, self._L = fields, recast, options, recast_of, L
            self._handle = ctypes.c_void_p()
            self._ops = ops
            _, part = self._adopt(plan_sources(ops, source, fields, recast_names, *args, dst, ahead, False, encoding))
            return self, part
        return gather

    def _configure(self, ops, fields, recast, options) -> None:
        """Fields, recast map and options, validated."""
        self._handle = ctypes.c_void_p()
        recast = dict(recast or {})
        for tgt, srcf in recast.items():
            assert tgt not in fields or tgt == srcf, \
                f"recast target {tgt!r} is also a copied field"
            assert srcf in fields, f"recast source field {srcf!r} is not moved"
        self.fields = list(fields)
        self.recast = recast
        self.options = options or PlanOptions()
        self._ops = list(ops)
        self._recast_of = {sf: t for t, sf in recast.items()}   # f32 field -> its bf16 target

    def _setup(self, ops, fields, recast, options) -> None:
        """Everything but the source specs: validation, destination shards and
        the op / meta tables of sr_lower."""
        self._configure(ops, fields, recast, options)
        ops = self._ops
        self._op_names = [op.param_name for op in ops]
        dst_ranks = {op.dst_rank for op in ops}
        assert len(dst_ranks) <= 1, f"ops target several ranks {sorted(dst_ranks)}"
        self.dst_rank = dst_ranks.pop() if dst_ranks else None

        # the destination shard of every tensor: attached by the schedule, else
        # inferred from the tensor's pieces
        by_name: Dict[str, List[TransferOp]] = {}
        for op in ops:
            by_name.setdefault(op.param_name, []).append(op)
        self._names = list(by_name)
        name_id = {name: i for i, name in enumerate(self._names)}
        self.dst_metas: Dict[str, TensorMeta] = {}
        for name, name_ops in by_name.items():
            shard = getattr(name_ops[0], "dst_shard_meta", None)
            self.dst_metas[name] = shard if shard is not None else infer_dst_shard(name_ops)

        # sr_lower's op and meta tables (the host extension reads the ops)
        self._metas_arr, self._ops_arr = _lib.host().encode_ops(ops, self.dst_metas, name_id)
        self._n_metas = len(self._metas_arr)

    def _build(self, specs_arr: np.ndarray, dtypes: List[torch.dtype]) -> None:
        """sr_lower on the tables, then sr_plan_create on its output."""
        L = self._L = _lib.lib()
        ops, nf = self._ops, len(self.fields)
        self._dtypes = dtypes   # torch dtype of the source of (op k, field f) at k * nf + f
        # one torch dtype per (tensor, field) across sources (the library
        # compares element types, which several torch dtypes share)
        for f in range(nf):
            if len(set(dtypes[f::nf])) > 1:
                seen: Dict[str, torch.dtype] = {}
                for k, op in enumerate(ops):
                    dt = seen.setdefault(op.param_name, dtypes[k * nf + f])
                    assert dt == dtypes[k * nf + f], \
                        f"{op.param_name}/{self.fields[f]}: dtype differs between sources"
        recast_arr = np.array([1 if f in self._recast_of else 0 for f in self.fields] or [0], dtype=np.int64)
        low = ctypes.POINTER(_lib.SrLowering)()
        rc = L.sr_lower(_lib.as_int64_ptr(self._metas_arr), self._n_metas, _lib.as_int64_ptr(self._ops_arr),
                        len(ops), _lib.as_int64_ptr(specs_arr), nf, _lib.as_int64_ptr(recast_arr),
                        ctypes.byref(low))
        if rc != _lib.SR_OK:
            names = self._names
            msg = re.sub(r"#(\d+)", lambda g: names[int(g.group(1))], _lib.last_error(L))
            raise _lib.PlanError(f"sr_lower: {_lib.STATUS_NAMES.get(rc, rc)}: {msg}")
        try:
            lw = low.contents
            self._src_arr = _lib.copy_table(lw.src, lw.n_src, _lib.SR_TENSOR_DTYPE)
            self._dst_arr = _lib.copy_table(lw.dst, lw.n_dst, _lib.SR_TENSOR_DTYPE)
            self._piece_arr = _lib.copy_table(lw.pieces, lw.n_pieces, _lib.SR_PIECE_DTYPE)
            self.peers: List[int] = _lib.copy_table(lw.peer_rank, lw.n_peers, np.int64).tolist()
            src_rows = _lib.copy_table(lw.src_key, lw.n_src, (np.int64, _lib.SR_KEY_WORDS))
            self._dst_rows = _lib.copy_table(lw.dst_key, lw.n_dst, (np.int64, _lib.SR_KEY_WORDS))
            self._empty_rows = _lib.copy_table(lw.empty, lw.n_empty, (np.int64, _lib.SR_KEY_WORDS))
        finally:
            L.sr_lowering_destroy(low)
        self._src_rows = src_rows
        self._views = None

        self.n_pieces = len(self._piece_arr)
        self._pieces_view = self._c_src_view = self._c_dst_view = None
        opt = self.options.to_c()
        rc = L.sr_plan_create(_lib.as_tensors(self._src_arr), len(self._src_arr),
                              _lib.as_tensors(self._dst_arr), len(self._dst_arr), len(self.peers),
                              _lib.as_pieces(self._piece_arr), self.n_pieces, ctypes.byref(opt),
                              ctypes.byref(self._handle))
        _lib.check(rc, "sr_plan_create", L)
        self.peer_bytes: List[int] = []
        for i in range(len(self.peers)):
            b = ctypes.c_uint64()
            _lib.check(L.sr_plan_peer_bytes(self._handle, i, ctypes.byref(b)), "sr_plan_peer_bytes", L)
            self.peer_bytes.append(int(b.value))
        info = _lib.SrPlanInfo()
        _lib.check(L.sr_plan_info_get(self._handle, ctypes.byref(info)), "sr_plan_info_get", L)
        self.info = info

    # ----------------------------------------------- slots as (rank, name, field)
    def _dst_entry(self, row) -> Tuple[DstKey, SlotSpec]:
        k, f, is_recast, _, nd = row[:5]
        name = self._ops[k].param_name
        field = self.fields[f]
        shape = tuple(row[5:5 + nd])
        if is_recast:
            return (name, self._recast_of[field]), SlotSpec(shape, torch.bfloat16)
        return (name, field), SlotSpec(shape, self._dtypes[k * len(self.fields) + f])

    def _key_views(self):
        """Slot keys and specs as dicts, built on first use."""
        if self._views is None:
            nf = len(self.fields)
            src_keys: List[SrcKey] = []
            src_specs: Dict[SrcKey, SlotSpec] = {}
            for k, f, _, _, nd, *shape in self._src_rows.tolist():
                op = self._ops[k]
                key = (op.src_rank, op.param_name, self.fields[f])
                src_keys.append(key)
                src_specs[key] = SlotSpec(tuple(shape[:nd]), self._dtypes[k * nf + f])
            dst_keys: List[DstKey] = []
            dst_specs: Dict[DstKey, SlotSpec] = {}
            for row in self._dst_rows.tolist():
                key, spec = self._dst_entry(row)
                dst_keys.append(key)
                dst_specs[key] = spec
            empty = dict(self._dst_entry(row) for row in self._empty_rows.tolist())
            self._views = (src_keys, src_specs, dst_keys, dst_specs, empty)
        return self._views

    @property
    def src_keys(self) -> List[SrcKey]:
        """(source rank, name, field) of every source slot, in slot order."""
        return self._key_views()[0]

    @property
    def src_specs(self) -> Dict[SrcKey, SlotSpec]:
        return self._key_views()[1]

    @property
    def dst_keys(self) -> List[DstKey]:
        """(name, field) of every destination slot, in slot order."""
        return self._key_views()[2]

    @property
    def dst_specs(self) -> Dict[DstKey, SlotSpec]:
        return self._key_views()[3]

    @property
    def empty_dst(self) -> Dict[DstKey, SlotSpec]:
        """Zero-element destinations: no slot, no piece."""
        return self._key_views()[4]

    def alloc_dst_ptrs(self, device) -> Tuple[Dict[str, Dict[str, torch.Tensor]], List[int]]:
        """Fresh destination tensors (as ``alloc_dst``) and the device
        address of every destination slot (a uint64 array), straight from
        the slot table."""
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        recast_names = [self._recast_of.get(f) for f in self.fields]
        out, ptrs = _lib.host().alloc_dst(self._dst_rows.reshape(-1, _lib.SR_KEY_WORDS),
                                          self._empty_rows.reshape(-1, _lib.SR_KEY_WORDS),
                                          self._op_names, self.fields, recast_names, self._dtypes, device)
        return out, ptrs

    def bind_dst_ptrs(self, dst: Mapping[str, Mapping[str, torch.Tensor]], device) -> List[int]:
        """Addresses of caller-provided destination tensors in slot order,
        each checked against its slot (contiguous, planned shape and dtype,
        on ``device``)."""
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        recast_names = [self._recast_of.get(f) for f in self.fields]
        return _lib.host().bind_dst(dst, self._dst_rows.reshape(-1, _lib.SR_KEY_WORDS), self._op_names,
                                    self.fields, recast_names, self._dtypes, device)

    # -------------------------------------------------------------- sizes
    @property
    def pack_bytes(self) -> int:
        return int(self.info.pack_bytes_read + self.info.pack_bytes_written)

    @property
    def unpack_bytes(self) -> int:
        return int(self.info.unpack_bytes_read + self.info.unpack_bytes_written)

    def piece_offset(self, k: int) -> int:
        off = ctypes.c_uint64()
        _lib.check(self._L.sr_plan_piece_offset(self._handle, k, ctypes.byref(off)),
                   "sr_plan_piece_offset", self._L)
        return int(off.value)

    # ------------------------------------------------- the C tables, read back
    @property
    def pieces(self) -> list:
        """The sr_piece records, as named tuples (built on first use)."""
        if self._pieces_view is None:
            self._pieces_view = [_lib.PieceRecord(*r) for r in self._piece_arr.tolist()]
        return self._pieces_view

    @property
    def c_src(self) -> list:
        """The source sr_tensor records, as named tuples."""
        if self._c_src_view is None:
            self._c_src_view = [_lib.TensorRecord(*r) for r in self._src_arr.tolist()]
        return self._c_src_view

    @property
    def c_dst(self) -> list:
        """The destination sr_tensor records, as named tuples."""
        if self._c_dst_view is None:
            self._c_dst_view = [_lib.TensorRecord(*r) for r in self._dst_arr.tolist()]
        return self._c_dst_view

    # --------------------------------------------------------- allocation
    def alloc_buffers(self, device) -> List[torch.Tensor]:
        """One byte buffer per peer (torch's allocator aligns to 512 bytes)."""
        return [torch.empty(max(1, n), dtype=torch.uint8, device=device) for n in self.peer_bytes]

    ARENA_ALIGN = 256

    def arena_layout(self) -> Tuple[int, Dict[DstKey, int]]:
        """Byte size of a destination arena and the offset of every
        destination tensor in it: field by field (all ``param`` tensors, then
        ``master``, ...), tensors in plan order within a field, each at a
        256-byte aligned offset.  A field's tensors are thus one contiguous
        span, e.g. a flat parameter buffer."""
        fields: List[str] = []
        for _, f in self.dst_keys:
            if f not in fields:
                fields.append(f)
        offsets: Dict[DstKey, int] = {}
        end = 0
        a = self.ARENA_ALIGN
        for f in fields:
            for key in self.dst_keys:
                if key[1] != f:
                    continue
                spec = self.dst_specs[key]
                end = (end + a - 1) // a * a
                offsets[key] = end
                end += _numel(spec.shape) * spec.dtype.itemsize
        return end, offsets

    def alloc_dst(self, device, arena: bool = False) -> Dict[str, Dict[str, torch.Tensor]]:
        """Fresh destination tensors, one per (name, field).  With ``arena``
        they share the storage of one allocation laid out by ``arena_layout`` (one
        allocator call instead of one per tensor; a model adopting them with
        ``load_state_dict(assign=True)`` keeps them in place)."""
        if not arena:
            return self.alloc_dst_ptrs(device)[0]
        out: Dict[str, Dict[str, torch.Tensor]] = {}
        for (name, field), spec in self.empty_dst.items():
            out.setdefault(name, {})[field] = torch.empty(spec.shape, dtype=spec.dtype, device=device)
        total, offsets = self.arena_layout()
        buf = torch.empty(max(1, total), dtype=torch.uint8, device=device)
        names, fields, rows, dtypes = [], [], [], []
        for (name, field) in self.dst_keys:
            spec = self.dst_specs[(name, field)]
            names.append(name)
            fields.append(field)
            rows.extend((offsets[(name, field)], len(spec.shape), *spec.shape, *_SHAPE_PAD[len(spec.shape)]))
            dtypes.append(spec.dtype)
        views = _lib.host().arena_views(buf, names, fields, np.array(rows, dtype=np.int64).reshape(-1, 10),
                                        dtypes)
        for name, entry in views.items():
            out.setdefault(name, {}).update(entry)
        return out

    # ---------------------------------------------------------- execution
    @staticmethod
    def _check_tensor(t: torch.Tensor, spec: SlotSpec, what, device: int) -> int:
        assert isinstance(t, torch.Tensor), f"{what}: not a tensor"
        assert t.is_cuda, f"{what}: tensor is on {t.device}, the reshard engine needs HBM"
        assert t.get_device() == device, \
            f"{what}: tensor is on cuda:{t.get_device()}, the kernels run on the current device cuda:{device}"
        assert t.is_contiguous(), f"{what}: tensor is not contiguous"
        assert tuple(t.shape) == tuple(spec.shape), f"{what}: shape {tuple(t.shape)} != {spec.shape}"
        assert t.dtype == spec.dtype, f"{what}: dtype {t.dtype} != {spec.dtype}"
        return t.data_ptr()

    def src_pointers(self, sources: Mapping[int, Mapping[str, Mapping[str, torch.Tensor]]]):
        dev = torch.cuda.current_device()
        ptrs = []
        for key in self.src_keys:
            rank, name, field = key
            t = sources[rank][name][field]
            ptrs.append(self._check_tensor(t, self.src_specs[key], key, dev))
        return ptrs

    def dst_pointers(self, dst: Mapping[str, Mapping[str, torch.Tensor]]):
        return self.bind_dst_ptrs(dst, torch.device("cuda", torch.cuda.current_device()))

    def buf_pointers(self, buffers: Sequence[torch.Tensor]):
        assert len(buffers) == len(self.peers), f"{len(buffers)} buffers for {len(self.peers)} peers"
        dev = torch.cuda.current_device()
        ptrs = []
        for i, b in enumerate(buffers):
            assert b.is_cuda and b.is_contiguous(), f"buffer {i} must be a contiguous HBM tensor"
            assert b.get_device() == dev, \
                f"buffer {i} is on cuda:{b.get_device()}, the kernels run on the current device cuda:{dev}"
            assert b.numel() * b.element_size() >= self.peer_bytes[i], \
                f"buffer {i} holds {b.numel() * b.element_size()} bytes, needs {self.peer_bytes[i]}"
            ptrs.append(b.data_ptr())
        return ptrs

    @staticmethod
    def _carray(ptrs):
        """A pointer array for the C ABI: a uint64 numpy array is passed by
        address (no copy; the caller keeps it alive for the call); a list is
        converted."""
        if isinstance(ptrs, np.ndarray):
            assert ptrs.dtype == np.uint64 and ptrs.flags["C_CONTIGUOUS"], "address arrays are contiguous uint64"
            return ptrs.__array_interface__["data"][0]
        return (ctypes.c_void_p * max(1, len(ptrs)))(*ptrs)

    def pack_ptrs(self, src_ptrs: List[int], buf_ptrs: List[int], stream=None) -> None:
        rc = self._L.sr_pack(self._handle, self._carray(src_ptrs), self._carray(buf_ptrs),
                                _stream_handle(stream))
        _lib.check(rc, "sr_pack", self._L)

    def unpack_ptrs(self, buf_ptrs: List[int], dst_ptrs: List[int], stream=None) -> None:
        rc = self._L.sr_unpack(self._handle, self._carray(buf_ptrs), self._carray(dst_ptrs),
                                  _stream_handle(stream))
        _lib.check(rc, "sr_unpack", self._L)

    def gather_ptrs(self, src_ptrs: List[int], dst_ptrs: List[int], stream=None) -> None:
        rc = self._L.sr_gather(self._handle, self._carray(src_ptrs), self._carray(dst_ptrs),
                               _stream_handle(stream))
        _lib.check(rc, "sr_gather", self._L)

    def stage_pack_ptrs(self, src_ptrs, buf_ptrs: List[int], stream=None) -> None:
        """``sr_stage_pack``: the pack, for sources in host memory (or on the
        device), into device peer buffers, through the library's pinned
        windows; returns once the host sources have been read."""
        rc = self._L.sr_stage_pack(self._handle, self._carray(src_ptrs), self._carray(buf_ptrs),
                                   _stream_handle(stream))
        _lib.check(rc, "sr_stage_pack", self._L)

    def gather_noalloc_ptrs(self, src_ptrs: List[int], dst_ptrs: List[int], stream=None) -> None:
        """``sr_gather_noalloc``: the same gather with its device tables in
        the library's static per-GPU scratch (no device allocation); calls
        that overlap on one GPU race for it."""
        rc = self._L.sr_gather_noalloc(self._handle, self._carray(src_ptrs), self._carray(dst_ptrs),
                                       _stream_handle(stream))
        _lib.check(rc, "sr_gather_noalloc", self._L)

    def gather(self, sources, dst, stream=None) -> None:
        """Source shards -> destination shards directly (async on ``stream``)."""
        self.gather_ptrs(self.src_pointers(sources), self.dst_pointers(dst), stream)

    @property
    def gather_bytes(self) -> int:
        return int(self.info.gather_bytes_read + self.info.gather_bytes_written)

    def pack(self, sources, buffers, stream=None) -> None:
        """Source shards -> peer buffers (async on ``stream``)."""
        self.pack_ptrs(self.src_pointers(sources), self.buf_pointers(buffers), stream)

    def unpack(self, buffers, dst, stream=None) -> None:
        """Peer buffers -> destination shards (async on ``stream``)."""
        self.unpack_ptrs(self.buf_pointers(buffers), self.dst_pointers(dst), stream)

    def pack_host_ptrs(self, src_ptrs, buf_ptrs) -> None:
        """``sr_pack_host``: the pack from host-memory sources into host
        buffers (a null buffer address skips its peer), on host threads."""
        rc = self._L.sr_pack_host(self._handle, self._carray(src_ptrs), self._carray(buf_ptrs))
        _lib.check(rc, "sr_pack_host", self._L)

    def stage_pack(self, sources, buffers, stream=None) -> None:
        """Source shards in host memory (or on the device) -> peer buffers on
        the device (``sr_stage_pack``); the buffers then hold what ``pack``
        writes from the same contents."""
        ptrs = []
        for key in self.src_keys:
            rank, name, field = key
            t = sources[rank][name][field]
            spec = self.src_specs[key]
            assert isinstance(t, torch.Tensor) and t.is_contiguous(), f"{key}: not a contiguous tensor"
            assert tuple(t.shape) == tuple(spec.shape) and t.dtype == spec.dtype, \
                f"{key}: {tuple(t.shape)} {t.dtype} != {spec.shape} {spec.dtype}"
            assert t.is_cpu or t.get_device() == torch.cuda.current_device(), f"{key}: on {t.device}"
            ptrs.append(t.data_ptr())
        self.stage_pack_ptrs(ptrs, self.buf_pointers(buffers), stream)

    def close(self) -> None:
        if getattr(self, "_handle", None) is not None and self._handle.value:
            self._L.sr_plan_destroy(self._handle)
            self._handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

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

The plan is built once from shapes and dtypes and can then be executed on any
tensors of those shapes: ``pack`` and ``unpack`` are asynchronous on the
current HIP stream.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, List, Mapping, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib
from .geometry import infer_dst_shard, local_matrix, lower_op, pad_boxes, view_axis
from .meta import TensorMeta, TransferOp

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


@dataclass
class PlanOptions:
    tile_bytes: int = 0          # 0 = library default
    max_blocks: int = 0          # 0 = one workgroup per tile
    nontemporal: bool = True     # streaming loads/stores (library default)
    skip_coverage: bool = False
    address_order: bool = True   # tiles ordered by tensor address (library default)
    xcd_order: bool = True       # tiles interleaved 8 ways, one eighth per XCD (default)
    row_groups: bool = True      # side-by-side strided pieces dealt out by row block (default)

    def to_c(self) -> _lib.SrPlanOptions:
        flags = (0 if self.nontemporal else _lib.SR_OPT_TEMPORAL) | \
                (_lib.SR_OPT_SKIP_COVERAGE if self.skip_coverage else 0) | \
                (0 if self.address_order else _lib.SR_OPT_PIECE_ORDER) | \
                (0 if self.xcd_order else _lib.SR_OPT_NO_XCD_INTERLEAVE) | \
                (0 if self.row_groups else _lib.SR_OPT_NO_ROW_GROUPS)
        return _lib.SrPlanOptions(self.tile_bytes, self.max_blocks, flags, 0)


@dataclass(frozen=True)
class SlotSpec:
    shape: Tuple[int, ...]
    dtype: torch.dtype


def _geometry_key(m: TensorMeta) -> tuple:
    """What region lowering depends on: global shape, shard and kind (not
    the name or dtype; TensorMeta's own equality ignores the shard index)."""
    return (tuple(int(d) for d in m.shape), None if m.tp_meta is None else tuple(m.tp_meta),
            m.kind, tuple(m.kind_args), m.rows)


def _numel(shape: Sequence[int]) -> int:
    n = 1
    for s in shape:
        n *= int(s)
    return n


def _matrix_of(shape: Sequence[int], view: int) -> Tuple[int, int]:
    shape = [int(s) for s in shape]
    if not shape:
        return 1, 1
    if view == 1:
        r = 1
        for s in shape[:-1]:
            r *= s
        return r, shape[-1]
    c = 1
    for s in shape[1:]:
        c *= s
    return shape[0], c


def _stream_handle(stream) -> ctypes.c_void_p:
    if stream is None:
        stream = torch.cuda.current_stream()
    if isinstance(stream, torch.cuda.Stream):
        return ctypes.c_void_p(stream.cuda_stream)
    return ctypes.c_void_p(int(stream))


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
        self._handle = ctypes.c_void_p()
        recast = dict(recast or {})
        for tgt, srcf in recast.items():
            assert tgt not in fields or tgt == srcf, \
                f"recast target {tgt!r} is also a copied field"
            assert srcf in fields, f"recast source field {srcf!r} is not moved"
        self.fields = list(fields)
        self.recast = recast
        self.options = options or PlanOptions()

        by_name: Dict[str, List[TransferOp]] = {}
        for op in ops:
            by_name.setdefault(op.param_name, []).append(op)
        dst_ranks = {op.dst_rank for op in ops}
        assert len(dst_ranks) <= 1, f"ops target several ranks {sorted(dst_ranks)}"
        self.dst_rank = dst_ranks.pop() if dst_ranks else None

        self.peers: List[int] = sorted({op.src_rank for op in ops})
        peer_index = {r: i for i, r in enumerate(self.peers)}

        self.src_keys: List[SrcKey] = []
        src_index: Dict[SrcKey, int] = {}
        self.src_specs: Dict[SrcKey, SlotSpec] = {}
        self.dst_keys: List[DstKey] = []
        dst_index: Dict[DstKey, int] = {}
        self.dst_specs: Dict[DstKey, SlotSpec] = {}
        self.dst_metas: Dict[str, TensorMeta] = {}

        # rows of the C tables (sr_tensor / sr_piece field order), converted
        # to arrays in one step: thousands of ctypes records cost milliseconds
        c_src: List[tuple] = []
        c_dst: List[tuple] = []
        c_pieces: List[tuple] = []

        # Slots are made once per (tensor, field); the 2-D view ``rc`` is the
        # same for every field of a tensor and is computed by the caller.
        def src_slot(key: SrcKey, rc: Tuple[int, int]) -> int:
            if key not in src_index:
                spec = src_specs[key]
                src_index[key] = len(self.src_keys)
                self.src_keys.append(key)
                self.src_specs[key] = spec
                c_src.append((rc[0], rc[1], sr_dtype(spec.dtype), 0))
            return src_index[key]

        def dst_slot(key: DstKey, shape: Tuple[int, ...], rc: Tuple[int, int], dtype: torch.dtype) -> int:
            if key not in dst_index:
                dst_index[key] = len(self.dst_keys)
                self.dst_keys.append(key)
                self.dst_specs[key] = SlotSpec(shape, dtype)
                c_dst.append((rc[0], rc[1], sr_dtype(dtype), 0))
            else:
                assert self.dst_specs[key].dtype == dtype, \
                    f"{key}: sources disagree on dtype ({self.dst_specs[key].dtype} vs {dtype})"
            return dst_index[key]

        recast_of = {sf: t for t, sf in recast.items()}   # f32 field -> its bf16 target

        self.empty_dst: Dict[DstKey, SlotSpec] = {}   # zero-element destinations (no pieces)
        lowered: Dict[tuple, list] = {}
        self.piece_owner: List[Tuple[str, int]] = []   # (name, peer) per piece
        for name, name_ops in by_name.items():
            dst_shard = infer_dst_shard(name_ops)
            self.dst_metas[name] = dst_shard
            view = view_axis(dst_shard, *[op.src_meta for op in name_ops])
            field_dtype: Dict[str, torch.dtype] = {}
            for op in name_ops:
                checked = set()
                for f in self.fields:
                    key = (op.src_rank, name, f)
                    assert key in src_specs, f"[{op.src_rank}]: param missing in source {name}/{f}"
                    shape = tuple(src_specs[key].shape)
                    if shape not in checked:
                        op.check_send(shape)
                        checked.add(shape)
                    field_dtype.setdefault(f, src_specs[key].dtype)
                    assert field_dtype[f] == src_specs[key].dtype, \
                        f"{name}/{f}: dtype differs between sources"
            shape = tuple(int(d) for d in dst_shard.actual_shape())
            if _numel(shape) == 0:
                # nothing to move: an empty tensor per field, as clone() of an
                # empty piece gives in the reference (migration.py:538)
                for f in self.fields:
                    self.empty_dst[(name, f)] = SlotSpec(shape, field_dtype[f])
                    for tgt, sf in recast.items():
                        if sf == f:
                            self.empty_dst[(name, tgt)] = SlotSpec(shape, torch.bfloat16)
                continue
            # destination slots of every field, then the pieces that fill them
            drc = local_matrix(dst_shard, view)
            dslot: Dict[str, int] = {}
            for f in self.fields:
                dslot[f] = dst_slot((name, f), shape, drc, field_dtype[f])
                tgt = recast_of.get(f)
                if tgt is not None:
                    assert field_dtype[f] == torch.float32, f"{name}/{f}: recast source must be float32"
                    dslot[tgt] = dst_slot((name, tgt), shape, drc, torch.bfloat16)
            for op in name_ops:
                peer = peer_index[op.src_rank]
                if not self.fields:
                    continue
                src_rc = _matrix_of(src_specs[(op.src_rank, name, self.fields[0])].shape, view)
                sslot = {f: src_slot((op.src_rank, name, f), src_rc) for f in self.fields}
                # regions depend only on the shard geometry, which repeats
                # from layer to layer: lower each distinct geometry once
                gkey = (_geometry_key(op.src_meta), _geometry_key(op.dst_meta), _geometry_key(dst_shard))
                regions = lowered.get(gkey)
                if regions is None:
                    regions = lowered[gkey] = lower_op(op, dst_shard)
                for reg in regions:
                    for f in self.fields:
                        s = sslot[f]
                        tgt = recast_of.get(f)
                        if tgt is not None:
                            kind, d, d2 = _lib.SR_PIECE_RECAST, dslot[f], dslot[tgt]
                        else:
                            kind, d, d2 = _lib.SR_PIECE_COPY, dslot[f], -1
                        c_pieces.append((kind, peer, s, d, d2, 0, reg.rows, reg.cols,
                                         reg.src_row, reg.src_col, reg.dst_row, reg.dst_col))
                        self.piece_owner.append((name, peer))
            for box in pad_boxes(dst_shard, view):
                for f, slot in dslot.items():
                    c_pieces.append((_lib.SR_PIECE_ZERO, 0, -1, slot, -1, 0,
                                     box.rows, box.cols, 0, 0, box.row, box.col))
                    self.piece_owner.append((name, -1))

        self.n_pieces = len(c_pieces)
        self._src_arr = np.array(c_src, dtype=_lib.SR_TENSOR_DTYPE).reshape(-1)
        self._dst_arr = np.array(c_dst, dtype=_lib.SR_TENSOR_DTYPE).reshape(-1)
        self._piece_arr = np.array(c_pieces, dtype=_lib.SR_PIECE_DTYPE).reshape(-1)
        self._pieces_view = self._c_src_view = self._c_dst_view = None
        L = self._L = _lib.lib()
        opt = self.options.to_c()
        rc = L.sr_plan_create(_lib.as_tensors(self._src_arr), len(c_src),
                              _lib.as_tensors(self._dst_arr), len(c_dst), len(self.peers),
                              _lib.as_pieces(self._piece_arr), len(c_pieces), ctypes.byref(opt),
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
        they are views of one allocation laid out by ``arena_layout`` (one
        allocator call instead of one per tensor; a model adopting them with
        ``load_state_dict(assign=True)`` keeps them in place)."""
        out: Dict[str, Dict[str, torch.Tensor]] = {}
        for (name, field), spec in self.empty_dst.items():
            out.setdefault(name, {})[field] = torch.empty(spec.shape, dtype=spec.dtype, device=device)
        if not arena:
            for (name, field) in self.dst_keys:
                spec = self.dst_specs[(name, field)]
                out.setdefault(name, {})[field] = torch.empty(spec.shape, dtype=spec.dtype, device=device)
            return out
        total, offsets = self.arena_layout()
        buf = torch.empty(max(1, total), dtype=torch.uint8, device=device)
        for (name, field) in self.dst_keys:
            spec = self.dst_specs[(name, field)]
            off = offsets[(name, field)]
            n = _numel(spec.shape) * spec.dtype.itemsize
            out.setdefault(name, {})[field] = buf[off:off + n].view(spec.dtype).view(spec.shape)
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
        dev = torch.cuda.current_device()
        return [self._check_tensor(dst[name][field], self.dst_specs[(name, field)], (name, field), dev)
                for (name, field) in self.dst_keys]

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
    def _carray(ptrs: List[int]) -> ctypes.Array:
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

    def close(self) -> None:
        if getattr(self, "_handle", None) is not None and self._handle.value:
            self._L.sr_plan_destroy(self._handle)
            self._handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

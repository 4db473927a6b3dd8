"""Shard geometry on the host: which global elements a shard holds and where.

Used to cut synthetic shards from global tensors (benchmark and smoke
inputs) and to infer a destination shard from its pieces.  The plan's region
moves are computed in the library (``sr_lower``) from the same definitions.

Every tensor is viewed as a row-major 2-D matrix ``[R, C]``:
  * split along dim 0 (column-parallel weight/bias, embeddings, 1-D tensors):
    ``R = shape[0]``, ``C = prod(shape[1:])``;
  * split along the last dim (row-parallel weight): ``R = prod(shape[:-1])``,
    ``C = shape[-1]``.
A shard is a list of bands ``Seg``: a rectangle of the global matrix and the
position of the same rectangle in the shard's local matrix.  Padding rows of a
``vocab_pad`` shard are listed separately (they hold zeros and have no global
counterpart).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Tuple

from .meta import CHUNK, QKV_HEADS, VOCAB_PAD, TensorMeta, TransferOp


@dataclass(frozen=True)
class Seg:
    g_row: int   # origin in the global [R, C] matrix
    g_col: int
    l_row: int   # origin in the shard's local matrix
    l_col: int
    rows: int
    cols: int


@dataclass(frozen=True)
class Box:
    row: int
    col: int
    rows: int
    cols: int


def _prod(xs) -> int:
    n = 1
    for x in xs:
        n *= int(x)
    return n


def split_axis(meta: TensorMeta) -> Optional[int]:
    """0 = rows are split, 1 = columns are split, None = not split."""
    if not meta.is_tp():
        return None
    nd = len(meta.shape)
    d = meta.slice_dim() % nd if nd > 0 else 0
    if d == 0:
        return 0
    if d == nd - 1:
        return 1
    raise AssertionError(f"{meta.name}: slice_dim {meta.slice_dim()} of a {nd}-D tensor "
                         "is neither the first nor the last dim")


def view_axis(*metas: TensorMeta) -> int:
    """Matrix view shared by all shards of one tensor: 1 if any of them is
    split along the last dim, else 0."""
    axes = {split_axis(m) for m in metas} - {None}
    assert len(axes) <= 1, f"{metas[0].name}: shards split along different dims"
    return axes.pop() if axes else 0


def _matrix(shape, view: int) -> Tuple[int, int]:
    shape = [int(s) for s in shape]
    if len(shape) == 0:
        return 1, 1
    if view == 1:
        return _prod(shape[:-1]), shape[-1]
    return shape[0], _prod(shape[1:])


def global_matrix(meta: TensorMeta, view: Optional[int] = None) -> Tuple[int, int]:
    """``[R, C]`` of the unsharded (and unpadded) tensor."""
    return _matrix(meta.shape, view_axis(meta) if view is None else view)


def _split(n: int, deg: int, what: str) -> int:
    assert n % deg == 0, f"{what}: {n} is not divisible by tp degree {deg}"
    return n // deg


def segments(meta: TensorMeta, view: Optional[int] = None) -> Tuple[List[Seg], List[Box]]:
    """Bands of global data held by a shard (or piece), and its pad boxes."""
    if view is None:
        view = view_axis(meta)
    R, C = global_matrix(meta, view)
    if meta.rows is not None:                      # vocab piece: a row interval
        g0, g1 = meta.rows
        return [Seg(g0, 0, 0, 0, g1 - g0, C)], []
    axis = split_axis(meta)
    if axis is None:
        return [Seg(0, 0, 0, 0, R, C)], []
    assert axis == view, f"{meta.name}: split axis {axis} in view {view}"
    deg, idx = meta.tp_deg(), meta.tp_index()
    assert 0 <= idx < deg, f"{meta.name}: tp_index {idx} outside degree {deg}"
    if meta.kind == VOCAB_PAD:
        n = meta.padded_rows() // deg
        lo, hi = meta.valid_rows()
        segs = [Seg(lo, 0, 0, 0, hi - lo, C)] if hi > lo else []
        pads = [Box(hi - lo, 0, n - (hi - lo), C)] if hi - lo < n else []
        return segs, pads
    if meta.kind == QKV_HEADS:
        assert axis == 0, f"{meta.name}: qkv_heads splits rows"
        n_q, n_kv, hd = meta.kind_args
        q = _split(n_q, deg, f"{meta.name} q heads") * hd
        kv = _split(n_kv, deg, f"{meta.name} kv heads") * hd
        return [Seg(idx * q, 0, 0, 0, q, C),
                Seg(n_q * hd + idx * kv, 0, q, 0, kv, C),
                Seg((n_q + n_kv) * hd + idx * kv, 0, q + kv, 0, kv, C)], []
    assert meta.kind == CHUNK
    if axis == 0:
        n = _split(R, deg, f"{meta.name} rows")
        return [Seg(idx * n, 0, 0, 0, n, C)], []
    n = _split(C, deg, f"{meta.name} cols")
    return [Seg(0, idx * n, 0, 0, R, n)], []


def infer_dst_shard(ops: List[TransferOp]) -> TensorMeta:
    """Destination shard of a tensor from its pieces (when not attached).

    Pieces of a shard at degree t, cut at the source degree T >= t, are the
    T/t consecutive indices starting at idx*T/t (Suika/migration.py:103-118).
    The reference's own TransferOp / TensorMeta objects (no ``dst_shard_meta``,
    ``kind``, ``kind_args`` or ``rows``; Suika/migration.py:29-58, 257-282)
    read as chunk layouts.
    """
    first = ops[0]
    shard = getattr(first, "dst_shard_meta", None)
    if shard is not None:
        return shard
    m = first.dst_meta
    assert getattr(m, "rows", None) is None, f"{first.param_name}: vocab pieces need dst_shard_meta"
    tp = getattr(m, "tp_meta", None)
    if tp is None or len(ops) == 1:
        return m
    dim, _, T = tp
    idxs = sorted(getattr(op.dst_meta, "tp_meta")[1] for op in ops)
    s = len(idxs)
    assert T % s == 0 and idxs == list(range(idxs[0], idxs[0] + s)) and idxs[0] % s == 0, \
        f"{first.param_name}: pieces {idxs} at degree {T} do not form one shard"
    return TensorMeta(name=m.name, dtype=m.dtype, shape=m.shape, tp_meta=(dim, idxs[0] // s, T // s),
                      kind=getattr(m, "kind", CHUNK), kind_args=getattr(m, "kind_args", ()))

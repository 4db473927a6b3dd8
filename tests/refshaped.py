"""Stand-ins for the reference's own plan objects, carrying exactly their
attributes and nothing else (no methods, no extension fields):

* ``RefTensorMeta``  -- name, dtype, shape, tp_meta (Suika/migration.py:29-58;
  ``tp_meta`` is left unset when the reference builds a meta from dtype and
  shape alone, which ``omit_tp`` reproduces for replicated tensors);
* ``RefTransferOp``  -- param_name, src_rank, dst_rank, src_meta, dst_meta
  (:257-282);
* ``RefParamLayout`` -- layout: {rank: {name: meta}} (:161-170).

``ops_from_vector`` rebuilds the TransferOps the reference's
``schedule_param_transfer`` emitted for a recorded case
(tests/golden/schedule_vectors.json.gz): a piece that is the target shard
itself is that same object (``scale_to_tp`` returns ``[self]``), a finer
piece is a new meta with the recorded tp meta (:103-118).
"""
from __future__ import annotations

from typing import Dict, List

import torch

_UNSET = object()


class RefTensorMeta:
    def __init__(self, name, dtype, shape, tp_meta=_UNSET):
        self.name = name
        self.dtype = dtype
        self.shape = torch.Size(shape)
        if tp_meta is not _UNSET:
            self.tp_meta = tp_meta


class RefTransferOp:
    def __init__(self, param_name, src_rank, dst_rank, src_meta, dst_meta):
        self.param_name = param_name
        self.src_rank = src_rank
        self.dst_rank = dst_rank
        self.src_meta = src_meta
        self.dst_meta = dst_meta


class RefParamLayout:
    def __init__(self, layout: Dict[int, Dict[str, RefTensorMeta]]):
        self.layout = layout


def ref_layout(pl, omit_tp: bool = False) -> RefParamLayout:
    """A layout of this build's metas as reference-shaped objects (chunk
    kinds only: the reference cannot express the extensions)."""
    out = {}
    for rank, metas in pl.layout.items():
        out[rank] = {}
        for name, m in metas.items():
            assert m.kind == "chunk" and m.rows is None, f"{name}: not a reference layout"
            tp = tuple(m.tp_meta) if m.tp_meta is not None else None
            if tp is None and omit_tp:
                out[rank][name] = RefTensorMeta(name, m.dtype, tuple(m.shape))
            else:
                out[rank][name] = RefTensorMeta(name, m.dtype, tuple(m.shape), tp)
    return RefParamLayout(out)


def ops_from_vector(rows, names: List[str], spl: RefParamLayout, tpl: RefParamLayout) -> List[RefTransferOp]:
    """The reference's TransferOps of a recorded schedule: rows of
    (name id, src rank, dst rank, piece tp meta or None)."""
    ops = []
    for nid, src, dst, tp in rows:
        name = names[nid]
        tgt = tpl.layout[dst][name]
        tgt_tp = getattr(tgt, "tp_meta", None)
        tp = tuple(tp) if tp is not None else None
        piece = tgt if tp == tgt_tp else RefTensorMeta(name, tgt.dtype, tuple(tgt.shape), tp)
        ops.append(RefTransferOp(name, src, dst, spl.layout[src][name], piece))
    return ops

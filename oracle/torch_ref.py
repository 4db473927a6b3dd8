"""Torch-CPU restatement of the reference's CPU reshard -- test and CPU-baseline use only.

The reference reshards on the CPU in ``checkpoint_load`` by running
``execute_param_transfer`` in fake-source mode on CPU tensors
(Suika/migration.py:1235-1244): per op and sub-field
``chunk(n, dim)[k].contiguous()`` (or the whole shard, migration.py:299-310),
then per tensor ``torch.cat(pieces, dim=slice_dim)`` or ``clone()``
(migration.py:531-541).  This module restates that loop with torch CPU ops so
``bench.py`` can time the reference-style CPU path on the GPU box's host cores
next to the GPU kernels.  Extensions are restated with the same primitives:
vocab pieces are row ranges plus a zero pad block, fused QKV is chunked per
projection, the bf16 recast is ``Tensor.to(torch.bfloat16)``.

It consumes the oracle's op list (``reshard_oracle.schedule``) and is checked
against ``reshard_oracle.execute_fake_source`` in tests/test_oracle_torch.py.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence

import torch

from .reshard_oracle import OOp, QKV_HEADS, VOCAB_PAD, actual_shape, valid_rows


def get_send(op: OOp, src: torch.Tensor) -> torch.Tensor:
    sm, dm = op.src_meta, op.dst_meta
    if dm.kind == VOCAB_PAD:
        lo, hi = dm.rows
        slo, _ = valid_rows(sm)
        return src[lo - slo:hi - slo].contiguous()
    if sm.deg() >= dm.deg() or (sm.tp is None and dm.tp is None):
        return src                                   # whole shard, no copy (migration.py:299-300)
    if sm.tp is None:
        n, k = dm.deg(), dm.idx()
    else:
        n = dm.deg() // sm.deg()
        k = dm.idx() - sm.idx() * n
    if dm.kind == QKV_HEADS:
        nq, nkv, hd = sm.kind_args
        q = nq // sm.deg() * hd
        kv = nkv // sm.deg() * hd
        Q, K, V = src[:q], src[q:q + kv], src[q + kv:]
        return torch.cat([Q.chunk(n, 0)[k], K.chunk(n, 0)[k], V.chunk(n, 0)[k]], 0)
    axis = sm.tp[0] if sm.tp is not None else dm.tp[0]
    return src.chunk(n, dim=axis)[k].contiguous()


def execute_torch_cpu(ops: List[OOp], rank: int, fake_sources: Dict[int, Dict[str, Dict[str, torch.Tensor]]],
                      fields: Sequence[str], recast: Optional[Dict[str, str]] = None
                      ) -> Dict[str, Dict[str, torch.Tensor]]:
    pieces: Dict[str, Dict[str, List[torch.Tensor]]] = {}
    shards = {}
    piece_deg = {}
    for op in ops:
        if op.dst != rank:
            continue
        shards[op.name] = op.dst_shard
        piece_deg[op.name] = op.dst_meta.deg()
        ent = pieces.setdefault(op.name, {f: [] for f in fields})
        for f in fields:
            ent[f].append(get_send(op, fake_sources[op.src][op.name][f]))
    out: Dict[str, Dict[str, torch.Tensor]] = {}
    for name, ent in pieces.items():
        m = shards[name]
        res = {}
        for f, parts in ent.items():
            if m.kind == VOCAB_PAD:
                n = actual_shape(m)[0]
                body = torch.cat(parts, 0) if len(parts) > 1 else parts[0]
                pad = torch.zeros((n - body.shape[0],) + tuple(body.shape[1:]), dtype=body.dtype)
                res[f] = torch.cat([body, pad], 0)
            elif len(parts) > 1:
                if m.kind == QKV_HEADS:
                    nq, nkv, hd = m.kind_args
                    q = nq // piece_deg[name] * hd
                    kv = nkv // piece_deg[name] * hd
                    res[f] = torch.cat([torch.cat([p[:q] for p in parts], 0),
                                        torch.cat([p[q:q + kv] for p in parts], 0),
                                        torch.cat([p[q + kv:] for p in parts], 0)], 0)
                else:
                    res[f] = torch.cat(parts, dim=m.tp[0])
            else:
                res[f] = parts[0].clone()
        for tgt, srcf in (recast or {}).items():
            res[tgt] = res[srcf].to(torch.bfloat16)
        out[name] = res
    return out

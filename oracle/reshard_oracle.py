"""CPU oracle of Suika's reshard path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.  The product
(``suika_amd``) never imports it and has no CPU path.

It restates, in numpy and plain Python, the reference's single-process
reshard -- ``checkpoint_load`` -> ``schedule_param_transfer`` ->
``execute_param_transfer`` in fake-source mode (Suika/migration.py:1186-1305,
322-381, 397-556) -- independently of ``suika_amd``: its own metadata record,
its own schedule, ``torch.chunk`` / ``torch.cat`` semantics restated on numpy
arrays.  Tensors are raw bit patterns (bf16 -> uint16, f32 -> uint32 or
float32), so every comparison is bit-exact.

Pins (tests/test_oracle*.py, tests/test_golden.py):
  * ``chunk``/``cat``             vs torch.chunk / torch.cat (the library the
                                  reference calls), incl. uneven splits
  * ``execute_fake_source``       vs ``shard_of(G, dest)`` closed forms on
                                  seeded and index-coded global tensors, for
                                  every kind and TP/PP/DP change in the suite
  * ``schedule``                  vs the reference's own
                                  ``schedule_param_transfer`` output on 96
                                  recorded cases (greedy source choices
                                  included, data-parallel replicas too), and
                                  brute-force ownership / coverage invariants
  * ``rne_bf16``                  vs torch.Tensor.to(torch.bfloat16) on CPU,
                                  incl. ties, subnormals, inf and NaN
  * ``REFERENCE_KINDS`` /         vs the tp meta the reference's own model
    ``kind_of_name``              classes, ``parallelize_tp`` and
                                  ``get_param_tensor_meta`` produce for
                                  3404 recorded parameters (GPT / Llama /
                                  Qwen2 stages at TP 1-8), planted table
                                  mistakes shown to fail
  * index maps                    vs brute force on tiny shapes
No function here is left unpinned.
Extensions the reference lacks (vocab padding, head-granular fused QKV, bf16
recast, fp32 master, wpe) are defined by the closed forms in ``shard_of``.
"""
from __future__ import annotations

import math
import os
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

# --------------------------------------------------------------------------
# Metadata record, restating TensorMeta (Suika/migration.py:29-131)

CHUNK = "chunk"
VOCAB_PAD = "vocab_pad"
QKV_HEADS = "qkv_heads"


@dataclass
class OMeta:
    name: str
    itemsize: int                    # bytes of the param dtype (schedule volume)
    shape: Tuple[int, ...]           # global (unpadded) shape
    tp: Optional[Tuple[int, int, int]] = None    # (slice_dim, tp_index, tp_deg)
    kind: str = CHUNK
    kind_args: Tuple[int, ...] = ()
    rows: Optional[Tuple[int, int]] = None       # vocab piece row interval

    def deg(self) -> int:
        return self.tp[2] if self.tp else 1

    def idx(self) -> int:
        return self.tp[1] if self.tp else 0


def vocab_pad_rows(V: int, deg: int, multiple: int) -> int:
    return int(math.ceil(V / (multiple * deg))) * multiple * deg


def actual_shape(m: OMeta) -> Tuple[int, ...]:
    """Shard shape (migration.py:92-98; vocab_pad: padded rows / deg)."""
    s = list(m.shape)
    if m.rows is not None:
        s[0] = m.rows[1] - m.rows[0]
        return tuple(s)
    if m.tp is None:
        return tuple(s)
    if m.kind == VOCAB_PAD:
        s[0] = vocab_pad_rows(s[0], m.deg(), m.kind_args[0]) // m.deg()
    else:
        d = m.tp[0] % len(s)
        s[d] //= m.deg()
    return tuple(s)


def volume(m: OMeta) -> int:
    """numel * itemsize of the shard or piece (migration.py:62-67)."""
    return int(np.prod(actual_shape(m))) * m.itemsize


def scale_to_tp(m: OMeta, target: int) -> List[OMeta]:
    """migration.py:103-118: ascending finer pieces, or [m]."""
    if m.tp is not None and target > m.deg() and m.kind != VOCAB_PAD:
        sd, ti, deg = m.tp
        scale = target // deg
        return [OMeta(m.name, m.itemsize, m.shape, (sd, scale * ti + i, target), m.kind, m.kind_args)
                for i in range(scale)]
    return [m]


def valid_rows(m: OMeta) -> Tuple[int, int]:
    if m.rows is not None:
        return m.rows
    n = vocab_pad_rows(m.shape[0], m.deg(), m.kind_args[0]) // m.deg()
    lo = m.idx() * n
    return lo, max(lo, min(lo + n, m.shape[0]))


def tp_overlap(t1, t2) -> bool:
    """migration.py:220-244."""
    if t1 is None or t2 is None:
        return True
    sd1, i1, d1 = t1
    sd2, i2, d2 = t2
    assert sd1 == sd2, f"slice dim mismatch {sd1} vs {sd2}"
    if d1 > d2:
        i1, i2, d1, d2 = i2, i1, d2, d1
    return i2 // (d2 // d1) == i1


def tp_owned(src: OMeta, tgt: OMeta) -> bool:
    """migration.py:246-254 (vocab pieces: row containment)."""
    if tgt.kind == VOCAB_PAD:
        lo, hi = valid_rows(tgt)
        if lo == hi:
            return True      # empty piece of an all-padding shard
        slo, shi = valid_rows(src)
        return slo <= lo and hi <= shi
    ds = src.deg() if src.tp else 1
    dt = tgt.deg() if tgt.tp else 1
    return ds <= dt and tp_overlap(src.tp, tgt.tp)


def owners(layout: Dict[int, Dict[str, OMeta]], m: OMeta) -> List[int]:
    """migration.py:195-208."""
    return [r for r, metas in layout.items() if m.name in metas and tp_owned(metas[m.name], m)]


@dataclass
class OOp:
    name: str
    src: int
    dst: int
    src_meta: OMeta
    dst_meta: OMeta
    dst_shard: OMeta


def schedule(spl: Dict[int, Dict[str, OMeta]], tpl: Dict[int, Dict[str, OMeta]],
             minimum_est_peers: Optional[int] = None) -> List[OOp]:
    """Restatement of schedule_param_transfer (Suika/migration.py:322-381)."""
    max_tp = max(m.deg() for metas in spl.values() for m in metas.values())
    lat = [0.0 for _ in spl]
    if minimum_est_peers is None:
        ib = not (os.getenv("NCCL_IB_DISABLE", "False") in ["1", "true"])
        minimum_est_peers = 1 if ib else 2
    out: List[OOp] = []
    for dst, dparams in tpl.items():
        est = set()
        for name, dm in dparams.items():
            if dm.kind == VOCAB_PAD:
                lo, hi = valid_rows(dm)
                cuts = {lo, hi}
                for metas in spl.values():
                    if name in metas:
                        for b in valid_rows(metas[name]):
                            if lo < b < hi:
                                cuts.add(b)
                e = sorted(cuts)
                if lo == hi:
                    e = [lo, lo]
                pieces = [OMeta(name, dm.itemsize, dm.shape, dm.tp, dm.kind, dm.kind_args, (a, b))
                          for a, b in zip(e[:-1], e[1:])]
            else:
                pieces = scale_to_tp(dm, max_tp)
            for p in pieces:
                srcs = owners(spl, p)
                assert srcs, f"illegal transfer, {p} is not present in any source"
                if dst in srcs:
                    best = dst
                else:
                    est_srcs = [s for s in srcs if s in est]
                    pool = est_srcs if (est_srcs and len(est) >= minimum_est_peers) else srcs
                    best = min(pool, key=lambda s: lat[s] + volume(p))
                est.add(best)
                out.append(OOp(name, best, dst, spl[best][name], p, dm))
                lat[best] += volume(p)
    return out


# --------------------------------------------------------------------------
# torch.chunk / torch.cat restated on numpy

def chunk(a: np.ndarray, chunks: int, axis: int) -> List[np.ndarray]:
    """torch.chunk semantics: pieces of ceil(n / chunks) along ``axis``; the
    last may be shorter and fewer than ``chunks`` pieces may come back."""
    n = a.shape[axis]
    size = -(-n // chunks) if n else 0
    if size == 0:
        return [a]
    out = []
    for start in range(0, n, size):
        sl = [slice(None)] * a.ndim
        sl[axis] = slice(start, min(start + size, n))
        out.append(a[tuple(sl)])
    return out


def cat(parts: Sequence[np.ndarray], axis: int) -> np.ndarray:
    return np.concatenate(parts, axis=axis)


def get_send(op: OOp, src: np.ndarray) -> np.ndarray:
    """TransferOp.get_send_tensor (Suika/migration.py:290-312) for chunk
    kinds; qkv_heads chunks each projection (the build's head-granular split);
    vocab pieces are row ranges of the source shard."""
    sm, dm = op.src_meta, op.dst_meta
    assert tuple(src.shape) == actual_shape(sm), f"{op.name}: shard {src.shape} != {actual_shape(sm)}"
    if dm.kind == VOCAB_PAD:
        lo, hi = dm.rows
        slo, _ = valid_rows(sm)
        return src[lo - slo:hi - slo].copy()
    if sm.deg() >= dm.deg() or sm.tp is None and dm.tp is None:
        return src.copy()
    if sm.tp is None:
        # replicated source, TP piece: the piece's chunk of the full tensor
        n, k = dm.deg(), dm.idx()
    else:
        n = dm.deg() // sm.deg()
        k = dm.idx() - sm.idx() * n
    if dm.kind == QKV_HEADS:
        nq, nkv, hd = sm.kind_args
        q = nq // sm.deg() * hd
        kv = nkv // sm.deg() * hd
        Q, K, V = src[:q], src[q:q + kv], src[q + kv:]
        return cat([chunk(Q, n, 0)[k], chunk(K, n, 0)[k], chunk(V, n, 0)[k]], 0).copy()
    axis = sm.tp[0] if sm.tp is not None else dm.tp[0]
    return np.ascontiguousarray(chunk(src, n, axis)[k])


def _qkv_cat(pieces: List[np.ndarray], m: OMeta, piece_deg: int) -> np.ndarray:
    nq, nkv, hd = m.kind_args
    q = nq // piece_deg * hd
    kv = nkv // piece_deg * hd
    Qs = [p[:q] for p in pieces]
    Ks = [p[q:q + kv] for p in pieces]
    Vs = [p[q + kv:] for p in pieces]
    return cat([cat(Qs, 0), cat(Ks, 0), cat(Vs, 0)], 0)


def execute_fake_source(ops: List[OOp], rank: int, fake_sources: Dict[int, Dict[str, Dict[str, np.ndarray]]],
                        fields: Sequence[str], self_rank: Optional[int] = None,
                        recast: Optional[Dict[str, str]] = None) -> Dict[str, Dict[str, np.ndarray]]:
    """execute_param_transfer in fake-source mode (Suika/migration.py:426-541).

    Pieces are appended in op order and concatenated along the slice dim
    (one piece: a copy).  With ``self_rank`` set, pieces whose source is that
    rank are appended after all others, reproducing the reference's
    deferred self transfers (migration.py:454-459, 508-509) -- the ordering
    hazard the build deliberately does not follow.
    """
    pieces: Dict[str, Dict[str, List[np.ndarray]]] = {}
    deferred: List[Tuple[str, str, np.ndarray]] = []
    shards: Dict[str, OMeta] = {}
    piece_deg: Dict[str, int] = {}
    for op in ops:
        if op.dst != rank:
            continue
        shards[op.name] = op.dst_shard
        piece_deg[op.name] = op.dst_meta.deg()
        ent = pieces.setdefault(op.name, {f: [] for f in fields})
        for f in fields:
            t = get_send(op, fake_sources[op.src][op.name][f])
            if self_rank is not None and op.src == self_rank:
                deferred.append((op.name, f, t))
            else:
                ent[f].append(t)
    for name, f, t in deferred:
        pieces[name][f].append(t)
    out: Dict[str, Dict[str, np.ndarray]] = {}
    for name, ent in pieces.items():
        m = shards[name]
        res = {}
        for f, parts in ent.items():
            if m.kind == VOCAB_PAD:
                body = cat(parts, 0)
                n = actual_shape(m)[0]
                pad = np.zeros((n - body.shape[0],) + body.shape[1:], dtype=body.dtype)
                res[f] = cat([body, pad], 0)
            elif len(parts) > 1:
                if m.kind == QKV_HEADS:
                    res[f] = _qkv_cat(parts, m, piece_deg[name])
                else:
                    res[f] = cat(parts, m.tp[0])
            else:
                res[f] = parts[0].copy()
        for tgt, srcf in (recast or {}).items():
            res[tgt] = rne_bf16(res[srcf])
        out[name] = res
    return out


# --------------------------------------------------------------------------
# bf16 rounding (round half to even on the upper 16 bits; NaN -> 0x7FC0)

def rne_bf16(f32: np.ndarray) -> np.ndarray:
    """float32 (or its uint32 bits) -> bfloat16 bits (uint16).

    Pinned to torch's CPU ``.to(torch.bfloat16)`` bit for bit on every
    pattern, NaNs included, as torch converts element by element (a strided
    or 0-dim tensor); its vectorised loop over a contiguous tensor writes
    0xFFFF for a NaN instead of 0x7FC0."""
    u = np.ascontiguousarray(f32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


# --------------------------------------------------------------------------
# Closed forms: the shard of a global tensor, and global indices of a shard

def shard_of(G: np.ndarray, m: OMeta, xp=np) -> np.ndarray:
    """Local shard ``m`` of the global tensor ``G`` (any ndim), closed form.

    chunk rows : G[r n/t : (r+1) n/t]      (tensor_parallel.py:200-204)
    chunk cols : G[..., r n/t : (r+1) n/t] (tensor_parallel.py:378-381)
    qkv_heads  : cat(Q_r, K_r, V_r)         per-projection chunks, head-granular
    vocab_pad  : pad(G, Vpad)[r Vpad/t : (r+1) Vpad/t], pad rows zero
    """
    if m.tp is None:
        return G
    t, r = m.deg(), m.idx()
    if m.kind == VOCAB_PAD:
        Vp = vocab_pad_rows(G.shape[0], t, m.kind_args[0])
        n = Vp // t
        lo, hi = r * n, (r + 1) * n
        body = G[lo:min(hi, G.shape[0])]
        npad = n - body.shape[0]
        if npad == 0:
            return body
        pad = xp.zeros((npad,) + tuple(G.shape[1:]), dtype=G.dtype)
        if xp is not np:
            pad = pad.to(G.device)
        return xp.concatenate([body, pad], 0) if xp is np else xp.cat([body, pad], 0)
    if m.kind == QKV_HEADS:
        nq, nkv, hd = m.kind_args
        q, kv = nq // t * hd, nkv // t * hd
        Q = G[:nq * hd]
        K = G[nq * hd:(nq + nkv) * hd]
        V = G[(nq + nkv) * hd:]
        parts = [Q[r * q:(r + 1) * q], K[r * kv:(r + 1) * kv], V[r * kv:(r + 1) * kv]]
        return xp.concatenate(parts, 0) if xp is np else xp.cat(parts, 0)
    d = m.tp[0] % G.ndim
    n = G.shape[d] // t
    sl = [slice(None)] * G.ndim
    sl[d] = slice(r * n, (r + 1) * n)
    return G[tuple(sl)]


def shard_index(m: OMeta, xp=np, device=None):
    """Global flat index (row-major over ``m.shape``) of every element of the
    shard, -1 on vocab pad rows.  Works with numpy or torch (``xp``)."""
    shape = tuple(int(s) for s in m.shape)
    n = int(np.prod(shape)) if shape else 1
    if xp is np:
        G = np.arange(n, dtype=np.int64).reshape(shape)
    else:
        G = xp.arange(n, dtype=xp.int64, device=device).reshape(shape)
    if m.kind == VOCAB_PAD and m.tp is not None:
        t, r = m.deg(), m.idx()
        Vp = vocab_pad_rows(shape[0], t, m.kind_args[0])
        nrow = Vp // t
        lo = r * nrow
        body = G[lo:min(lo + nrow, shape[0])]
        npad = nrow - body.shape[0]
        if npad == 0:
            return body
        if xp is np:
            pad = np.full((npad,) + shape[1:], -1, dtype=np.int64)
            return np.concatenate([body, pad], 0)
        pad = xp.full((npad,) + shape[1:], -1, dtype=xp.int64, device=device)
        return xp.cat([body, pad], 0)
    return shard_of(G, m, xp)


# --------------------------------------------------------------------------
# Sharding kind of every parameter, by name suffix, as the reference assigns it
#   col  : column parallel, dim 0 chunked   (ColumnParallelLinear weight+bias,
#          tensor_parallel.py:200-204, 255-261; lm_head via the default
#          slice_dim="column", engine.py:51 / tensor_parallel.py:486-606)
#   row  : row parallel, last dim chunked   (tensor_parallel.py:378-381, 435-441)
#   repl : not sharded (norms, row-parallel bias, nn.Embedding: tensor_parallel.py:578)
# GPT: gpt_model.py:13-31; Llama: llama_model.py:16-35; Qwen2: qwen_model.py:17-40.
# Extensions of the build: vocab (padded vocab-parallel wte), qkv (fused
# head-granular QKV), wpe (learned positions, replicated).
REFERENCE_KINDS = {
    "ln_1.weight": "repl", "ln_1.bias": "repl", "ln_2.weight": "repl", "ln_2.bias": "repl",
    "attn.c_attn.linear.weight": "col", "attn.c_attn.linear.bias": "col",
    "attn.c_proj.linear.weight": "row", "attn.c_proj.linear.bias": "repl",
    "mlp.c_fc.linear.weight": "col", "mlp.c_fc.linear.bias": "col",
    "mlp.c_proj.linear.weight": "row", "mlp.c_proj.linear.bias": "repl",
    "self_attn.q_proj.weight": "col", "self_attn.k_proj.weight": "col",
    "self_attn.v_proj.weight": "col", "self_attn.q_proj.bias": "col",
    "self_attn.k_proj.bias": "col", "self_attn.v_proj.bias": "col",
    "self_attn.o_proj.weight": "row",
    "mlp.gate_proj.weight": "col", "mlp.up_proj.weight": "col", "mlp.down_proj.weight": "row",
    "input_layernorm.weight": "repl", "post_attention_layernorm.weight": "repl",
    "lm_head.weight": "col", "lm_head.bias": "col", "norm.weight": "repl", "wte.weight": "repl",
}
EXTENSION_KINDS = {
    "wte.weight": "vocab",
    "self_attn.qkv_proj.weight": "qkv", "self_attn.qkv_proj.bias": "qkv",
    "wpe.weight": "repl",
}


def kind_of_name(name: str, vocab_parallel: bool) -> str:
    """Reference kind of a parameter name (``h.<L>.`` prefix stripped)."""
    parts = name.split(".")
    suffix = ".".join(parts[2:]) if parts[0] == "h" else name
    if vocab_parallel and suffix in ("wte.weight",):
        return EXTENSION_KINDS[suffix]
    if suffix in REFERENCE_KINDS:
        return REFERENCE_KINDS[suffix]
    return EXTENSION_KINDS[suffix]

"""Shared test helpers: seeded state, oracle runs, GPU runs, plan simulation.

The oracle (oracle/reshard_oracle.py) is the checker; the product path is
``suika_amd.execute_param_transfer`` / ``ReshardPlan`` on the GPU.
"""
from __future__ import annotations

import contextlib
from typing import Dict, Iterable, List, Mapping, Optional, Tuple

import numpy as np
import torch

from oracle import reshard_oracle as O
from suika_amd.meta import ParamLayout, TensorMeta
from suika_amd.workloads import FIELD_STD, Workload

BITS = {torch.bfloat16: np.uint16, torch.float16: np.uint16, torch.float32: np.uint32,
        torch.float64: np.uint64, torch.int32: np.uint32, torch.int64: np.uint64,
        torch.uint8: np.uint8, torch.int8: np.uint8, torch.bool: np.uint8}
TORCH_BITS = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32,
              torch.float64: torch.int64, torch.int32: torch.int32, torch.int64: torch.int64,
              torch.uint8: torch.uint8}


def to_ometa(m: TensorMeta) -> O.OMeta:
    return O.OMeta(name=m.name, itemsize=m.dtype.itemsize, shape=tuple(int(s) for s in m.shape),
                   tp=None if m.tp_meta is None else tuple(m.tp_meta), kind=m.kind,
                   kind_args=tuple(m.kind_args), rows=m.rows)


def to_olayout(pl: ParamLayout) -> Dict[int, Dict[str, O.OMeta]]:
    return {r: {n: to_ometa(m) for n, m in metas.items()} for r, metas in pl.layout.items()}


def t2np(t: torch.Tensor) -> np.ndarray:
    """Bit pattern of a tensor as a numpy array (CPU copy)."""
    t = t.detach().contiguous().cpu()
    return t.view(TORCH_BITS[t.dtype]).numpy().view(BITS[t.dtype]).copy()


def np2t(a: np.ndarray, dtype: torch.dtype, device="cpu") -> torch.Tensor:
    """Tensor of ``dtype`` holding the bit pattern ``a``."""
    t = torch.from_numpy(np.ascontiguousarray(a).copy().view(_np_signed(a.dtype)))
    return t.view(dtype).to(device)


def _np_signed(dt):
    return {np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32,
            np.dtype(np.uint64): np.int64, np.dtype(np.uint8): np.uint8}[np.dtype(dt)]


def global_state(w: Workload, names: Iterable[str], seed: Optional[int] = None
                 ) -> Dict[str, Dict[str, np.ndarray]]:
    """Seeded global tensors (bit patterns): torch CPU generator, sorted names,
    fields (master|param, exp_avg, exp_avg_sq); param = bf16(master)."""
    spl, _ = w.layouts()
    any_meta = {}
    for metas in spl.layout.values():
        any_meta.update(metas)
    gen = torch.Generator("cpu").manual_seed(w.seed if seed is None else seed)
    dt = w.dtypes
    base = "master" if "master" in w.src_fields else "param"
    out: Dict[str, Dict[str, np.ndarray]] = {}
    for name in sorted(set(names)):
        shape = tuple(int(s) for s in any_meta[name].shape)
        ent: Dict[str, torch.Tensor] = {}
        for f in (base, "exp_avg", "exp_avg_sq"):
            if f not in w.src_fields:
                continue
            g = torch.randn(shape, generator=gen, dtype=torch.float32) * FIELD_STD[f]
            if f == "exp_avg_sq":
                g = g.abs()
            ent[f] = g.to(dt[f])
        if base == "master" and "param" in w.src_fields:
            ent["param"] = ent["master"].to(dt["param"])
        out[name] = {f: t2np(t) for f, t in ent.items()}
    return out


def index_state(w: Workload, names: Iterable[str], universe: Optional[Iterable[str]] = None
                ) -> Dict[str, Dict[str, np.ndarray]]:
    """Index-coded global tensors: element bits = f(name, field, flat index),
    unique within a tensor and different across tensors and fields.  A
    name's code depends on its place among ``universe`` (default: ``names``),
    so processes that each build a subset agree when they pass the same
    universe."""
    spl, _ = w.layouts()
    any_meta = {}
    for metas in spl.layout.values():
        any_meta.update(metas)
    dt = w.dtypes
    out = {}
    ids = {n: i for i, n in enumerate(sorted(set(universe if universe is not None else names)))}
    for name in sorted(set(names)):
        t_id = ids[name]
        shape = tuple(int(s) for s in any_meta[name].shape)
        n = int(np.prod(shape))
        idx = np.arange(n, dtype=np.uint64).reshape(shape)
        ent = {}
        for f_id, f in enumerate(("param", "master", "exp_avg", "exp_avg_sq")):
            if f not in w.src_fields:
                continue
            salt = np.uint64((t_id * 7919 + f_id * 104729) & 0xFFFFFFFF)
            if BITS[dt[f]] == np.uint16:
                ent[f] = ((idx * np.uint64(40503) + salt) & np.uint64(0xFFFF)).astype(np.uint16)
            else:
                # finite normal floats: exponent field 32..159
                code = (idx + salt) % np.uint64(1 << 30)
                ent[f] = (np.uint64(0x10000000) + code).astype(np.uint32)
        out[name] = ent
    return out


def source_shards(w: Workload, ranks: Iterable[int], glob: Mapping[str, Mapping[str, np.ndarray]]
                  ) -> Dict[int, Dict[str, Dict[str, np.ndarray]]]:
    """Source shards cut by the oracle's closed form."""
    spl, _ = w.layouts()
    ol = to_olayout(spl)
    out = {}
    for r in ranks:
        out[r] = {}
        for name, om in ol[r].items():
            if name not in glob:
                continue
            out[r][name] = {f: np.ascontiguousarray(O.shard_of(G, om)) for f, G in glob[name].items()}
    return out


def expected_dest(w: Workload, glob) -> Dict[str, Dict[str, np.ndarray]]:
    """Destination shards by closed form (independent of any schedule)."""
    _, tpl = w.layouts()
    ol = to_olayout(tpl)[w.dst_rank]
    out = {}
    for name, om in ol.items():
        ent = {f: np.ascontiguousarray(O.shard_of(glob[name][f], om)) for f in w.src_fields}
        for tgt, srcf in w.recast:
            ent[tgt] = O.rne_bf16(ent[srcf])
        out[name] = ent
    return out


def needed_source_ranks(w: Workload) -> List[int]:
    return sorted({op.src_rank for op in w.ops()})


def oracle_dest(w: Workload, srcs, self_rank=None):
    spl, tpl = w.layouts()
    ops = O.schedule(to_olayout(spl), to_olayout(tpl))
    return O.execute_fake_source(ops, w.dst_rank, srcs, list(w.src_fields), self_rank=self_rank,
                                 recast=w.recast_map)


def dest_names(w: Workload) -> List[str]:
    _, tpl = w.layouts()
    return list(tpl.layout[w.dst_rank])


def needed_names(w: Workload) -> List[str]:
    """Names held by the destination (all sources of those names are needed)."""
    return dest_names(w)


def to_device(srcs, w: Workload, device) -> Dict[int, Dict[str, Dict[str, torch.Tensor]]]:
    dt = w.dtypes
    return {r: {n: {f: np2t(a, dt[f], device) for f, a in e.items()} for n, e in sd.items()}
            for r, sd in srcs.items()}


POISON = 0xA5


@contextlib.contextmanager
def poisoned_allocations():
    """Fill every destination tensor and peer buffer the plan allocates with
    POISON bytes -- fresh destinations, arena views and buffers alike -- so a
    byte the kernels never write cannot pass as correct by holding a previous
    run's value."""
    from suika_amd import migration
    from suika_amd.plan import ReshardPlan
    alloc_dst, alloc_dst_ptrs = ReshardPlan.alloc_dst, ReshardPlan.alloc_dst_ptrs
    alloc_buffers, arena_views = ReshardPlan.alloc_buffers, migration._arena_views
    gather_sources = ReshardPlan.__dict__["gather_sources"]
    gatherer = ReshardPlan.__dict__["gatherer"]

    poisoned = {"tensors": 0}

    def poison(out):
        for ent in out.values():
            for t in ent.values():
                t.view(torch.uint8).fill_(POISON)
                poisoned["tensors"] += 1
        return out

    def dst(self, device, **kw):
        return poison(alloc_dst(self, device, **kw))

    def dst_ptrs(self, device):
        out, ptrs = alloc_dst_ptrs(self, device)
        return poison(out), ptrs

    def buffers(self, device):
        out = alloc_buffers(self, device)
        for b in out:
            b.fill_(POISON)
        return out

    def arena(*a, **kw):
        return poison(arena_views(*a, **kw))

    def gather(cls, ops, source, fields, device, recast=None, options=None, rank=None, stream=None, dst=None,
               ahead=None):
        # the one-call direct route, composed of its parts so that fresh
        # destinations can be poisoned between allocation and launch (arena
        # views come poisoned from _arena_views); `ahead` only moves where
        # the fresh tensors are allocated
        plan, src_ptrs = cls.from_sources(ops, source, fields, device, recast=recast, options=options, rank=rank)
        if dst is None:
            part, ptrs = plan.alloc_dst_ptrs(device)
            poison(part)
        else:
            part, ptrs = dst, plan.bind_dst_ptrs(dst, device)
        plan.gather_ptrs(src_ptrs, ptrs, stream)
        return plan, part

    def make_gatherer(cls, source, fields, device, recast=None, options=None, rank=None, stream=None,
                      encoding=None):
        return lambda ops, dst=None, ahead=None: gather(cls, ops, source, fields, device, recast, options, rank,
                                                        stream, dst, ahead)

    ReshardPlan.alloc_dst, ReshardPlan.alloc_dst_ptrs = dst, dst_ptrs
    ReshardPlan.alloc_buffers, migration._arena_views = buffers, arena
    ReshardPlan.gather_sources = classmethod(gather)
    ReshardPlan.gatherer = classmethod(make_gatherer)
    try:
        yield poisoned
    finally:
        ReshardPlan.alloc_dst, ReshardPlan.alloc_dst_ptrs = alloc_dst, alloc_dst_ptrs
        ReshardPlan.alloc_buffers, migration._arena_views = alloc_buffers, arena_views
        ReshardPlan.gather_sources = gather_sources
        ReshardPlan.gatherer = gatherer


def gpu_execute(w: Workload, srcs_np, device="cuda", plan_options=None, route="buffers", arena=False):
    """Product path: execute_param_transfer on the GPU with peer shards
    resident; destinations and buffers start as POISON bytes (the direct
    route's one native call is taken apart for it: the fused call itself is
    checked by dirty_cache_execute)."""
    from suika_amd import execute_param_transfer
    ops = w.ops()
    fake = to_device(srcs_np, w, device)
    expected_sub_fields = [(f, "normal") for f in w.src_fields]
    with poisoned_allocations() as poisoned:
        out = execute_param_transfer(ops, {}, torch.device(device), expected_sub_fields,
                                     rank=w.dst_rank, fake_source_state_dicts=fake,
                                     recast=w.recast_map, plan_options=plan_options, route=route,
                                     arena=arena)
    torch.cuda.synchronize()
    n_out = sum(len(e) for e in out.values())
    assert poisoned["tensors"] >= n_out, "destinations were not poisoned before the kernels ran"
    return {n: {f: t2np(t) for f, t in e.items()} for n, e in out.items()}


def simulate_plan(plan, srcs_np, esize_of) -> Dict[Tuple[str, str], np.ndarray]:
    """Execute a ReshardPlan's pieces with numpy (bytes), pack then unpack.

    Checks the host lowering and the library's buffer layout without a GPU."""
    return simulate_unpack(plan, simulate_pack(plan, srcs_np, esize_of), esize_of)


def simulate_pack(plan, srcs_np, esize_of) -> List[np.ndarray]:
    """The peer buffers of a ReshardPlan, packed with numpy from the source
    bit patterns ``srcs_np[rank][name][field]``; gaps between payloads are 0."""
    from suika_amd import _lib
    src_mats = []
    for (r, name, f) in plan.src_keys:
        a = np.ascontiguousarray(srcs_np[r][name][f])
        src_mats.append(a)
    bufs = [np.zeros(max(1, n), dtype=np.uint8) for n in plan.peer_bytes]
    c_src = plan.c_src
    for k, pc in enumerate(plan.pieces):
        if pc.kind == _lib.SR_PIECE_ZERO:
            continue
        st = c_src[pc.src]
        es = esize_of(st.dtype)
        sm = src_mats[pc.src].reshape(-1).view(np.uint8).reshape(st.rows, st.cols * es)
        payload = sm[pc.src_row:pc.src_row + pc.rows, pc.src_col * es:(pc.src_col + pc.cols) * es]
        off = plan.piece_offset(k)
        n = payload.size
        bufs[pc.peer][off:off + n] = payload.reshape(-1)
    return bufs


def payload_spans(plan, esize_of) -> List[Tuple[int, int, int]]:
    """(peer, offset, bytes) of every non-ZERO piece's payload."""
    from suika_amd import _lib
    out = []
    c_src = plan.c_src
    for k, pc in enumerate(plan.pieces):
        if pc.kind == _lib.SR_PIECE_ZERO:
            continue
        out.append((pc.peer, plan.piece_offset(k), pc.rows * pc.cols * esize_of(c_src[pc.src].dtype)))
    return out


def simulate_unpack(plan, bufs, esize_of) -> Dict[Tuple[str, str], np.ndarray]:
    """The destinations a ReshardPlan's unpack writes from peer buffers
    ``bufs`` (numpy bytes), computed with numpy."""
    from suika_amd import _lib
    dst = {}
    for key in plan.dst_keys:
        spec = plan.dst_specs[key]
        dst[key] = np.full(int(np.prod(spec.shape)) * spec.dtype.itemsize, 0xAB, dtype=np.uint8)
    c_src = plan.c_src
    c_dst = plan.c_dst
    for k, pc in enumerate(plan.pieces):
        if pc.kind == _lib.SR_PIECE_ZERO:
            dt_ = c_dst[pc.dst]
            es = esize_of(dt_.dtype)
            dm = dst[plan.dst_keys[pc.dst]].reshape(dt_.rows, dt_.cols * es)
            dm[pc.dst_row:pc.dst_row + pc.rows, pc.dst_col * es:(pc.dst_col + pc.cols) * es] = 0
            continue
        st = c_src[pc.src]
        es = esize_of(st.dtype)
        off = plan.piece_offset(k)
        payload = bufs[pc.peer][off:off + pc.rows * pc.cols * es].reshape(pc.rows, pc.cols * es)
        if pc.dst >= 0:
            dt_ = c_dst[pc.dst]
            dm = dst[plan.dst_keys[pc.dst]].reshape(dt_.rows, dt_.cols * es)
            dm[pc.dst_row:pc.dst_row + pc.rows, pc.dst_col * es:(pc.dst_col + pc.cols) * es] = payload
        if pc.kind == _lib.SR_PIECE_RECAST:
            dt2 = c_dst[pc.dst2]
            h = O.rne_bf16(np.ascontiguousarray(payload).view(np.uint32)).view(np.uint8)
            dm2 = dst[plan.dst_keys[pc.dst2]].reshape(dt2.rows, dt2.cols * 2)
            dm2[pc.dst_row:pc.dst_row + pc.rows, pc.dst_col * 2:(pc.dst_col + pc.cols) * 2] = \
                h.reshape(pc.rows, pc.cols * 2)
    out = {}
    for key, raw in dst.items():
        spec = plan.dst_specs[key]
        out[key] = raw.view(BITS[spec.dtype]).reshape(spec.shape)
    return out


GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def load_reshard_vectors():
    """{payload: {case: (sources, expected destination)}} from the fixture."""
    import json as _json
    z = np.load(GOLDEN / "reshard_vectors.npz")
    blob = z["blob"]
    manifest = _json.loads(bytes(z["manifest"]).decode())
    out: Dict[str, Dict[str, tuple]] = {}
    for key, (off, dtstr, shape) in manifest.items():
        dt = np.dtype(dtstr)
        n = int(np.prod(shape)) if shape else 1
        a = blob[off:off + n * dt.itemsize].view(dt).reshape(shape)
        parts = key.split("|")
        payload, case, side = parts[0], parts[1], parts[2]
        srcs, dst = out.setdefault(payload, {}).setdefault(case, ({}, {}))
        if side == "src":
            r, name, f = int(parts[3]), parts[4], parts[5]
            srcs.setdefault(r, {}).setdefault(name, {})[f] = a
        else:
            name, f = parts[3], parts[4]
            dst.setdefault(name, {})[f] = a
    return out


def load_schedule_vectors():
    import gzip
    import json as _json
    with gzip.open(GOLDEN / "schedule_vectors.json.gz", "rt") as fh:
        return _json.load(fh)


def round_robin_groups(k: int):
    """A launch grouping for tests: the tensors dealt round robin into ``k``
    groups (whole tensors, not contiguous in schedule order), as a stand-in
    for ``migration._pipeline_groups`` that forces several launch groups on
    small cases."""
    def groups(ops, elem_bytes, pipeline, tensors_per_name=1, runs=None):
        index: Dict[str, int] = {}
        out: List[list] = [[] for _ in range(k)]
        for op in ops:
            g = index.setdefault(op.param_name, len(index) % k)
            out[g].append(op)
        return [g for g in out if g]
    return groups


def dirty_allocator_cache(device="cuda", total=256 << 20):
    """Leave torch's caching allocator holding freed blocks full of POISON
    bytes (large ones, and small ones for tensors under 1 MiB), so that
    destinations it hands out next hold POISON rather than zeros unless the
    kernels write them.  A best effort: the allocator decides which blocks
    it reuses."""
    torch.cuda.empty_cache()
    held = [torch.full((total,), POISON, dtype=torch.uint8, device=device)]
    held += [torch.full((s,), POISON, dtype=torch.uint8, device=device) for s in (512 << 10,) * 16]
    held += [torch.full((s,), POISON, dtype=torch.uint8, device=device) for s in (4096,) * 64]
    torch.cuda.synchronize()
    del held


def dirty_cache_execute(w: Workload, srcs_np, device="cuda", plan_options=None, ops=None):
    """The drop-in call's default path (route "direct", fresh destinations:
    one native call per launch group) on the GPU, after dirtying the
    allocator cache.  ``ops``: the schedule to pass (default: this rank's
    ops as a plain list)."""
    from suika_amd import execute_param_transfer
    fake = to_device(srcs_np, w, device)
    dirty_allocator_cache(device)
    out = execute_param_transfer(w.ops() if ops is None else ops, {}, torch.device(device),
                                 [(f, "normal") for f in w.src_fields],
                                 rank=w.dst_rank, fake_source_state_dicts=fake, recast=w.recast_map,
                                 plan_options=plan_options)
    torch.cuda.synchronize()
    return {n: {f: t2np(t) for f, t in e.items()} for n, e in out.items()}

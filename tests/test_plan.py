"""Host side of the product path, checked on the CPU:

* ``schedule_param_transfer`` (suika_amd.meta) chooses the same source and
  piece for every op as the oracle's restatement of the reference schedule;
* executing a ``ReshardPlan``'s pieces with numpy (pack into the library's
  buffer layout, then unpack) reproduces the oracle bit for bit -- this pins
  the lowering (the library's ``sr_lower``), the buffer offsets and the
  coverage check;
* the benchmark plans have the documented sizes (P, D, pieces).
"""
from collections import OrderedDict

import numpy as np
import pytest
import torch

from oracle import reshard_oracle as O
from suika_amd import ParamLayout, TensorMeta, schedule_param_transfer
from suika_amd.plan import ReshardPlan, SlotSpec
from suika_amd.workloads import CONFIG_ORDER, CONFIGS, fields_of
from tests import cases
from tests.harness import (expected_dest, global_state, index_state, oracle_dest, simulate_plan,
                           source_shards, to_olayout)

SMALL = cases.all_small_cases()


def _names(w):
    spl, _ = w.layouts()
    out = set()
    for metas in spl.layout.values():
        out |= set(metas)
    return out


def _sig(m):
    return (tuple(m.tp) if m.tp else None, m.rows)


@pytest.mark.parametrize("w", SMALL + [CONFIGS[k] for k in CONFIG_ORDER],
                         ids=[w.key for w in SMALL] + CONFIG_ORDER)
@pytest.mark.parametrize("min_peers", [1, 2])
def test_schedule_matches_oracle(w, min_peers):
    spl, tpl = w.layouts()
    ours = schedule_param_transfer(spl, tpl, minimum_est_peers=min_peers)
    ref = O.schedule(to_olayout(spl), to_olayout(tpl), minimum_est_peers=min_peers)
    assert len(ours) == len(ref)
    for a, b in zip(ours, ref):
        assert (a.param_name, a.src_rank, a.dst_rank) == (b.name, b.src, b.dst)
        assert (tuple(a.dst_meta.tp_meta) if a.dst_meta.tp_meta else None, a.dst_meta.rows) == _sig(b.dst_meta)


def test_schedule_respects_nccl_ib_disable(monkeypatch):
    w = cases.scaled_configs()["gpt6.7b_tp1pp4_tp8"]
    spl, tpl = w.layouts()
    monkeypatch.setenv("NCCL_IB_DISABLE", "1")
    a = schedule_param_transfer(spl, tpl)
    b = schedule_param_transfer(spl, tpl, minimum_est_peers=2)
    assert [(o.param_name, o.src_rank) for o in a] == [(o.param_name, o.src_rank) for o in b]


def test_schedule_rejects_missing_source():
    spl = ParamLayout.from_metas({0: {"a": TensorMeta(name="a", dtype=torch.float32, shape=(4, 4),
                                                      tp_meta=(0, 0, 2))}})
    tpl = ParamLayout.from_metas({0: {"a": TensorMeta(name="a", dtype=torch.float32, shape=(4, 4),
                                                      tp_meta=(0, 0, 1))}})
    with pytest.raises(AssertionError, match="not present in any source"):
        schedule_param_transfer(spl, tpl)


def _plan_for(w, srcs_np=None):
    ops = w.ops()
    dt = w.dtypes
    specs = {(op.src_rank, op.param_name, f): SlotSpec(tuple(op.src_meta.actual_shape()), dt[f])
             for op in ops for f in w.src_fields}
    return ReshardPlan(ops, specs, fields_of(w), recast=w.recast_map)


def _esize(dt_code):
    from suika_amd import _lib
    return {_lib.SR_DT_U8: 1, _lib.SR_DT_BF16: 2, _lib.SR_DT_F16: 2, _lib.SR_DT_F32: 4,
            _lib.SR_DT_F64: 8, _lib.SR_DT_I32: 4, _lib.SR_DT_I64: 8}[dt_code]


@pytest.mark.parametrize("w", SMALL, ids=[w.key for w in SMALL])
@pytest.mark.parametrize("payload", ["seeded", "index"])
def test_plan_simulation_matches_oracle(w, payload):
    glob = (global_state if payload == "seeded" else index_state)(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    plan = _plan_for(w)
    got = simulate_plan(plan, srcs, _esize)
    want = oracle_dest(w, srcs)
    closed = expected_dest(w, glob)
    assert {k[0] for k in got} == set(want)
    for (name, f), arr in got.items():
        np.testing.assert_array_equal(arr, want[name][f], err_msg=f"{name}/{f}")
        np.testing.assert_array_equal(arr, closed[name][f], err_msg=f"{name}/{f}")
    plan.close()


# P (bytes read by pack), D (bytes written by unpack), pieces per field.
DOCUMENTED = {
    "gpt125m_tp2_tp4": (0.835e9, 0.835e9, 147),
    "llama7b_tp4pp2_tp2pp2": (23.585e9, 23.585e9, 258),
    "llama13b_tp8_tp4pp2": (22.780e9, 22.780e9, 323),
    "gpt6.7b_tp1pp4_tp8": (12.132e9, 12.132e9, 388),
    "qwen7b_tp2_tp4": (22.849e9, 26.657e9, 339),
}


@pytest.mark.parametrize("key", CONFIG_ORDER)
def test_benchmark_plan_sizes(key):
    w = CONFIGS[key]
    plan = _plan_for(w)
    info = plan.info
    P, D, pieces = DOCUMENTED[key]
    assert abs(info.pack_bytes_read - P) < 0.0005e9
    assert info.pack_bytes_written == info.pack_bytes_read == info.unpack_bytes_read
    assert abs(info.unpack_bytes_written - D) < 0.0005e9
    copies = [p for p in plan.pieces if p.kind != 2]
    assert len(copies) == pieces * len(w.src_fields)
    # every buffer offset is 256-byte aligned
    for k in range(0, plan.n_pieces, 37):
        off = plan.piece_offset(k)
        assert off == np.iinfo(np.uint64).max or off % 256 == 0
    plan.close()


def test_benchmark_shortest_row_runs():
    """Every strided run (a region narrower than its tensor, on the source,
    destination or bf16 side) is a 16-B multiple of at least 768 bytes at the
    benchmark shapes (GPT-125M attn c_proj: 192 f32 columns), so the 16-byte
    vector path covers all of them and no LDS staging is needed."""
    shortest = {}
    for key in CONFIG_ORDER:
        w = CONFIGS[key]
        plan = _plan_for(w)
        for p in plan.pieces:
            sides = [(plan.c_dst[d], _esize(plan.c_dst[d].dtype)) for d in (p.dst, p.dst2) if d >= 0]
            if p.src >= 0:
                sides.append((plan.c_src[p.src], _esize(plan.c_src[p.src].dtype)))
            for t, es in sides:
                if p.rows > 1 and p.cols != t.cols:
                    run = p.cols * es
                    assert run % 16 == 0, (key, p.rows, p.cols)
                    shortest[key] = min(shortest.get(key, run), run)
        plan.close()
    assert min(shortest.values()) == 768 and shortest["gpt125m_tp2_tp4"] == 768, shortest


def test_lowering_rejects_uncovered_piece():
    """A source that does not hold its piece: the lowering names the tensor
    and the missing elements instead of planning a wrong copy."""
    from suika_amd import TransferOp
    src = TensorMeta(name="a", dtype=torch.float32, shape=(8, 4), tp_meta=(0, 1, 2))
    dst = TensorMeta(name="a", dtype=torch.float32, shape=(8, 4), tp_meta=(0, 0, 2))
    specs = {(1, "a", "param"): SlotSpec((4, 4), torch.float32)}
    with pytest.raises(AssertionError, match="a: source rank 1 holds 0 of the 16 elements"):
        ReshardPlan([TransferOp("a", 1, 0, src, dst)], specs, ["param"])


def test_lowering_rejects_wrong_source_shape():
    """get_send_tensor's shape check (migration.py:293-294), by name."""
    from suika_amd import TransferOp
    src = TensorMeta(name="w", dtype=torch.float32, shape=(8, 4), tp_meta=(0, 0, 2))
    dst = TensorMeta(name="w", dtype=torch.float32, shape=(8, 4), tp_meta=(0, 0, 2))
    specs = {(0, "w", "param"): SlotSpec((4, 5), torch.float32)}
    with pytest.raises(AssertionError, match=r"param w - src_tensor shape \(4, 5\) mismatch with src_meta \(4, 4\)"):
        ReshardPlan([TransferOp("w", 0, 0, src, dst)], specs, ["param"])


def test_arena_layout_and_views():
    """Destination arena: field by field, plan order within a field, every
    tensor 256-byte aligned and disjoint; alloc_dst(arena=True) returns views
    of one storage with the planned shapes and dtypes."""
    w = CONFIGS["llama7b_tp4pp2_tp2pp2"]
    plan = _plan_for(w)
    total, offs = plan.arena_layout()
    spans = []
    for key in plan.dst_keys:
        spec = plan.dst_specs[key]
        n = int(np.prod(spec.shape)) * spec.dtype.itemsize
        assert offs[key] % 256 == 0
        spans.append((offs[key], offs[key] + n, key))
    spans.sort()
    for (a0, a1, ka), (b0, b1, kb) in zip(spans, spans[1:]):
        assert a1 <= b0, (ka, kb)
    assert spans[-1][1] == total
    fields = [k[1] for _, _, k in spans]
    assert fields == sorted(fields, key=list(dict.fromkeys(k[1] for k in plan.dst_keys)).index)
    plan.close()

    small = cases.scaled_configs()["qwen7b_tp2_tp4"]          # includes a recast bf16 field
    plan = _plan_for(small)
    dst = plan.alloc_dst("cpu", arena=True)
    base = None
    total, offs = plan.arena_layout()
    for (name, f), spec in plan.dst_specs.items():
        t = dst[name][f]
        assert tuple(t.shape) == tuple(spec.shape) and t.dtype == spec.dtype and t.is_contiguous()
        ptr = t.untyped_storage().data_ptr()
        base = ptr if base is None else base
        assert ptr == base, "all destinations share one storage"
        assert t.data_ptr() - base == offs[(name, f)]
    plan.close()


def _arena_restated(ops, dtypes, fields, recast):
    """execute_param_transfer's arena layout placed tensor by tensor: recast
    targets first, then the moved fields; names in schedule order within a
    field; each start rounded up to 256 bytes."""
    from suika_amd.geometry import infer_dst_shard
    names = list(dict.fromkeys(op.param_name for op in ops))
    order = [t for t, sf in recast.items() if sf in fields] + [f for f in fields if f not in recast]
    end, want = 0, {}
    for f in order:
        for name in names:
            shape = tuple(infer_dst_shard([op for op in ops if op.param_name == name]).actual_shape())
            dtype = torch.bfloat16 if f in recast else dtypes[f]
            end = -(-end // 256) * 256
            want[(name, f)] = (end, shape, dtype)
            end += int(np.prod(shape, dtype=np.int64)) * dtype.itemsize
    return want, end


@pytest.mark.parametrize("case", list(cases.scaled_configs()) + ["empty"])
def test_execute_arena_views_layout(case):
    """The drop-in call's destination arena (built before any plan, then
    filled by the launch groups) against the placement restated tensor by
    tensor; a recast target whose source field is not moved gets no slot."""
    from suika_amd import migration
    if case == "empty":
        ops, fields, recast, dtypes = _empty_case(2, 1), ["param"], {}, {"param": torch.float32}
    else:
        w = cases.scaled_configs()[case]
        ops, fields, dtypes = w.ops(), list(w.src_fields), w.dtypes
        recast = dict(w.recast_map, extra_bf16="not_moved")
    src = {}
    for op in ops:
        src.setdefault(op.src_rank, {})[op.param_name] = {f: torch.empty(0, dtype=dtypes[f]) for f in fields}
    views = migration._arena_views(ops, src.__getitem__, fields, recast, torch.device("cpu"))
    want, end = _arena_restated(ops, dtypes, fields, recast)
    got_keys = {(n, f) for n, e in views.items() for f in e}
    assert got_keys == set(want)
    base = next(iter(next(iter(views.values())).values())).untyped_storage()
    assert base.nbytes() == max(1, end)
    for (name, f), (off, shape, dtype) in want.items():
        t = views[name][f]
        assert t.untyped_storage().data_ptr() == base.data_ptr(), (name, f)
        # (data_ptr() of a zero-element tensor is 0; its storage offset still counts)
        assert t.storage_offset() * t.element_size() == off, (name, f)
        assert tuple(t.shape) == shape and t.dtype == dtype and t.is_contiguous(), (name, f)


def test_execute_arena_errors():
    """The arena builder's checks: pieces that do not form one destination
    shard, and a source entry without a moved field."""
    from suika_amd import TransferOp, migration
    src = TensorMeta(name="w", dtype=torch.float32, shape=(8, 4), tp_meta=(0, 0, 4))
    pieces = [TransferOp("w", 0, 0, src, TensorMeta(name="w", dtype=torch.float32, shape=(8, 4),
                                                    tp_meta=(0, i, 4))) for i in (0, 2)]
    sd = {0: {"w": {"param": torch.empty(0)}}}
    with pytest.raises(AssertionError, match=r"w: pieces \[0, 2\] at degree 4 do not form one shard"):
        migration._arena_views(pieces, sd.__getitem__, ["param"], {}, torch.device("cpu"))
    ok = pieces[:1]
    with pytest.raises(AssertionError, match="w has no tensor exp_avg"):
        migration._arena_views(ok, sd.__getitem__, ["param", "exp_avg"], {}, torch.device("cpu"))
    with pytest.raises(AssertionError, match="param missing in source w"):
        migration._arena_views(ok, {0: {}}.__getitem__, ["param"], {}, torch.device("cpu"))


def _empty_case(tp_src, tp_dst):
    def metas(tp):
        return ParamLayout.from_metas({r: {
            "w": TensorMeta(name="w", dtype=torch.float32, shape=(8, 4), tp_meta=(0, r, tp)),
            "none": TensorMeta(name="none", dtype=torch.float32, shape=(0,)),
            "none2d": TensorMeta(name="none2d", dtype=torch.float32, shape=(0, 4), tp_meta=(-1, r, tp)),
        } for r in range(tp)})
    return schedule_param_transfer(metas(tp_src), metas(tp_dst))


def test_zero_element_tensors_are_planned_as_empty():
    """A parameter with no elements moves nothing; its destination is an
    empty tensor of the right shape and dtype per field (the reference's
    clone() of an empty piece), on both allocation paths."""
    ops = [o for o in _empty_case(2, 1) if o.dst_rank == 0]
    specs = {(o.src_rank, o.param_name, f): SlotSpec(tuple(o.src_meta.actual_shape()), torch.float32)
             for o in ops for f in ("master", "exp_avg")}
    plan = ReshardPlan(ops, specs, ["master", "exp_avg"], recast={"param": "master"})
    assert {k[0] for k in plan.dst_keys} == {"w"}
    for arena in (False, True):
        dst = plan.alloc_dst("cpu", arena=arena)
        assert tuple(dst["none"]["master"].shape) == (0,) and dst["none"]["param"].dtype == torch.bfloat16
        assert tuple(dst["none2d"]["exp_avg"].shape) == (0, 4)
        assert tuple(dst["w"]["master"].shape) == (8, 4)
    plan.close()


def _group_costs(w, groups, elem, tpn):
    """(plan ns, GPU ns) of each launch group under the migration module's
    cost model."""
    from suika_amd import migration as M
    out = []
    for g in groups:
        names = {op.param_name for op in g}
        numel = sum(op.dst_meta.numel() for op in g)
        out.append((M.PLAN_NS_PER_GROUP + M.PLAN_NS_PER_TENSOR * tpn * len(names),
                    numel * 2.0 * elem / M.GATHER_BYTES_PER_NS))
    return out


def test_pipeline_groups_keep_tensors_whole():
    """Launch groups of execute_param_transfer: every op in exactly one
    group, every op of a tensor in the same group, at most ``pipeline``
    groups, within a group the tensors largest first (the order their
    destinations are allocated in) and each tensor's ops in schedule order,
    the largest tensor in the first group."""
    from suika_amd import migration
    for key in CONFIG_ORDER:
        w = CONFIGS[key]
        ops = w.ops()
        elem = sum(w.dtypes[f].itemsize for f in w.src_fields)
        tpn = len(w.src_fields) + len(w.recast_map)
        position = {id(op): i for i, op in enumerate(ops)}
        for pipeline in (1, 2, 3, 4, 8, 100):
            groups = migration._pipeline_groups(ops, elem, pipeline, tpn).cut()
            assert sorted(position[id(op)] for g in groups for op in g) == list(range(len(ops)))
            assert 1 <= len(groups) <= pipeline
            per_name = {}
            for op in ops:
                per_name[op.param_name] = per_name.get(op.param_name, 0) + op.dst_meta.numel()
            seen = set()
            for g in groups:
                names = list(dict.fromkeys(op.param_name for op in g))
                assert not set(names) & seen, "a tensor split across groups"
                seen |= set(names)
                if len(groups) > 1:
                    sizes = [per_name[n] for n in names]
                    assert sizes == sorted(sizes, reverse=True), "tensors not largest first"
                for n in names:
                    run = [position[id(op)] for op in g if op.param_name == n]
                    assert run == sorted(run)
                    at = [i for i, op in enumerate(g) if op.param_name == n]
                    assert at == list(range(at[0], at[0] + len(at))), "a tensor's ops not together"
            if pipeline == 1:
                assert groups == [ops]
            if len(groups) > 1:
                assert max(per_name, key=per_name.get) in {op.param_name for op in groups[0]}
    # a tensor whose ops are not consecutive still lands whole in one group
    w = CONFIGS["llama7b_tp4pp2_tp2pp2"]
    ops = list(w.ops())
    ops = ops[1:] + ops[:1]                  # the first tensor's first op moves to the end
    groups = migration._pipeline_groups(ops, 14, 8, 5).cut()
    owner = {}
    for gi, g in enumerate(groups):
        for op in g:
            assert owner.setdefault(op.param_name, gi) == gi
    assert sorted(map(id, (op for g in groups for op in g))) == sorted(map(id, ops))


def test_pipeline_groups_follow_the_cost_model():
    """The cut: the first group carries FIRST_GROUP_NS of GPU work (the
    fewest largest tensors that do); each later group but the last is
    planned within PLAN_SHARE of its predecessor's GPU time and holds at
    least MIN_GROUP_TENSORS names; tensors go largest first, so no tensor of
    a later group is larger than one of an earlier group."""
    from suika_amd import migration as M
    for key in CONFIG_ORDER:
        w = CONFIGS[key]
        ops = w.ops()
        elem = sum(w.dtypes[f].itemsize for f in w.src_fields)
        tpn = len(w.src_fields) + len(w.recast_map)
        groups = M._pipeline_groups(ops, elem, 8, tpn).cut()
        costs = _group_costs(w, groups, elem, tpn)
        sizes = []
        for g in groups:
            per = {}
            for op in g:
                per[op.param_name] = per.get(op.param_name, 0) + op.dst_meta.numel()
            sizes.append(sorted(per.values()))
        for a, b in zip(sizes[:-1], sizes[1:]):
            assert a[0] >= b[-1], (key, "a later group holds a larger tensor")
        first_gpu = costs[0][1]
        assert first_gpu >= M.FIRST_GROUP_NS or len(groups) == 1
        assert first_gpu - sizes[0][0] * 2.0 * elem / M.GATHER_BYTES_PER_NS < M.FIRST_GROUP_NS
        for j in range(1, len(groups) - 1):
            names = len(sizes[j])
            assert names >= M.MIN_GROUP_TENSORS
            assert costs[j][0] <= costs[j - 1][1] * M.PLAN_SHARE + 1e-6, (key, j)
            assert costs[j][1] >= M.PLAN_NS_PER_GROUP, (key, j)
    # the benchmark shares pipeline in 3 or 4 groups; a single tensor or
    # pipeline=1 runs as one
    shapes = {key: len(M._pipeline_groups(CONFIGS[key].ops(), 14, 8, 5).cut()) for key in CONFIG_ORDER}
    assert all(2 <= k <= 8 for k in shapes.values()), shapes
    w = CONFIGS["gpt125m_tp2_tp4"]
    one = [op for op in w.ops() if op.param_name == w.ops()[0].param_name]
    assert M._pipeline_groups(one, 12, 8, 3).cut() == [one] == list(M._pipeline_groups(one, 12, 8, 3))
    assert M._pipeline_groups([], 12, 8, 3).cut() == [[]]


def test_launch_groups_adapt_to_the_measured_planning_rate(monkeypatch):
    """Iterated, the launch groups are sized by the planning rate measured on
    the groups so far: on a host four times slower than the prior, later
    groups get smaller, and every group after a timed one is planned within
    PLAN_SHARE of its predecessor's GPU time at that rate."""
    from suika_amd import migration as M
    clock = [0]
    monkeypatch.setattr(M, "_clock_ns", lambda: clock[0])
    w = CONFIGS["gpt6.7b_tp1pp4_tp8"]
    ops = w.ops()
    elem = sum(w.dtypes[f].itemsize for f in w.src_fields)
    tpn = len(w.src_fields) + len(w.recast_map)
    runs = {}
    for rate in (M.PLAN_NS_PER_TENSOR, 4 * M.PLAN_NS_PER_TENSOR):
        groups = []
        for g in M._pipeline_groups(ops, elem, 8, tpn):
            groups.append(g)
            names = len({op.param_name for op in g})
            clock[0] += M.PLAN_NS_PER_GROUP + rate * tpn * names     # the simulated planning time
        assert sorted(map(id, (op for g in groups for op in g))) == sorted(map(id, ops))
        costs = _group_costs(w, groups, elem, tpn)
        sizes = [len({op.param_name for op in g}) for g in groups]
        for j in range(2, len(groups) - 1):
            plan = M.PLAN_NS_PER_GROUP + rate * tpn * sizes[j]
            assert plan <= costs[j - 1][1] * M.PLAN_SHARE + 1e-6, (rate, j)
        runs[rate] = sizes
    fast, slow = runs[M.PLAN_NS_PER_TENSOR], runs[4 * M.PLAN_NS_PER_TENSOR]
    assert fast[:2] == slow[:2]                  # sized before any group was timed
    assert slow[2] < fast[2], (fast, slow)


@pytest.mark.parametrize("share", [0.0, 1e-5, 1.0])
def test_launch_groups_survive_a_group_planned_within_the_overhead(monkeypatch, share):
    """A timed group of MIN_GROUP_TENSORS or more names planned in no more
    than PLAN_NS_PER_GROUP (a fast host, or a consumer that plans nothing)
    still yields every op exactly once: the measured per-tensor rate is
    floored at MIN_PLAN_NS_PER_TENSOR instead of reaching zero, and the next
    group then takes all that is left."""
    from suika_amd import migration as M
    spent_ns = int(share * M.PLAN_NS_PER_GROUP)   # none, 0.6 ns, exactly the overhead
    clock = [0]
    monkeypatch.setattr(M, "_clock_ns", lambda: clock[0])
    w = CONFIGS["gpt125m_tp2_tp4"]
    ops = w.ops()
    elem = sum(w.dtypes[f].itemsize for f in w.src_fields)
    tpn = len(w.src_fields) + len(w.recast_map)
    groups = []
    for g in M._pipeline_groups(ops, elem, 8, tpn):
        groups.append(g)
        # the first group is slow; the later ones take spent_ns
        clock[0] += 10 * M.PLAN_NS_PER_GROUP if len(groups) == 1 else spent_ns
    assert sorted(map(id, (op for g in groups for op in g))) == sorted(map(id, ops))
    sizes = [len({op.param_name for op in g}) for g in groups]
    timed = [j for j in range(1, len(sizes) - 1) if sizes[j] >= M.MIN_GROUP_TENSORS]
    assert timed, sizes                           # a group was timed at spent_ns
    assert len(groups) == timed[0] + 2, sizes     # and the one after it takes the rest


def test_encoded_ops_match_the_attribute_walk():
    """The schedule keeps the tables its ops were made from (sr_op table,
    both layouts' sr_meta rows and meta objects, each op's piece); with the
    schedule's encoding, encode_ops copies an op's rows and rank_runs
    computes its piece's size from them instead of reading the metas'
    attributes.  Both give the same tables op by op, on every config and
    rank, whether or not rank_runs found the positions first.  An op the
    encoding does not describe any more -- whose source or piece meta was
    replaced, an op of another schedule, one whose shard is not the one the
    caller names, any op once the list changed -- is read from its
    attributes."""
    import copy

    from suika_amd import _lib
    from suika_amd.geometry import infer_dst_shard
    host = _lib.host()

    def decode(ops, shards, ids, enc=None):
        metas, rows = host.encode_ops(ops, shards, ids, enc)
        return [(tuple(r[[0, 1, 2, 5, 6, 7, 8]]), tuple(metas[r[3]]), tuple(metas[r[4]])) for r in rows]

    def same_runs(a, b):
        for x, y in zip(a, b):
            assert (x == y) if isinstance(x, (bool, dict, list)) else x.tolist() == y.tolist()

    for key in CONFIG_ORDER:
        w = CONFIGS[key]
        world = schedule_param_transfer(*w.layouts())
        for r in sorted({op.dst_rank for op in world}):
            ops = [op for op in world if op.dst_rank == r]
            ids = {n: i for i, n in enumerate(dict.fromkeys(op.param_name for op in ops))}
            shards = {op.param_name: op.dst_shard_meta for op in ops}
            walked = decode(ops, shards, ids)
            assert decode(ops, shards, ids, world.encoding()) == walked, (key, r)   # positions found on use
            enc = world.encoding()
            same_runs(host.rank_runs(world, r, world.positions_of(r), enc)[1:], host.rank_runs(list(world), r)[1:])
            assert decode(ops, shards, ids, enc) == walked, (key, r)   # positions rank_runs found
    w = CONFIGS["gpt125m_tp2_tp4"]
    world = schedule_param_transfer(*w.layouts())
    enc = world.encoding()
    ops = [op for op in world if op.dst_rank == w.dst_rank]
    ids = {n: i for i, n in enumerate(dict.fromkeys(op.param_name for op in ops))}
    shards = {op.param_name: op.dst_shard_meta for op in ops}
    before = decode(ops, shards, ids, enc)
    # a caller's own shard object (equal, not the op's) takes the walk
    inferred = {n: infer_dst_shard([op for op in ops if op.param_name == n]) for n in ids}
    assert decode(ops, inferred, ids, enc) == decode(ops, inferred, ids)
    # ops of another schedule of the same layouts, with this schedule's encoding
    other = [op for op in schedule_param_transfer(*w.layouts()) if op.dst_rank == w.dst_rank]
    assert decode(other, {op.param_name: op.dst_shard_meta for op in other}, ids, enc) == before
    # a source meta of another shape, and a copied piece meta, put in place
    ops[0].src_meta = TensorMeta(name=ops[0].param_name, dtype=torch.float64, shape=(3, 5))
    ops[1].dst_meta = copy.copy(ops[1].dst_meta)
    got = decode(ops, shards, ids, enc)
    assert got == decode(ops, shards, ids) and got[0][1] != before[0][1]
    same_runs(host.rank_runs(world, w.dst_rank, world.positions_of(w.dst_rank), enc)[1:],
              host.rank_runs(list(world), w.dst_rank)[1:])
    # the tables are what is read (a doctored source element size shows), and
    # only while the schedule holds them: a changed list drops them, also for
    # an encoding made before the change
    world = schedule_param_transfer(*w.layouts())
    ops = [op for op in world if op.dst_rank == w.dst_rank]
    shards = {op.param_name: op.dst_shard_meta for op in ops}
    before = decode(ops, shards, ids)
    table, src, *rest = world._tables
    world._tables = (table, src.copy(), *rest)
    world._tables[1][:, 2] += 1    # column 2: element size
    enc = world.encoding()
    doctored = decode(ops, shards, ids, enc)
    assert [m[2] for _, m, _ in doctored] == [m[2] + 1 for _, m, _ in before]
    world.append(world[0])
    assert decode(ops, shards, ids, enc) == before
    assert world.encoding() is None and world.positions_of(w.dst_rank) is None


def test_copied_and_pickled_schedules_encode_like_the_walk():
    """A schedule copied (copy.copy, copy.deepcopy) or pickled and loaded is
    a list of its own: whatever it keeps of the tables, rank_runs and
    encode_ops give what reading the ops' attributes gives, and a change to
    the copy leaves the original's tables in place."""
    import copy
    import pickle

    from suika_amd import _lib
    from suika_amd.meta import Schedule
    host = _lib.host()
    w = CONFIGS["llama7b_tp4pp2_tp2pp2"]
    world = schedule_param_transfer(*w.layouts())
    r = w.dst_rank

    def tables(s):
        enc = s.encoding() if type(s) is Schedule else None
        runs = host.rank_runs(s, r, s.positions_of(r) if type(s) is Schedule else None, enc)
        ops = runs[0]
        ids = {n: i for i, n in enumerate(dict.fromkeys(op.param_name for op in ops))}
        shards = {op.param_name: op.dst_shard_meta for op in ops}
        metas, rows = host.encode_ops(ops, shards, ids, enc)
        return ([tuple(x.tolist()) if hasattr(x, "tolist") else x for x in runs[1:5]],
                [(tuple(q[[0, 1, 2, 5, 6, 7, 8]]), tuple(metas[q[3]]), tuple(metas[q[4]])) for q in rows])

    want = tables(list(world))
    for other in (copy.copy(world), copy.deepcopy(world), pickle.loads(pickle.dumps(world))):
        assert type(other) is Schedule and list(map(type, other)) == list(map(type, world))
        assert tables(other) == want
        other.append(other[0])
        assert tables(other[:-1]) == want
    assert world.encoding() is not None and tables(world) == want


def test_schedule_positions_match_a_scan():
    """schedule_param_transfer's list keeps each destination rank's op
    positions; rank_runs given them returns what a scan of the whole
    schedule returns, falls back to the scan on positions that do not hold
    the rank's ops, and any change to the list drops the positions."""
    from suika_amd import _lib
    from suika_amd.meta import Schedule
    host = _lib.host()

    def same(a, b):
        assert a[0] == b[0]
        for x, y in zip(a[1:], b[1:]):
            assert (x == y) if isinstance(x, (bool, dict, list)) else x.tolist() == y.tolist()

    for key in CONFIG_ORDER:
        sched = schedule_param_transfer(*CONFIGS[key].layouts())
        assert type(sched) is Schedule
        for r in sorted({op.dst_rank for op in sched}) + [99]:
            pos = sched.positions_of(r)
            assert pos.tolist() == [i for i, op in enumerate(sched) if op.dst_rank == r]
            same(host.rank_runs(sched, r, pos), host.rank_runs(list(sched), r))
    r = sched[0].dst_rank
    others = np.array([i for i, op in enumerate(sched) if op.dst_rank != r][:3], dtype=np.int64)
    for bad in (others, np.array([len(sched)], dtype=np.int64), sched.positions_of(r)[::-1].copy()):
        same(host.rank_runs(sched, r, bad), host.rank_runs(list(sched), r))
    for change in (lambda s: s.append(s[0]), lambda s: s.__setitem__(0, s[1]), lambda s: s.sort(key=id),
                   lambda s: s.pop(), lambda s: s.__iadd__([s[0]]), lambda s: s.__delitem__(slice(0, 2))):
        s = schedule_param_transfer(*CONFIGS["gpt125m_tp2_tp4"].layouts())
        change(s)
        assert s.positions_of(0) is None


def test_rank_runs_and_ordered_result():
    """The one-pass prologue (a rank's ops, their tensor groups in order of
    first appearance and each tensor's elements) against a Python
    restatement, with tensors whose ops are not consecutive and a tuple
    schedule; and the result dict's order (schedule order of names, the
    given field order, absent fields skipped)."""
    from suika_amd import _lib
    host = _lib.host()
    for key in CONFIG_ORDER:
        w = CONFIGS[key]
        world = schedule_param_transfer(*w.layouts())
        for sched in (world, tuple(world[::-1]), world[5:] + world[:5]):
            for r in sorted({op.dst_rank for op in sched}):
                ops, order, starts, numel, single, index, padded, launch, total = host.rank_runs(sched, r)
                want_ops = [op for op in sched if op.dst_rank == r]
                assert ops == want_ops, (key, r)
                names = list(dict.fromkeys(op.param_name for op in want_ops))
                members = {n: [i for i, op in enumerate(want_ops) if op.param_name == n] for n in names}
                assert order.tolist() == [i for n in names for i in members[n]]
                assert starts.tolist() == [0] + list(np.cumsum([len(members[n]) for n in names]))
                assert numel.tolist() == [sum(want_ops[i].dst_meta.numel() for i in members[n]) for n in names]
                assert single == all(m == list(range(m[0], m[0] + len(m))) for m in members.values())
                assert index == {n: i for i, n in enumerate(names)}
                # tensors largest first (ties in index order) and their running total
                assert launch.tolist() == np.argsort(-numel, kind="stable").tolist()
                assert total == np.cumsum(numel[launch]).tolist()
                # a padded vocabulary shard is larger than its pieces' total
                assert padded.tolist() == [want_ops[members[n][0]].dst_shard_meta.kind == "vocab_pad"
                                           for n in names]
                for n in names:
                    shard = want_ops[members[n][0]].dst_shard_meta
                    if shard.kind != "vocab_pad":
                        assert numel[index[n]] == shard.numel(), (key, n)
    assert host.rank_runs([], 0)[0] == []
    # a launch group's ops: the picked tensors in picked order, each one's
    # ops in schedule order (tensors whose ops are not consecutive included)
    sched = CONFIGS["llama7b_tp4pp2_tp2pp2"].ops()
    sched = sched[7:] + sched[:7]
    ops, order, starts, numel, single, index = host.rank_runs(sched, sched[0].dst_rank)[:6]
    names = list(index)
    rng = np.random.default_rng(5)
    for size in (1, 5, len(names)):
        picked = rng.permutation(len(names))[:size]
        want = [op for i in picked for op in ops if op.param_name == names[i]]
        assert host.take_ops(ops, order, starts, picked) == want
    assert host.take_ops(ops, order, starts, np.array([], dtype=np.int64)) == []
    for bad in ([len(names)], [-1], [2, 2]):
        with pytest.raises(ValueError, match="take_ops"):
            host.take_ops(ops, order, starts, np.array(bad, dtype=np.int64))
    ops = CONFIGS["gpt125m_tp2_tp4"].ops()
    target = {}
    for op in reversed(ops):
        target[op.param_name] = {"exp_avg": 1, "param": 2, "master": 3}
    out = host.ordered_result(ops, target, ["master", "param", "step", "exp_avg"])
    assert list(out) == list(dict.fromkeys(op.param_name for op in ops))
    assert all(list(e) == ["master", "param", "exp_avg"] for e in out.values())
    # entries already in field order are returned as they are; others
    # (out of order, an extra field, a dict subclass) are rebuilt in order
    order = ["master", "param", "step", "exp_avg"]
    names = list(dict.fromkeys(op.param_name for op in ops))
    kinds = [{"master": 3, "param": 2, "exp_avg": 1}, {"param": 2, "exp_avg": 1},
             {"exp_avg": 1, "master": 3}, {"master": 3, "extra": 0, "param": 2},
             OrderedDict(master=3, param=2)]
    target = {n: dict(kinds[i % len(kinds)]) if i % len(kinds) < 4 else OrderedDict(kinds[4])
              for i, n in enumerate(names)}
    out = host.ordered_result(ops, target, order)
    for i, n in enumerate(names):
        src = target[n]
        assert list(out[n]) == [f for f in order if f in src], n
        assert (out[n] is src) == (i % len(kinds) in (0, 1)), n
    with pytest.raises(KeyError):
        host.ordered_result(ops, {}, ["param"])


def test_from_sources_rejects_bad_sources_by_name():
    """ReshardPlan.from_sources (the drop-in operator's planner) reads the
    source tensors themselves; what it cannot use is rejected with the
    tensor's name before anything reaches a GPU."""
    from suika_amd import TransferOp
    src = TensorMeta(name="w", dtype=torch.float32, shape=(8, 4), tp_meta=(0, 0, 2))
    dst = TensorMeta(name="w", dtype=torch.float32, shape=(8, 4), tp_meta=(0, 0, 2))
    ops = [TransferOp("w", 3, 0, src, dst)]
    dev = torch.device("cuda", 0)

    def plan(sd):
        return ReshardPlan.from_sources(ops, lambda r: sd, ["param"], dev, rank=0)

    with pytest.raises(AssertionError, match=r"source w/param of rank 3 is in host memory, not on cuda:0"):
        plan({"w": {"param": torch.zeros(4, 4)}})
    with pytest.raises(AssertionError, match=r"\[0\]: param missing in source w"):
        plan({})
    with pytest.raises(AssertionError, match="expected_sub_fields mismatch: w has no param"):
        plan({"w": {"exp_avg": torch.zeros(4, 4)}})
    with pytest.raises(AssertionError, match="source w/param of rank 3: not a tensor"):
        plan({"w": {"param": [0.0] * 16}})


def test_get_send_tensor_host_rules():
    """get_send_tensor's host side (migration.py:293-300): the reference's
    shape assertion, the whole-tensor case without any GPU, and no CPU
    fallback for a piece that needs cutting."""
    from suika_amd import TransferOp
    coarse = TensorMeta(name="w", dtype=torch.float32, shape=(8, 4), tp_meta=(0, 0, 1))
    fine = TensorMeta(name="w", dtype=torch.float32, shape=(8, 4), tp_meta=(0, 0, 2))
    t = torch.zeros(4, 4)
    assert TransferOp("w", 0, 1, fine, coarse).get_send_tensor(t) is t
    with pytest.raises(AssertionError, match=r"src_tensor shape \(4, 4\) mismatch with src_meta"):
        TransferOp("w", 0, 1, coarse, fine).get_send_tensor(t)
    with pytest.raises(AssertionError, match="runs on the GPU; src_tensor is on cpu"):
        TransferOp("w", 0, 1, coarse, fine).get_send_tensor(torch.zeros(8, 4))


def test_from_sources_reports_errors_in_op_order():
    """Source state dicts are fetched rank by rank in op order, so the first
    op decides the error, as in the reference's loop (migration.py:426-494):
    a missing own parameter is an AssertionError, a remote rank without a
    local copy the caller's own error."""
    from suika_amd import TransferOp
    m = TensorMeta(name="w", dtype=torch.float32, shape=(8, 4), tp_meta=(0, 0, 2))
    m1 = TensorMeta(name="w", dtype=torch.float32, shape=(8, 4), tp_meta=(0, 1, 2))
    dst = TensorMeta(name="w", dtype=torch.float32, shape=(8, 4), tp_meta=(0, 0, 1))

    def source(r):
        if r == 0:
            return {}
        raise NotImplementedError("remote rank")

    own_first = [TransferOp("w", 0, 0, m, m, dst), TransferOp("w", 1, 0, m1, m1, dst)]
    with pytest.raises(AssertionError, match="param missing in source w"):
        ReshardPlan.from_sources(own_first, source, ["param"], torch.device("cuda", 0), rank=0)
    with pytest.raises(NotImplementedError, match="remote rank"):
        ReshardPlan.from_sources(own_first[::-1], source, ["param"], torch.device("cuda", 0), rank=0)


def test_bind_dst_checks_every_destination():
    """Caller-provided destinations (an arena's views, or any dict) are
    bound slot by slot and rejected by name when they do not match."""
    ops = [o for o in _empty_case(2, 1) if o.dst_rank == 0]
    specs = {(o.src_rank, o.param_name, f): SlotSpec(tuple(o.src_meta.actual_shape()), torch.float32)
             for o in ops for f in ("master", "exp_avg")}
    plan = ReshardPlan(ops, specs, ["master", "exp_avg"], recast={"param": "master"})
    cpu = torch.device("cpu")
    dst = plan.alloc_dst(cpu)
    ptrs = plan.bind_dst_ptrs(dst, cpu)
    assert ptrs.tolist() == [dst[n][f].data_ptr() for n, f in plan.dst_keys]
    arena = plan.alloc_dst(cpu, arena=True)
    assert plan.bind_dst_ptrs(arena, cpu).tolist() == [arena[n][f].data_ptr() for n, f in plan.dst_keys]
    bad = {n: dict(e) for n, e in dst.items()}
    bad["w"]["param"] = torch.empty(8, 4)                 # f32 where bf16 is planned
    with pytest.raises(AssertionError, match=r"\('w', 'param'\): dtype differs"):
        plan.bind_dst_ptrs(bad, cpu)
    bad["w"]["param"] = torch.empty(4, 8, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match=r"\('w', 'param'\): shape differs"):
        plan.bind_dst_ptrs(bad, cpu)
    del bad["w"]["param"]
    with pytest.raises(AssertionError, match=r"\('w', 'param'\): no destination tensor"):
        plan.bind_dst_ptrs(bad, cpu)
    with pytest.raises(AssertionError, match="tensor is on cpu, the kernels run on cuda:0"):
        plan.bind_dst_ptrs(dst, torch.device("cuda", 0))
    plan.close()


def test_pieces_must_belong_to_their_shard():
    """A hand-built op whose piece is not a part of its destination shard
    (another tensor shape, or split along another dim) is rejected by name
    when the plan's tables are encoded."""
    from suika_amd import TransferOp
    src = TensorMeta(name="w", dtype=torch.float32, shape=(8, 4), tp_meta=(0, 0, 2))
    shard = TensorMeta(name="w", dtype=torch.float32, shape=(8, 4), tp_meta=(0, 0, 1))
    specs = {(0, "w", "param"): SlotSpec((4, 4), torch.float32)}
    other_shape = TensorMeta(name="w", dtype=torch.float32, shape=(8, 8), tp_meta=(0, 0, 2))
    with pytest.raises(AssertionError, match="w: piece .* is not part of shard"):
        ReshardPlan([TransferOp("w", 0, 0, src, other_shape, shard)], specs, ["param"])
    other_dim = TensorMeta(name="w", dtype=torch.float32, shape=(8, 4), tp_meta=(-1, 0, 2))
    with pytest.raises(AssertionError, match="w: piece .* is split along another dim than shard"):
        ReshardPlan([TransferOp("w", 0, 0, src, other_dim, shard)], specs, ["param"])


def test_utils_helpers():
    """forcefully_free_tensor releases a tensor's storage now and cuda_gc runs
    without a GPU (Suika/utils.py:248-260)."""
    from suika_amd import cuda_gc, forcefully_free_tensor
    t = torch.ones(1024)
    view = t[:8]
    forcefully_free_tensor(t)
    assert t.untyped_storage().nbytes() == 0 and view.untyped_storage().nbytes() == 0
    forcefully_free_tensor("not a tensor")   # ignored, as in the reference
    cuda_gc()


def test_reference_meta_accessors():
    """TensorMeta.numel / volumn / __eq__ and TransferOp.get_recv_tensor keep
    the reference's meaning (migration.py:62-67, 120-127, 285-287)."""
    from suika_amd import TransferOp
    shard = TensorMeta(name="w", dtype=torch.bfloat16, shape=(8, 6), tp_meta=(-1, 1, 2))
    assert shard.numel() == 24 and shard.volumn() == 48
    assert tuple(shard.actual_shape()) == (8, 3)
    # equality ignores the shard index, as the reference's does
    assert shard == TensorMeta(name="x", dtype=torch.bfloat16, shape=(8, 6), tp_meta=(-1, 0, 2))
    assert shard != TensorMeta(name="w", dtype=torch.float32, shape=(8, 6), tp_meta=(-1, 1, 2))
    recv = TransferOp("w", 0, 1, shard, shard).get_recv_tensor(torch.device("cpu"))
    assert tuple(recv.shape) == (8, 3) and recv.dtype == torch.bfloat16

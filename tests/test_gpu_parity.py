"""GPU parity: the HIP pack/unpack path against the CPU oracle, bit-exact.

Every small case (reference TEST shapes under TP/PP/DP changes, scaled
benchmark plans, padded vocab, non-16-byte rows) runs through
``execute_param_transfer`` on the GPU and must equal the oracle's reshard of
the same seeded source shards.  Kernel tunings that change the tiling or its
order (tile size, grid cap, cached access, plan order, linear order, row
groups off) are swept on a subset, so tiles that start mid-row and
grid-stride loops are covered.
"""
import numpy as np
import pytest
import torch

from suika_amd import PlanOptions
from tests import cases
from tests.harness import (global_state, gpu_execute, index_state, oracle_dest, source_shards)

pytestmark = pytest.mark.gpu

SMALL = cases.all_small_cases()


def _names(w):
    spl, _ = w.layouts()
    out = set()
    for metas in spl.layout.values():
        out |= set(metas)
    return out


def _check(w, payload="seeded", options=None, route="buffers"):
    print(f"[gpu parity] {w.key} payload={payload} options={options} route={route}", flush=True)
    glob = (global_state if payload == "seeded" else index_state)(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    got = gpu_execute(w, srcs, plan_options=options, route=route)
    assert set(got) == set(want)
    for name in want:
        assert set(got[name]) == set(want[name]), name
        for f in want[name]:
            np.testing.assert_array_equal(got[name][f], want[name][f], err_msg=f"{w.key}: {name}/{f}")
    return got


@pytest.mark.parametrize("route", ["buffers", "direct"])
@pytest.mark.parametrize("w", SMALL, ids=[w.key for w in SMALL])
def test_gpu_matches_oracle(w, route):
    _check(w, route=route)


PIPELINED = list(cases.scaled_configs().values()) + cases.dp_cases()[:2]


@pytest.mark.parametrize("route", ["buffers", "direct"])
@pytest.mark.parametrize("w", PIPELINED, ids=[w.key for w in PIPELINED])
def test_gpu_pipelined_launch_groups_match_oracle(w, route, monkeypatch):
    """execute_param_transfer in several launch groups (each planned while
    the previous one runs), forced on small cases: tensors dealt round robin
    into four groups, so no group is contiguous in schedule order."""
    from suika_amd import migration
    from tests.harness import round_robin_groups
    monkeypatch.setattr(migration, "_pipeline_groups", round_robin_groups(4))
    got = _check(w, payload="index", route=route)
    # the result lists the tensors in schedule order, whatever the launch order
    assert list(got) == list(dict.fromkeys(op.param_name for op in w.ops()))


@pytest.mark.parametrize("groups", [1, 4])
@pytest.mark.parametrize("w", SMALL, ids=[w.key for w in SMALL])
def test_gpu_one_call_direct_route_matches_oracle(w, groups, monkeypatch):
    """The drop-in call's default path -- per launch group one native call
    that plans, allocates the destinations and launches the gather -- run
    as is (no poisoning between allocation and launch, so the allocator's
    cache is left full of POISON bytes first), in one and in four launch
    groups, bit-exact against the oracle and listing the tensors in
    schedule order."""
    from suika_amd import migration
    from tests.harness import dirty_cache_execute, round_robin_groups
    print(f"[gpu parity] one-call {w.key} groups={groups}", flush=True)
    if groups > 1:
        monkeypatch.setattr(migration, "_pipeline_groups", round_robin_groups(groups))
    glob = index_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    got = dirty_cache_execute(w, srcs)
    assert list(got) == list(dict.fromkeys(op.param_name for op in w.ops()))
    for name in want:
        assert set(got[name]) == set(want[name]), name
        for f in want[name]:
            np.testing.assert_array_equal(got[name][f], want[name][f], err_msg=f"{w.key}: {name}/{f}")


SWEEP = cases.alignment_cases() + list(cases.scaled_configs().values())


@pytest.mark.parametrize("w", SWEEP, ids=[w.key for w in SWEEP])
@pytest.mark.parametrize("opt", [
    PlanOptions(tile_bytes=4096),
    PlanOptions(tile_bytes=8192, max_blocks=7),
    PlanOptions(nontemporal=False),
    PlanOptions(tile_bytes=1 << 20, nontemporal=False, max_blocks=300),
    PlanOptions(tile_bytes=4096, address_order=False),
    PlanOptions(tile_bytes=4096, xcd_order=False, max_blocks=33),
    PlanOptions(tile_bytes=4096, row_groups=False),
], ids=["tile4k", "tile8k_grid7", "temporal", "tile1m_temporal_grid300", "tile4k_piece_order",
        "tile4k_linear_grid33", "tile4k_no_row_groups"])
def test_gpu_tunings_match_oracle(w, opt):
    _check(w, "index", opt)
    _check(w, "index", opt, route="direct")


def test_gpu_repeat_and_streams():
    """A plan reused across calls, streams and rebound pointers stays exact."""
    from suika_amd.plan import ReshardPlan, SlotSpec
    from tests.harness import t2np, to_device
    w = cases.scaled_configs()["qwen7b_tp2_tp4"]
    print(f"[gpu repeat] {w.key}", flush=True)
    glob = global_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    ops = w.ops()
    dt = w.dtypes
    specs = {(op.src_rank, op.param_name, f): SlotSpec(tuple(op.src_meta.actual_shape()), dt[f])
             for op in ops for f in w.src_fields}
    plan = ReshardPlan(ops, specs, list(w.src_fields), recast=w.recast_map)
    dev = torch.device("cuda")
    side = torch.cuda.Stream()
    for it in range(4):
        sources = to_device(srcs, w, dev)
        bufs = plan.alloc_buffers(dev)
        dst = plan.alloc_dst(dev)
        for e in dst.values():
            for t in e.values():
                t.view(torch.uint8).fill_(0xA5)
        stream = side if it % 2 else torch.cuda.current_stream()
        if it % 2:
            side.wait_stream(torch.cuda.current_stream())
        plan.pack(sources, bufs, stream)
        plan.unpack(bufs, dst, stream)
        torch.cuda.synchronize()
        for name in want:
            for f in want[name]:
                np.testing.assert_array_equal(t2np(dst[name][f]), want[name][f],
                                              err_msg=f"iter {it}: {name}/{f}")
    plan.close()


@pytest.mark.parametrize("payload", ["seeded", "index"])
@pytest.mark.parametrize("case", sorted(cases.golden_cases()))
def test_gpu_reproduces_golden_vectors(payload, case):
    """The committed fixtures through the HIP path, bit for bit."""
    from tests.harness import load_reshard_vectors
    w = cases.golden_cases()[case]
    print(f"[gpu golden] {case} {payload}", flush=True)
    srcs, want = load_reshard_vectors()[payload][case]
    got = gpu_execute(w, srcs, route="direct" if payload == "index" else "buffers")
    assert set(got) == set(want)
    for name, ent in want.items():
        for f, a in ent.items():
            np.testing.assert_array_equal(got[name][f], a, err_msg=f"{case}: {name}/{f}")

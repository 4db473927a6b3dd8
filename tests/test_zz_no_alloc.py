"""The allocation-free gather (``sr_gather_noalloc``) against ``sr_gather``.

Both are called through the C ABI on the same plan and the same resident
sources, into separately poisoned destinations; the results must be equal
byte for byte, and equal to the oracle's reshard of the same seeded shards.
Two calls run in a row on the one per-GPU scratch, the second on a smaller
share, so stale tables of the first call cannot pass.
"""
import numpy as np
import pytest
import torch

from suika_amd.plan import ReshardPlan
from tests import cases
from tests.harness import POISON, global_state, oracle_dest, source_shards, t2np, to_device

pytestmark = pytest.mark.gpu


def _names(w):
    spl, _ = w.layouts()
    return {n for metas in spl.layout.values() for n in metas}


def _poisoned_dst(plan, dev):
    out, ptrs = plan.alloc_dst_ptrs(dev)
    for ent in out.values():
        for t in ent.values():
            t.view(torch.uint8).fill_(POISON)
    return out, ptrs


def _gather_both(w):
    """(sr_gather result, sr_gather_noalloc result, oracle result) of one share."""
    dev = torch.device("cuda", torch.cuda.current_device())
    glob = global_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    fake = to_device(srcs, w, dev)
    ops = [op for op in w.ops() if op.dst_rank == w.dst_rank]
    plan, src_ptrs = ReshardPlan.from_sources(ops, lambda r: fake[r], list(w.src_fields), dev,
                                              recast=w.recast_map, rank=w.dst_rank)
    try:
        ref, ref_ptrs = _poisoned_dst(plan, dev)
        got, got_ptrs = _poisoned_dst(plan, dev)
        plan.gather_ptrs(src_ptrs, ref_ptrs)
        plan.gather_noalloc_ptrs(src_ptrs, got_ptrs)
        torch.cuda.synchronize()
    finally:
        plan.close()
    to_np = lambda d: {n: {f: t2np(t) for f, t in e.items()} for n, e in d.items()}  # noqa: E731
    return to_np(ref), to_np(got), want


def _check(w):
    ref, got, want = _gather_both(w)
    assert set(got) == set(ref) == set(want)
    for name, ent in want.items():
        for f, a in ent.items():
            np.testing.assert_array_equal(got[name][f], ref[name][f], err_msg=f"{w.key}: {name}/{f} vs sr_gather")
            np.testing.assert_array_equal(got[name][f], a, err_msg=f"{w.key}: {name}/{f} vs oracle")


def test_noalloc_matches_gather_twice_second_smaller():
    cfg = cases.scaled_configs()
    big, small = cfg["qwen7b_tp2_tp4"], cfg["gpt125m_tp2_tp4"]
    for w in (big, small):
        print(f"[noalloc] {w.key}", flush=True)
        _check(w)


def test_noalloc_full_size_share_matches_gather():
    """The Llama2-7B share at full size fits the scratch at the default tile
    size; on index-coded sources the two gathers write the same bytes."""
    from oracle import reshard_oracle as O
    from suika_amd.plan import SlotSpec
    from suika_amd.workloads import CONFIGS
    from tests.harness import to_olayout
    from tests.test_gpu_fullsize import code
    w = CONFIGS["llama7b_tp4pp2_tp2pp2"]
    print(f"[noalloc] full size {w.key}", flush=True)
    dev = torch.device("cuda", torch.cuda.current_device())
    ops = w.ops()
    dt = w.dtypes
    specs = {(op.src_rank, op.param_name, f): SlotSpec(tuple(op.src_meta.actual_shape()), dt[f])
             for op in ops for f in w.src_fields}
    plan = ReshardPlan(ops, specs, list(w.src_fields), recast=w.recast_map)
    try:
        osrc = to_olayout(w.layouts()[0])
        names = sorted({n for metas in w.layouts()[0].layout.values() for n in metas})
        tid = {n: i for i, n in enumerate(names)}
        sources = {}
        for (r, name, f) in plan.src_keys:
            gidx = O.shard_index(osrc[r][name], xp=torch, device=dev)
            sources.setdefault(r, {}).setdefault(name, {})[f] = code(gidx, tid[name], f, dt[f]).contiguous()
            del gidx
        src_ptrs = plan.src_pointers(sources)
        ref, ref_ptrs = _poisoned_dst(plan, dev)
        got, got_ptrs = _poisoned_dst(plan, dev)
        plan.gather_ptrs(src_ptrs, ref_ptrs)
        plan.gather_noalloc_ptrs(src_ptrs, got_ptrs)
        torch.cuda.synchronize()
        del sources
    finally:
        plan.close()
    bad = [(name, f) for name, ent in ref.items() for f, t in ent.items()
           if not torch.equal(got[name][f].view(torch.uint8), t.view(torch.uint8))]
    assert not bad, f"{len(bad)} tensors differ, first {bad[:5]}"


def _small_plan():
    w = cases.scaled_configs()["gpt125m_tp2_tp4"]
    dev = torch.device("cuda", torch.cuda.current_device())
    srcs = source_shards(w, sorted(w.layouts()[0].layout), global_state(w, _names(w)))
    fake = to_device(srcs, w, dev)
    ops = [op for op in w.ops() if op.dst_rank == w.dst_rank]
    plan, src_ptrs = ReshardPlan.from_sources(ops, lambda r: fake[r], list(w.src_fields), dev,
                                              recast=w.recast_map, rank=w.dst_rank)
    dst, dst_ptrs = _poisoned_dst(plan, dev)
    return plan, fake, src_ptrs, dst, dst_ptrs


def test_noalloc_second_call_allocates_nothing():
    """After a first call (which, in a fresh process, also loads the
    library's GPU code and so places the scratch), a call changes neither
    the device's free memory nor torch's reserved memory."""
    print("[noalloc] allocation check", flush=True)
    plan, fake, src_ptrs, dst, dst_ptrs = _small_plan()
    try:
        plan.gather_noalloc_ptrs(src_ptrs, dst_ptrs)
        torch.cuda.synchronize()
        free0, _ = torch.cuda.mem_get_info()
        reserved0 = torch.cuda.memory_reserved()
        plan.gather_noalloc_ptrs(src_ptrs, dst_ptrs)
        torch.cuda.synchronize()
        free1, _ = torch.cuda.mem_get_info()
        assert free1 == free0, f"device free memory changed by {free0 - free1} bytes"
        assert torch.cuda.memory_reserved() == reserved0
    finally:
        plan.close()


def test_noalloc_refuses_graph_capture():
    """A stream that is capturing a graph is refused before any device work
    (the tables are uploaded from pageable memory at every call); the
    capture itself stays valid and holds only the work around the call."""
    print("[noalloc] capture refused", flush=True)
    plan, fake, src_ptrs, dst, dst_ptrs = _small_plan()
    try:
        plan.gather_noalloc_ptrs(src_ptrs, dst_ptrs)
        torch.cuda.synchronize()
        x = torch.zeros(16, device="cuda")
        g = torch.cuda.CUDAGraph()
        with pytest.raises(AssertionError, match="capturing a graph"):
            with torch.cuda.graph(g):
                x.add_(1)
                plan.gather_noalloc_ptrs(src_ptrs, dst_ptrs)
        torch.cuda.synchronize()
        for k in range(2):
            g.replay()
            torch.cuda.synchronize()
            assert float(x[0]) == k + 1
    finally:
        plan.close()

"""Randomised reshard cases: families, shapes, uneven stage partitions, TP
degrees 1/2/4/8 and DP replicas on both sides, every shard kind, random
destination rank.

CPU: the numpy execution of the product plan equals the oracle and the
closed form on index-coded state.  GPU: the HIP path equals the oracle.
Cases are drawn from fixed seeds, so a failure names a reproducible case.
"""
import random

import numpy as np
import pytest
import torch

from suika_amd.inventory import ModelSpec, Parallel
from suika_amd.plan import ReshardPlan, SlotSpec
from suika_amd.workloads import Workload
from tests.harness import (expected_dest, gpu_execute, index_state, oracle_dest, simulate_plan,
                           source_shards)
from tests.test_plan import _esize

_BF16_4 = (("param", torch.bfloat16), ("master", torch.float32),
           ("exp_avg", torch.float32), ("exp_avg_sq", torch.float32))
_F32_3 = (("param", torch.float32), ("exp_avg", torch.float32), ("exp_avg_sq", torch.float32))
_RECAST = (("master", torch.float32), ("exp_avg", torch.float32),
           ("exp_avg_sq", torch.float32), ("param", torch.bfloat16))


def random_case(seed: int) -> Workload:
    rng = random.Random(seed)
    family = rng.choice(["gpt", "llama", "qwen"])
    stp, dtp = rng.choice([1, 2, 4, 8]), rng.choice([1, 2, 4, 8])
    lcm = max(stp, dtp)
    n_layer = rng.randint(1, 5)
    spp = rng.choice([p for p in (1, 2, 3, 4) if p <= n_layer])
    dpp = rng.choice([p for p in (1, 2, 3, 4) if p <= n_layer])
    head_dim = rng.choice([2, 4, 6])
    n_kv = lcm * rng.choice([1, 2])
    n_head = n_kv * rng.choice([1, 2]) if family != "gpt" else lcm * rng.choice([1, 2])
    hidden = n_head * head_dim if family == "gpt" else lcm * rng.choice([2, 3, 4])
    if family == "gpt":
        head_dim = None
        n_kv = None
    ffn = lcm * rng.choice([3, 5, 8])
    vocab = lcm * rng.choice([5, 7, 12])
    vocab_parallel = rng.random() < 0.6
    fused = family != "gpt" and rng.random() < 0.4
    positions = rng.choice([0, 6]) if family == "gpt" else 0
    model = ModelSpec(family, n_layer=n_layer, hidden=hidden, n_head=n_head, ffn=ffn, vocab=vocab,
                      n_kv_head=n_kv, head_dim=head_dim, fused_qkv=fused,
                      vocab_parallel=vocab_parallel, pad_multiple=rng.choice([1, 3, 4]),
                      positions=positions)
    kind = rng.choice(["bf16", "f32", "recast"])
    fields = {"bf16": _BF16_4, "f32": _F32_3, "recast": _RECAST}[kind]
    recast = (("param", "master"),) if kind == "recast" else ()
    src_fields = tuple(f for f, _ in fields if f not in dict(recast))
    # data-parallel replicas on either side (one case in three)
    sdp, ddp = (rng.choice([1, 2]), rng.choice([1, 2])) if rng.random() < 0.34 else (1, 1)
    dst = Parallel(dtp, dpp, ddp)
    return Workload(key=f"fuzz{seed}", model=model, src=Parallel(stp, spp, sdp), dst=dst,
                    dst_pp=rng.randrange(dpp), dst_tp=rng.randrange(dtp), src_fields=src_fields,
                    field_dtypes=fields, recast=recast, seed=seed,
                    param_dtype=torch.float32 if kind == "f32" else torch.bfloat16,
                    dst_dp=rng.randrange(ddp))


SEEDS = list(range(60))
GPU_SEEDS = list(range(60, 120))


def _names(w):
    return {n for metas in w.layouts()[0].layout.values() for n in metas}


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_plan_simulation(seed):
    w = random_case(seed)
    glob = index_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    ops = w.ops()
    dt = w.dtypes
    specs = {(op.src_rank, op.param_name, f): SlotSpec(tuple(op.src_meta.actual_shape()), dt[f])
             for op in ops for f in w.src_fields}
    plan = ReshardPlan(ops, specs, list(w.src_fields), recast=w.recast_map)
    got = simulate_plan(plan, srcs, _esize)
    want = oracle_dest(w, srcs)
    closed = expected_dest(w, glob)
    assert {k[0] for k in got} == set(closed), w
    for (name, f), a in got.items():
        np.testing.assert_array_equal(a, want[name][f], err_msg=f"{w}: {name}/{f}")
        np.testing.assert_array_equal(a, closed[name][f], err_msg=f"{w}: {name}/{f}")
    plan.close()


@pytest.mark.gpu
@pytest.mark.parametrize("seed", GPU_SEEDS)
def test_fuzz_gpu(seed):
    w = random_case(seed)
    print(f"[gpu fuzz] {w}", flush=True)
    glob = index_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    # both routes, and every third case into one destination arena
    got = gpu_execute(w, srcs, route="direct" if seed % 2 else "buffers", arena=seed % 3 == 0)
    assert set(got) == set(want)
    for name, ent in want.items():
        for f, a in ent.items():
            np.testing.assert_array_equal(got[name][f], a, err_msg=f"{w.key}: {name}/{f}")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", GPU_SEEDS[::3])
def test_fuzz_gpu_fused_direct(seed, monkeypatch):
    """The drop-in call's default path -- one native call per launch group,
    fresh destinations built on the helper thread's blocks -- on random
    layouts, after dirtying the allocator cache; every other case in three
    round-robin launch groups, and half of them (of both kinds) given the
    world's whole schedule (its positions and encoding tables)."""
    from suika_amd import migration as M
    from suika_amd import schedule_param_transfer
    from tests.harness import dirty_cache_execute, round_robin_groups
    if seed % 2:
        monkeypatch.setattr(M, "_pipeline_groups", round_robin_groups(3))
    w = random_case(seed)
    print(f"[gpu fuzz fused] {w}", flush=True)
    glob = index_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    world = schedule_param_transfer(*w.layouts()) if seed % 4 in (0, 3) else None
    got = dirty_cache_execute(w, srcs, ops=world)
    assert set(got) == set(want)
    for name, ent in want.items():
        for f, a in ent.items():
            np.testing.assert_array_equal(got[name][f], a, err_msg=f"{w.key}: {name}/{f}")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", GPU_SEEDS[1::3])
def test_fuzz_gpu_host_sources(seed):
    """The staged route on random layouts: every source shard in host
    memory (the reference's checkpoint_load passes them so), the pieces'
    bytes packed by host threads and unpacked on the GPU, the result on the
    GPU or, every other case, back in host memory (``device="cpu"``);
    device-side destinations and buffers start as POISON bytes."""
    from suika_amd import execute_param_transfer
    from tests.harness import poisoned_allocations, t2np, to_device
    w = random_case(seed)
    device = "cpu" if seed % 2 else "cuda"
    print(f"[gpu fuzz host sources -> {device}] {w}", flush=True)
    glob = index_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    fake = to_device(srcs, w, "cpu")
    with poisoned_allocations():
        out = execute_param_transfer(w.ops(), {}, torch.device(device), [(f, "normal") for f in w.src_fields],
                                     rank=w.dst_rank, fake_source_state_dicts=fake, recast=w.recast_map)
    torch.cuda.synchronize()
    assert set(out) == set(want)
    for name, ent in want.items():
        for f, a in ent.items():
            t = out[name][f]
            assert t.device.type == device, f"{w.key}: {name}/{f} on {t.device}"
            np.testing.assert_array_equal(t2np(t), a, err_msg=f"{w.key}: {name}/{f}")

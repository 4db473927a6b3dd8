"""Processes of a live-migration test on one GPU (imported by spawned
children; see tests/test_gpu_live_migration.py).

An old rank plays a training process of the old plan: it starts like a fresh
launch (``migration_load`` reads the launcher's placeholder), fills its model
and AdamW state with seeded values cut from global tensors by the oracle's
closed form, reports ready, and calls ``migration_save``.  A new rank builds
its stage model on the meta device, calls ``migration_load`` with an optimizer
provider, and checks every parameter and optimizer state tensor it received
against the oracle's closed form of the same global tensors, bit for bit.
"""
from __future__ import annotations

import os
import sys
import traceback
from dataclasses import replace

import torch
import torch.distributed as dist

from oracle import reshard_oracle as O
from suika_amd.inventory import Parallel, build_module
from suika_amd.workloads import Workload
from tests import cases
from tests.harness import global_state, t2np, to_ometa

FIELDS = (("param", torch.float32), ("exp_avg", torch.float32), ("exp_avg_sq", torch.float32))
STEP = 7.0


def live_workload(old: Parallel, new: Parallel) -> Workload:
    base = cases.scaled_configs()["llama7b_tp4pp2_tp2pp2"]
    return replace(base, key="live", src=old, dst=new, dst_pp=0, dst_tp=0,
                   src_fields=tuple(f for f, _ in FIELDS), field_dtypes=FIELDS, recast=(), seed=11)


def _init(rank: int, world: int, port: int) -> None:
    os.environ.update(MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port))
    dist.init_process_group("gloo", rank=rank, world_size=world)
    torch.cuda.set_device(0)


def _logger(role: str, rank: int, sink: list):
    def log(msg: str) -> None:
        sink.append(msg)
        print(f"[{role} rank {rank}] {msg}", file=sys.stderr, flush=True)
    return log


def _glob(w: Workload):
    spl, _ = w.layouts()
    return global_state(w, {n for metas in spl.layout.values() for n in metas})


def old_rank(rank, world, port, queues, old, new, events):
    from suika_amd import migration_load, migration_save
    log = []
    try:
        _init(rank, world, port)
        w = live_workload(old, new)
        model = build_module(w.model, old, rank, torch.float32, device="cuda")
        optimizer = torch.optim.AdamW(model.parameters(), lr=1e-3)
        say = _logger("old", rank, log)
        assert migration_load(queues[rank], model, optimizer, log_func=say) is None, "fresh launch returns None"
        spl, _ = w.layouts()
        glob = _glob(w)
        metas = spl.layout[rank]
        for name, p in model.named_parameters():
            om = to_ometa(metas[name])
            shard = {f: torch.from_numpy(O.shard_of(glob[name][f], om).copy()).view(torch.float32).cuda()
                     for f, _ in FIELDS}
            with torch.no_grad():
                p.copy_(shard["param"])
            optimizer.state[p] = {"step": torch.tensor(STEP), "exp_avg": shard["exp_avg"],
                                  "exp_avg_sq": shard["exp_avg_sq"]}
        torch.cuda.synchronize()
        events.put(("ready", rank, None))
        migration_save(queues[rank], model, optimizer, other_context={"iter": 42}, log_func=say)
        events.put(("saved", rank, log))
    except BaseException:
        events.put(("error", rank, traceback.format_exc()))
    finally:
        if dist.is_initialized():
            dist.destroy_process_group()


def new_rank(rank, world, port, queues, old, new, events, wait_for_release=None):
    from suika_amd import migration_load
    log = []
    try:
        _init(rank, world, port)
        w = live_workload(old, new)
        model = build_module(w.model, new, rank, torch.float32, device="meta")
        optimizer, ctx = migration_load(queues[rank], model,
                                        lambda: torch.optim.AdamW(model.parameters(), lr=1e-3),
                                        log_func=_logger("new", rank, log), wait_for_release=wait_for_release)
        assert ctx == {"iter": 42}, ctx
        _, tpl = w.layouts()
        glob = _glob(w)
        metas = tpl.layout[rank]
        state = optimizer.state_dict()["state"]
        bad = []
        for idx, (name, p) in enumerate(model.named_parameters()):
            om = to_ometa(metas[name])
            want = {f: O.shard_of(glob[name][f], om) for f, _ in FIELDS}
            got = {"param": p, "exp_avg": state[idx]["exp_avg"], "exp_avg_sq": state[idx]["exp_avg_sq"]}
            for f, t in got.items():
                if not t.is_cuda or tuple(t.shape) != want[f].shape or not (t2np(t) == want[f]).all():
                    bad.append(f"{name}/{f}")
            if float(state[idx]["step"]) != STEP:
                bad.append(f"{name}/step")
        n = sum(1 for _ in model.parameters())
        events.put(("loaded", rank, {"tensors": 3 * n, "bad": bad, "log": log}))
    except BaseException:
        events.put(("error", rank, traceback.format_exc()))
    finally:
        if dist.is_initialized():
            dist.destroy_process_group()

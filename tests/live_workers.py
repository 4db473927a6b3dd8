"""Processes of a live-migration test on one GPU (imported by spawned
children; see tests/test_gpu_live_migration.py).

An old rank plays a training process of the old plan: it starts like a fresh
launch (``migration_load`` reads the launcher's placeholder), fills its model
and AdamW state with values cut from global tensors by the oracle's closed
form, reports ready, and calls ``migration_save``.  A new rank builds its
stage model on the meta device, calls ``migration_load`` with an optimizer
provider, and checks every parameter and optimizer state tensor it received
against the oracle's closed form of the same global tensors, bit for bit.

``opts`` (a dict) varies a run:
* ``wait_for_release`` / ``return_before_release``: passed to migration_load;
* ``mode`` / ``wave_bytes``: the hand-off order, passed to migration_save;
  ``ring=False`` gives every wave hand-off allocations of its own;
* ``spec``: a ModelSpec replacing the small default model, whose global
  tensors are then index-coded (cheap to build at a larger size);
* ``gate``: an event both worlds wait for after reporting ready (the new
  ranks having loaded the library), so the test can take device memory
  once every process holds its own;
* ``fail``: ``(side, rank, where)`` forces a failure in that process's host
  code: ``"survey"`` (the old rank finds a tensor too large for a hand-off
  allocation), ``"map"`` (the new rank cannot map the hand-off), ``"wave1"``
  (the new rank fails on the second wave's reshard).
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
from tests.harness import global_state, index_state, t2np, to_ometa

FIELDS = (("param", torch.float32), ("exp_avg", torch.float32), ("exp_avg_sq", torch.float32))
STEP = 7.0
GATE_TIMEOUT_S = 300


def live_workload(old: Parallel, new: Parallel, spec=None) -> Workload:
    base = cases.scaled_configs()["llama7b_tp4pp2_tp2pp2"]
    w = replace(base, key="live", src=old, dst=new, dst_pp=0, dst_tp=0,
                src_fields=tuple(f for f, _ in FIELDS), field_dtypes=FIELDS, recast=(), seed=11)
    return replace(w, model=spec) if spec is not None else w


def state_bytes(w: Workload) -> int:
    """Device bytes of the old world's state (every old rank's fields)."""
    spl, _ = w.layouts()
    n = 0
    for metas in spl.layout.values():
        for m in metas.values():
            numel = 1
            for d in m.actual_shape():
                numel *= int(d)
            n += numel * 4 * len(FIELDS)
    return n


def _init(rank: int, world: int, port: int) -> None:
    os.environ.update(MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port))
    dist.init_process_group("gloo", rank=rank, world_size=world)
    torch.cuda.set_device(0)


def _logger(role: str, rank: int, sink: list):
    def log(msg: str) -> None:
        sink.append(msg)
        print(f"[{role} rank {rank}] {msg}", file=sys.stderr, flush=True)
    return log


def _glob(w: Workload, names, indexed: bool):
    spl, _ = w.layouts()
    universe = {n for metas in spl.layout.values() for n in metas}
    if indexed:
        return index_state(w, names, universe=universe)
    return global_state(w, universe)


def _wait_gate(opts) -> None:
    gate = opts.get("gate")
    if gate is not None:
        assert gate.wait(GATE_TIMEOUT_S), "the test never opened the gate"


def _force(opts, side: str, rank: int) -> None:
    fail = opts.get("fail")
    if not fail or fail[0] != side or fail[1] != rank:
        return
    from suika_amd import _lib
    from suika_amd import handoff as H
    where = fail[2]
    if where == "survey":
        _lib.HANDOFF_MAX_BYTES = 1
    elif where == "map":
        class Unmappable:
            def __init__(self, *a, **k):
                raise RuntimeError("forced failure: cannot map the hand-off")
        H.MappedSources = Unmappable
    elif where == "wave1":
        real = H._NewWorld._reshard
        calls = []

        def reshard(self, *a, **k):
            calls.append(1)
            if len(calls) == 2:
                raise RuntimeError("forced failure in the second wave")
            return real(self, *a, **k)
        H._NewWorld._reshard = reshard
    else:
        raise ValueError(where)


def old_rank(rank, world, port, queues, old, new, events, opts=None):
    from suika_amd import migration_load, migration_save
    opts = opts or {}
    log = []
    try:
        _init(rank, world, port)
        w = live_workload(old, new, opts.get("spec"))
        model = build_module(w.model, old, rank, torch.float32, device="cuda")
        optimizer = torch.optim.AdamW(model.parameters(), lr=1e-3)
        say = _logger("old", rank, log)
        assert migration_load(queues[rank], model, optimizer, log_func=say) is None, "fresh launch returns None"
        spl, _ = w.layouts()
        metas = spl.layout[rank]
        glob = _glob(w, list(metas), opts.get("spec") is not None)
        for name, p in model.named_parameters():
            om = to_ometa(metas[name])
            shard = {f: torch.from_numpy(O.shard_of(glob[name][f], om).copy()).view(torch.float32).cuda()
                     for f, _ in FIELDS}
            with torch.no_grad():
                p.copy_(shard["param"])
            optimizer.state[p] = {"step": torch.tensor(STEP), "exp_avg": shard["exp_avg"],
                                  "exp_avg_sq": shard["exp_avg_sq"]}
            del glob[name]
        del glob
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        if opts.get("ring") is False:
            from suika_amd import handoff as H
            H.USE_RING = False
        _force(opts, "old", rank)
        events.put(("ready", rank, None))
        _wait_gate(opts)
        migration_save(queues[rank], model, optimizer, other_context={"iter": 42}, log_func=say,
                       handoff_mode=opts.get("mode"), wave_bytes=opts.get("wave_bytes"))
        events.put(("saved", rank, log))
    except BaseException:
        events.put(("error-old", rank, {"trace": traceback.format_exc(), "log": log}))
    finally:
        if dist.is_initialized():
            dist.destroy_process_group()


def new_rank(rank, world, port, queues, old, new, events, opts=None):
    from suika_amd import migration_load
    opts = opts or {}
    log = []
    try:
        _init(rank, world, port)
        w = live_workload(old, new, opts.get("spec"))
        model = build_module(w.model, new, rank, torch.float32, device="meta")
        if opts.get("gate") is not None:
            # the library's code and this process's first-use allocations in
            # place before the test measures the free memory
            from suika_amd.handoff import _WarmUp
            _WarmUp(torch.device("cuda", 0), optimizer=True).run()
            torch.cuda.synchronize()
            events.put(("ready-new", rank, None))
            _wait_gate(opts)
        _force(opts, "new", rank)
        optimizer, ctx = migration_load(queues[rank], model,
                                        lambda: torch.optim.AdamW(model.parameters(), lr=1e-3),
                                        log_func=_logger("new", rank, log),
                                        wait_for_release=opts.get("wait_for_release"),
                                        return_before_release=opts.get("return_before_release", False))
        assert ctx == {"iter": 42}, ctx
        _, tpl = w.layouts()
        metas = tpl.layout[rank]
        glob = _glob(w, list(metas), opts.get("spec") is not None)
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
        events.put(("error-new", rank, {"trace": traceback.format_exc(), "log": log}))
    finally:
        if dist.is_initialized():
            dist.destroy_process_group()

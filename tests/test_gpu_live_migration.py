"""Live migration between processes on one GPU (Suika/migration.py:1357-1727).

The test plays Suika's launcher (training.py:319-323).  One queue pair per
rank index, with the fresh-launch entries on the forward queues: 0 on rank
0's, and the placeholder dict on every one.  The old plan's processes start
first; once every one of them holds its seeded state, the new plan's
processes start.  ``migration_save`` / ``migration_load`` then run their
handshake, hand-off and reshard (suika_amd/handoff.py) with no checkpoint.
Each new rank checks its parameters and AdamW state against the oracle's
closed form, bit for bit.

Both of the reference's branches run:
* a world that shrinks (TP2 -> TP1: 2 old + 1 new processes);
* one that grows (TP1 -> TP2);
* one of equal size whose stages change (TP2 x PP2 -> TP4: 4 + 4 processes).

The small states leave room on the device, so the new world allocates its
destinations beside the old state; one more run of the last case makes it
wait for the old world's release (``WANT_RELEASED`` / ``RELEASED``) first.

Every process uses the GPU.  All stay within the box's per-card process limit.
"""
import multiprocessing as mp
import queue
import time

import pytest

from suika_amd.handoff import dummy_migration_IPC_state_dict
from suika_amd.inventory import Parallel

pytestmark = pytest.mark.gpu

TIMEOUT_S = 120


def _free_port() -> int:
    import socket
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _run(old: Parallel, new: Parallel, wait_for_release=None):
    from tests import live_workers as W
    ctx = mp.get_context("spawn")
    n = max(old.world, new.world)
    queues = [(ctx.Queue(), ctx.Queue()) for _ in range(n)]
    queues[0][0].put(0)
    for q in queues:
        q[0].put(dummy_migration_IPC_state_dict)
    events = ctx.Queue()
    procs = []
    deadline = time.time() + TIMEOUT_S
    results = {}

    def wait_for(kind, count):
        """Until ``count`` events of ``kind`` have arrived (since the start)."""
        while sum(1 for ev, _ in results if ev == kind) < count:
            try:
                ev, rank, payload = events.get(timeout=max(1.0, deadline - time.time()))
            except queue.Empty:
                raise AssertionError(f"timed out waiting for {kind}; so far {sorted(results)}")
            if ev == "error":
                raise AssertionError(f"rank {rank} failed:\n{payload}")
            results[(ev, rank)] = payload

    try:
        p_old, p_new = _free_port(), _free_port()
        for r in range(old.world):
            p = ctx.Process(target=W.old_rank, args=(r, old.world, p_old, queues, old, new, events))
            p.start()
            procs.append(p)
        wait_for("ready", old.world)
        for r in range(new.world):
            p = ctx.Process(target=W.new_rank, args=(r, new.world, p_new, queues, old, new, events,
                                                     wait_for_release))
            p.start()
            procs.append(p)
        wait_for("loaded", new.world)
        wait_for("saved", old.world)
        for p in procs:
            p.join(timeout=max(1.0, deadline - time.time()))
            assert p.exitcode == 0, f"process {p.pid} exit code {p.exitcode}"
    finally:
        for p in procs:
            if p.is_alive():
                p.kill()
                p.join(10)
    return results


@pytest.mark.parametrize("old,new", [(Parallel(tp=2), Parallel(tp=1)),
                                     (Parallel(tp=1), Parallel(tp=2)),
                                     (Parallel(tp=2, pp=2), Parallel(tp=4))],
                         ids=["tp2_to_tp1", "tp1_to_tp2", "tp2pp2_to_tp4"])
def test_live_migration_on_one_gpu(old, new):
    print(f"[gpu live migration] {old} -> {new}", flush=True)
    res = _run(old, new)
    for r in range(new.world):
        rec = res[("loaded", r)]
        assert rec["tensors"] > 0 and rec["bad"] == [], f"new rank {r}: {rec['bad'][:5]}"
        print(f"[gpu live migration] new rank {r}: {rec['tensors']} tensors exact; "
              f"{[m for m in rec['log'] if 'resharded' in m]}", flush=True)
    for r in range(old.world):
        log = res[("saved", r)]
        assert any("packed" in m for m in log) and log[-1] == "migration_save: end", log
    for r in range(new.world):
        assert any("beside the old state" in m for m in res[("loaded", r)]["log"]), res[("loaded", r)]["log"]


def test_live_migration_waiting_for_release():
    old, new = Parallel(tp=2, pp=2), Parallel(tp=4)
    print(f"[gpu live migration] {old} -> {new}, destinations after the old world's release", flush=True)
    res = _run(old, new, wait_for_release=True)
    for r in range(new.world):
        rec = res[("loaded", r)]
        assert rec["tensors"] > 0 and rec["bad"] == [], f"new rank {r}: {rec['bad'][:5]}"
        assert any("after the old world released its state" in m for m in rec["log"]), rec["log"]
    for r in range(old.world):
        assert res[("saved", r)][-1] == "migration_save: end"

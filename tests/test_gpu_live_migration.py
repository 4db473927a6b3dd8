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
* one of equal size whose stages change (TP2 x PP2 -> TP4: 4 + 4 processes);
* one whose old world holds data-parallel replicas (TP2 x DP2 -> TP4).

The small states leave room on the device, so the hand-off is whole and the
new world allocates its destinations beside the old state.  More runs of the
last case:
* the destinations wait for the old world's release (``WANT_RELEASED`` /
  ``RELEASED``);
* the new world returns without waiting for that release;
* the hand-off forced into many small waves, through the two-slot ring and
  with allocations of every wave's own, and into new worlds with pipeline
  stages (waves that give some new ranks nothing);
* a larger state while this process holds device memory so that less than
  the state itself is free: the old world picks waves, and the device's
  low-water free memory, as every rank logged it, shows at most two waves
  in use beyond the state;
* failures forced in one process's host code (an old rank's survey, a new
  rank's mapping, a new rank's second wave): every process of both worlds
  raises ``HandoffError`` and exits, none waits for the others.

Every process uses the GPU.  All stay within the box's per-card process limit.
"""
import multiprocessing as mp
import queue
import re
import time

import pytest

from suika_amd.handoff import dummy_migration_IPC_state_dict
from suika_amd.inventory import ModelSpec, Parallel

pytestmark = pytest.mark.gpu

TIMEOUT_S = 120


def _free_port() -> int:
    import socket
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _run(old: Parallel, new: Parallel, opts=None, expect_errors=False, on_ready=None, timeout_s=TIMEOUT_S):
    """Start both worlds; returns {(event, rank): payload} once every process
    has reported.  Without ``expect_errors`` a failing process fails the
    test.  ``on_ready`` runs once every process reported ready (with a
    ``gate`` in ``opts``, before the gate opens)."""
    from tests import live_workers as W
    opts = dict(opts or {})
    ctx = mp.get_context("spawn")
    n = max(old.world, new.world)
    queues = [(ctx.Queue(), ctx.Queue()) for _ in range(n)]
    queues[0][0].put(0)
    for q in queues:
        q[0].put(dummy_migration_IPC_state_dict)
    events = ctx.Queue()
    gated = bool(opts.pop("gated", False))
    if gated:
        opts["gate"] = ctx.Event()
    procs = []
    deadline = time.time() + timeout_s
    results = {}

    def wait_for(kinds, count):
        """Until ``count`` events of the ``kinds`` have arrived (since the start)."""
        while sum(1 for ev, _ in results if ev in kinds) < count:
            try:
                ev, rank, payload = events.get(timeout=max(1.0, deadline - time.time()))
            except queue.Empty:
                raise AssertionError(f"timed out waiting for {kinds}; so far {sorted(results)}")
            if ev.startswith("error") and not expect_errors:
                raise AssertionError(f"{ev} rank {rank} failed:\n{payload['trace']}")
            results[(ev, rank)] = payload

    try:
        p_old, p_new = _free_port(), _free_port()
        for r in range(old.world):
            p = ctx.Process(target=W.old_rank, args=(r, old.world, p_old, queues, old, new, events, opts))
            p.start()
            procs.append(p)
        wait_for(("ready", "error-old"), old.world)
        for r in range(new.world):
            p = ctx.Process(target=W.new_rank, args=(r, new.world, p_new, queues, old, new, events, opts))
            p.start()
            procs.append(p)
        if gated:
            wait_for(("ready-new",), new.world)
        if on_ready is not None:
            on_ready()
        if gated:
            opts["gate"].set()
        wait_for(("loaded", "error-new"), new.world)
        wait_for(("saved", "error-old"), old.world)
        for p in procs:
            p.join(timeout=max(1.0, deadline - time.time()))
            assert p.exitcode == 0, f"process {p.pid} exit code {p.exitcode}"
    finally:
        for p in procs:
            if p.is_alive():
                p.kill()
                p.join(10)
    return results


def _check_exact(res, new: Parallel, opts=None):
    for r in range(new.world):
        rec = res[("loaded", r)]
        assert rec["tensors"] > 0 and rec["bad"] == [], f"new rank {r}: {rec['bad'][:5]}"


def _low_water(log) -> float:
    """GB, from a rank's low-water line."""
    line = next(m for m in log if "low-water free device memory" in m)
    return float(re.search(r"memory ([0-9.]+) GB", line).group(1))


@pytest.mark.parametrize("old,new", [(Parallel(tp=2), Parallel(tp=1)),
                                     (Parallel(tp=1), Parallel(tp=2)),
                                     (Parallel(tp=2, pp=2), Parallel(tp=4)),
                                     (Parallel(tp=2, dp=2), Parallel(tp=4))],
                         ids=["tp2_to_tp1", "tp1_to_tp2", "tp2pp2_to_tp4", "tp2dp2_to_tp4"])
def test_live_migration_on_one_gpu(old, new):
    print(f"[gpu live migration] {old} -> {new}", flush=True)
    res = _run(old, new)
    _check_exact(res, new)
    for r in range(new.world):
        rec = res[("loaded", r)]
        print(f"[gpu live migration] new rank {r}: {rec['tensors']} tensors exact; "
              f"{[m for m in rec['log'] if 'resharded' in m]}", flush=True)
        assert any("beside the old state" in m for m in rec["log"]), rec["log"]
        assert any("the old world has released its state" in m for m in rec["log"]), rec["log"]
    for r in range(old.world):
        log = res[("saved", r)]
        assert any("hand-off whole" in m for m in log) and any("packed" in m for m in log), log
        assert log[-1] == "migration_save: end", log


def test_live_migration_waiting_for_release():
    old, new = Parallel(tp=2, pp=2), Parallel(tp=4)
    print(f"[gpu live migration] {old} -> {new}, destinations after the old world's release", flush=True)
    res = _run(old, new, {"wait_for_release": True})
    _check_exact(res, new)
    for r in range(new.world):
        assert any("after the old world released its state" in m for m in res[("loaded", r)]["log"])
    for r in range(old.world):
        assert res[("saved", r)][-1] == "migration_save: end"


def test_live_migration_returning_before_release():
    """With ``return_before_release`` the new world does not wait for the old
    world's release: the old world sends no RELEASED, and both finish."""
    old, new = Parallel(tp=2, pp=2), Parallel(tp=4)
    print(f"[gpu live migration] {old} -> {new}, returning before the release", flush=True)
    res = _run(old, new, {"return_before_release": True})
    _check_exact(res, new)
    for r in range(new.world):
        log = res[("loaded", r)]["log"]
        assert any("beside the old state" in m for m in log), log
        assert not any("the old world has released its state" in m for m in log), log
    for r in range(old.world):
        assert res[("saved", r)][-1] == "migration_save: end"


@pytest.mark.parametrize("ring", [True, False], ids=["ring", "per_wave_allocations"])
def test_live_migration_in_many_waves(ring):
    """The hand-off forced into waves of 64 KiB: names move a few at a time,
    every wave a reshard of its own, and the result is exact -- through the
    two slots every wave reuses, and with allocations of every wave's own."""
    old, new = Parallel(tp=2, pp=2), Parallel(tp=4)
    print(f"[gpu live migration] {old} -> {new}, waves of 64 KiB, ring {ring}", flush=True)
    res = _run(old, new, {"mode": "waves", "wave_bytes": 64 << 10, "ring": ring})
    _check_exact(res, new)
    waves = None
    for r in range(old.world):
        log = res[("saved", r)]
        assert any("in waves of at most" in m for m in log), log
        assert any("ring of 2 x" in m for m in log) == ring, log
        line = next(m for m in log if "handed off in" in m)
        k = int(re.search(r"in (\d+) wave", line).group(1))
        assert waves in (None, k)
        waves = k
    assert waves > 4, waves
    for r in range(new.world):
        assert any(f"destinations of {waves} wave(s)" in m for m in res[("loaded", r)]["log"])


@pytest.mark.parametrize("old,new", [(Parallel(tp=4), Parallel(tp=2, pp=2)),
                                     (Parallel(tp=1, pp=2), Parallel(tp=2, pp=2)),
                                     (Parallel(tp=2, dp=2), Parallel(tp=4))],
                         ids=["tp4_to_tp2pp2", "tp1pp2_to_tp2pp2", "tp2dp2_to_tp4"])
def test_live_migration_waves_into_stages(old, new):
    """Waves into a new world with pipeline stages: a wave whose names all
    belong to one stage gives the other stage's ranks nothing to reshard,
    and they still report it consumed; the world grows from 2 to 4 ranks in
    the second case.  The third case comes from data-parallel replicas: each
    new rank maps only the replicas the schedule picked for its pieces.
    Exact against the oracle."""
    print(f"[gpu live migration] {old} -> {new}, waves of 32 KiB", flush=True)
    res = _run(old, new, {"mode": "waves", "wave_bytes": 32 << 10})
    _check_exact(res, new)
    for r in range(old.world):
        assert any("handed off in" in m for m in res[("saved", r)]), res[("saved", r)]


# about 2.4 GB of fp32 parameters and Adam moments over the four old ranks
SQUEEZE_SPEC = ModelSpec("llama", n_layer=12, hidden=1024, n_head=8, ffn=2816, vocab=16000)


@pytest.mark.timeout(300)
def test_live_migration_when_the_device_lacks_room_for_two_states():
    """This process holds device memory until less than the old state itself
    is free (70% of it) beside the eight processes: a whole hand-off does
    not fit, so the old world moves the state in waves, and every new rank
    is exact.  The device's low-water free memory over every rank's samples
    shows at most two waves (plus the per-process reserve) in use beyond
    what was in use when the migration began."""
    import torch

    from suika_amd.handoff import RESERVE_BYTES
    from tests.live_workers import live_workload, state_bytes
    old, new = Parallel(tp=2, pp=2), Parallel(tp=4)
    S = state_bytes(live_workload(old, new, SQUEEZE_SPEC))
    print(f"[gpu live migration] {old} -> {new}, {S / 1e9:.2f} GB state, 0.7x of it free", flush=True)
    held = {}

    def squeeze():
        torch.cuda.synchronize()
        free, _ = torch.cuda.mem_get_info()
        hold = free - int(0.7 * S)
        assert hold > 0, (free, S)
        held["t"] = torch.empty(hold, dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()
        held["free"] = torch.cuda.mem_get_info()[0]
        print(f"[gpu live migration] holding {hold / 1e9:.1f} GB; {held['free'] / 1e9:.3f} GB free", flush=True)

    try:
        res = _run(old, new, {"spec": SQUEEZE_SPEC, "gated": True}, on_ready=squeeze, timeout_s=300)
    finally:
        held.pop("t", None)
        torch.cuda.empty_cache()
    _check_exact(res, new)
    log0 = res[("saved", 0)]
    line = next(m for m in log0 if "hand-off in waves of at most" in m)
    wave = float(re.search(r"at most ([0-9.]+) GB", line).group(1)) * 1e9
    lows = [_low_water(res[("saved", r)]) for r in range(old.world)] + \
        [_low_water(res[("loaded", r)]["log"]) for r in range(new.world)]
    extra = held["free"] - min(lows) * 1e9
    bound = 2 * wave + RESERVE_BYTES * (old.world + new.world)
    print(f"[gpu live migration] waves of {wave / 1e9:.3f} GB; peak beyond the start "
          f"{extra / 1e9:.3f} GB (bound {bound / 1e9:.3f} GB)", flush=True)
    assert extra <= bound, (extra, bound)


@pytest.mark.parametrize("fail,opts", [
    (("old", 1, "survey"), {}),
    (("new", 2, "map"), {}),
    (("new", 1, "wave1"), {"mode": "waves", "wave_bytes": 256 << 10}),
], ids=["old_survey", "new_map", "new_wave1"])
def test_a_failure_on_one_rank_ends_both_worlds(fail, opts):
    """A failure forced in one process's host code raises HandoffError on
    every process of both worlds, and every process exits on its own well
    within the test's time limit."""
    old, new = Parallel(tp=2, pp=2), Parallel(tp=4)
    print(f"[gpu live migration] {old} -> {new}, failure forced at {fail}", flush=True)
    t0 = time.time()
    res = _run(old, new, {**opts, "fail": fail}, expect_errors=True)
    took = time.time() - t0
    for side, world in (("old", old.world), ("new", new.world)):
        for r in range(world):
            ev = res.get((f"error-{side}", r))
            assert ev is not None, f"{side} rank {r} did not fail: {sorted(res)}"
            assert "HandoffError" in ev["trace"], ev["trace"]
    assert took < TIMEOUT_S, took

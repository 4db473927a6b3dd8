"""The same-GPU hand-off on the host: the C ABI's argument checks (no device
call is made for a rejected argument) and the packing layout."""
import ctypes

import pytest

from suika_amd import _lib
from suika_amd.handoff import ALIGN, pack_layout


def test_handoff_abi_rejects_bad_arguments_before_any_device_call():
    L = _lib.lib()
    ptr, h = ctypes.c_void_p(), _lib.SrIpcHandle()
    assert ctypes.sizeof(h) == 64
    assert L.sr_handoff_alloc(0, ctypes.byref(ptr), ctypes.byref(h)) == _lib.SR_EINVAL
    assert L.sr_handoff_alloc(_lib.HANDOFF_MAX_BYTES + 1, ctypes.byref(ptr), ctypes.byref(h)) == _lib.SR_EINVAL
    assert "outside 1..2146435072" in _lib.last_error()
    assert L.sr_handoff_alloc(64, None, ctypes.byref(h)) == _lib.SR_EINVAL
    assert L.sr_handoff_open(None, ctypes.byref(ptr)) == _lib.SR_EINVAL
    assert L.sr_handoff_open(ctypes.byref(h), None) == _lib.SR_EINVAL
    assert L.sr_handoff_close(None) == _lib.SR_EINVAL
    assert L.sr_handoff_free(None) == _lib.SR_EINVAL
    assert _lib.HANDOFF_MAX_BYTES == (2 << 30) - (1 << 20) and _lib.HANDOFF_MAX_BYTES < 2 << 30


def test_pack_layout_aligned_chunks_within_limits():
    sizes_in = [100, 1000, 3000, 5000, 70000, 10, 1]
    where, sizes = pack_layout(sizes_in, chunk_bytes=8192)
    ends = {}
    for n, (c, off) in zip(sizes_in, where):
        assert off % ALIGN == 0
        assert off + n <= sizes[c]
        ends.setdefault(c, []).append((off, off + n))
    for c, spans in ends.items():
        spans.sort()
        assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:])), "tensors of a chunk overlap"
        assert sizes[c] == spans[-1][1], "a chunk ends where its last tensor does"
        assert sizes[c] <= 8192 or len(spans) == 1, "only a lone tensor exceeds the chunk size"
    assert [c for c, _ in where] == [0, 0, 0, 1, 2, 3, 3]
    assert where[4] == (2, 0) and sizes[2] == 70000     # larger than a chunk: alone


def test_pack_layout_refuses_tensors_beyond_the_limit():
    with pytest.raises(AssertionError, match="does not fit one hand-off allocation"):
        pack_layout([_lib.HANDOFF_MAX_BYTES + 1])
    with pytest.raises(AssertionError):
        pack_layout([0])
    where, sizes = pack_layout([_lib.HANDOFF_MAX_BYTES, 1])
    assert sizes == [_lib.HANDOFF_MAX_BYTES, 1] and where == [(0, 0), (1, 0)]


def test_destination_bytes_sum_the_new_ranks_shards():
    """The bytes a new rank reserves beside the old state: every name of its
    layout once, its shard's elements times each field's item size from the
    old ranks' records, each tensor rounded up to 256 bytes."""
    from suika_amd import schedule_param_transfer
    from suika_amd.handoff import _destination_bytes
    from suika_amd.workloads import CONFIGS
    w = CONFIGS["gpt125m_tp2_tp4"]
    spl, tpl = w.layouts()
    ops = schedule_param_transfer(spl, tpl)
    fields = {"param": "torch.bfloat16", "exp_avg": "torch.float32", "exp_avg_sq": "torch.float32"}
    records = [{"rank": r, "tensors": {n: {f: (0, 0, tuple(m.actual_shape()), dt) for f, dt in fields.items()}
                                       for n, m in metas.items()}}
               for r, metas in spl.layout.items()]
    per_elem = {"torch.bfloat16": 2, "torch.float32": 4}
    for rank, metas in tpl.layout.items():
        want = 0
        for n, m in metas.items():
            numel = 1
            for d in m.actual_shape():
                numel *= int(d)
            want += sum((numel * per_elem[dt] + ALIGN - 1) // ALIGN * ALIGN for dt in fields.values())
        assert _destination_bytes(ops, rank, records) == want, rank
    # a rank with no ops of its own needs nothing
    assert _destination_bytes([op for op in ops if op.dst_rank != 0], 0, records) == 0


def test_plan_waves_interleaves_stages_and_keeps_each_name_whole():
    """Names are taken round-robin over the old ranks' own orders (pipeline
    stages share every wave), each once, and a wave closes before the name
    that would take its bytes, summed over the ranks, past the limit."""
    from suika_amd.handoff import plan_waves
    stage0 = [("emb", 40), ("l0", 10), ("l1", 10)]
    stage1 = [("l2", 10), ("l3", 10), ("head", 40)]
    per_rank = [stage0, stage0, stage1, stage1]          # TP2 x PP2
    # bytes summed over the ranks holding a name: emb 80, each layer 20, head 80
    assert plan_waves(per_rank, 100) == [["emb", "l2"], ["l0", "l3", "l1"], ["head"]]
    assert plan_waves(per_rank, 79) == [["emb"], ["l2", "l0", "l3"], ["l1"], ["head"]]
    assert plan_waves(per_rank, 1) == [["emb"], ["l2"], ["l0"], ["l3"], ["l1"], ["head"]]
    assert plan_waves(per_rank, 10 ** 9) == [["emb", "l2", "l0", "l3", "l1", "head"]]
    assert plan_waves([], 10) == [] and plan_waves([[], []], 10) == []


def test_plan_waves_brute_force_properties():
    import random

    from suika_amd.handoff import plan_waves
    rng = random.Random(5)
    for _ in range(300):
        names = [f"n{i}" for i in range(rng.randint(0, 12))]
        ranks = []
        for _ in range(rng.randint(1, 5)):
            mine = [n for n in names if rng.random() < 0.7]
            rng.shuffle(mine)
            ranks.append([(n, rng.randint(0, 50)) for n in mine])
        limit = rng.randint(1, 120)
        waves = plan_waves(ranks, limit)
        total = {}
        for r in ranks:
            for n, b in r:
                total[n] = total.get(n, 0) + b
        # the round-robin order, each name once
        order, seen = [], set()
        for i in range(max((len(r) for r in ranks), default=0)):
            for r in ranks:
                if i < len(r) and r[i][0] not in seen:
                    seen.add(r[i][0])
                    order.append(r[i][0])
        assert [n for w in waves for n in w] == order
        for k, w in enumerate(waves):
            s = sum(total[n] for n in w)
            assert w and (s <= limit or len(w) == 1)
            if k + 1 < len(waves):      # greedy: the next name did not fit
                assert s + total[waves[k + 1][0]] > limit


def test_choose_order_whole_waves_and_refusals():
    from suika_amd.handoff import RESERVE_BYTES, HandoffError, choose_order
    GB = 10 ** 9
    reserve = RESERVE_BYTES * 8
    # room for the hand-off beside the state: whole
    assert choose_order(100 * GB, GB, 100 * GB + reserve, 8) == ("whole", 0)
    # less: waves of a third of the room, at least the largest name
    room = 60 * GB
    assert choose_order(100 * GB, GB, room + reserve, 8) == ("waves", room // 3)
    assert choose_order(100 * GB, 25 * GB, room + reserve, 8) == ("waves", 25 * GB)
    # two waves of the largest name must fit
    with pytest.raises(HandoffError, match="lacks memory for a hand-off in waves"):
        choose_order(100 * GB, 31 * GB, room + reserve, 8)
    with pytest.raises(HandoffError, match="lacks memory"):
        choose_order(100 * GB, GB, reserve // 2, 8)
    # forced orders
    assert choose_order(GB, GB, 100 * GB + reserve, 8, mode="waves", wave_bytes=2 * GB) == ("waves", 2 * GB)
    assert choose_order(GB, 3 * GB, 100 * GB + reserve, 8, mode="waves", wave_bytes=2 * GB) == ("waves", 3 * GB)
    with pytest.raises(HandoffError, match="does not fit beside the old state"):
        choose_order(100 * GB, GB, room + reserve, 8, mode="whole")
    with pytest.raises(ValueError, match="hand-off mode"):
        choose_order(GB, GB, 100 * GB, 8, mode="chunks")


def test_error_notes_and_agreement_helpers():
    """The protocol's error note is recognised, and a queue read that times
    out turns into one."""
    import queue as _queue

    from suika_amd import handoff as H
    assert H._is_error(H._error_note("x")) and not H._is_error(("wave", 0)) and not H._is_error(H.DONE)
    q = _queue.Queue()
    old = H.QUEUE_TIMEOUT_S
    H.QUEUE_TIMEOUT_S = 0.05
    try:
        note = H._recv(q, "a test message")
    finally:
        H.QUEUE_TIMEOUT_S = old
    assert H._is_error(note) and "no a test message from the other world" in note[1]
    q.put(H.DONE)
    assert H._recv(q, "DONE") == H.DONE


def _agree_worker(rank, port, out):
    import os

    import torch.distributed as dist

    from suika_amd import handoff as H
    os.environ.update(MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port))
    dist.init_process_group("gloo", rank=rank, world_size=2)
    try:
        H._agree(None, None, "a step both pass")
        try:
            H._agree(None, "ValueError: boom" if rank == 1 else None, "a step rank 1 fails")
            out.put((rank, "no error"))
        except H.HandoffError as e:
            out.put((rank, (str(e), e.notify)))
    finally:
        dist.destroy_process_group()


def test_agree_raises_on_every_rank_of_the_world():
    """An error on one rank of a world raises on every rank (gloo, two
    processes), naming the failing rank, with the other world still to be
    told."""
    import multiprocessing as mp
    import socket
    with socket.socket() as s_:
        s_.bind(("127.0.0.1", 0))
        port = s_.getsockname()[1]
    ctx = mp.get_context("spawn")
    out = ctx.Queue()
    procs = [ctx.Process(target=_agree_worker, args=(r, port, out)) for r in range(2)]
    for p in procs:
        p.start()
    got = dict(out.get(timeout=120) for _ in procs)
    for p in procs:
        p.join(60)
        assert p.exitcode == 0
    for r in range(2):
        msg, notify = got[r]
        assert msg == "a step rank 1 fails failed on rank 1: ValueError: boom" and notify is True

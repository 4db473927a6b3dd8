"""The plan tables built on the GPU: per-peer buffer offsets (a wavefront
prefix sum per peer), the tile table (a prefix sum over item tile counts,
emitted in XCD-interleaved order) and the item table bound to the caller's
pointers.

The host computes the same buffer layout at plan creation
(``sr_plan_piece_offset``) -- that layout is the wire format between
peers -- so after ``sr_pack`` every piece's payload must sit at the host's
offset in its peer buffer, with the alignment gaps untouched.  The plan has
more than 256 pieces per peer and more than 1024 items, so both scans carry
across several workgroup-sized chunks, and u8 payloads of odd length, so
the 256-byte rounding is exercised.
"""
import ctypes
import random

import numpy as np
import pytest
import torch

from suika_amd import _lib

ROWS, COLS, SPLIT = 3000, 333, 150
BLOCK_FROM, BLOCK_ROWS = 2000, 100
N_PEERS = 3
POISON = 0xEE


def _pieces(seed):
    """Rows [0, BLOCK_FROM): two single-row pieces per row; the rest in
    blocks of BLOCK_ROWS rows cut at column SPLIT (strided pieces).  Peers
    are drawn at random; destination = source (an identity reshard)."""
    rng = random.Random(seed)
    out = []

    def add(r0, rows, c0, cols):
        out.append(_lib.SrPiece(_lib.SR_PIECE_COPY, rng.randrange(N_PEERS), 0, 0, -1, 0,
                                rows, cols, r0, c0, r0, c0))

    for r in range(BLOCK_FROM):
        add(r, 1, 0, SPLIT)
        add(r, 1, SPLIT, COLS - SPLIT)
    for r in range(BLOCK_FROM, ROWS, BLOCK_ROWS):
        add(r, BLOCK_ROWS, 0, SPLIT)
        add(r, BLOCK_ROWS, SPLIT, COLS - SPLIT)
    rng.shuffle(out)
    return out


def _vp(ptrs):
    return (ctypes.c_void_p * len(ptrs))(*ptrs)


@pytest.mark.gpu
@pytest.mark.parametrize("flags", [0, _lib.SR_OPT_PIECE_ORDER | _lib.SR_OPT_NO_XCD_INTERLEAVE])
def test_device_offsets_match_host_layout(flags):
    print(f"[gpu device-plan] flags={flags}", flush=True)
    L = _lib.lib()
    pcs = _pieces(seed=7 + flags)
    per_peer = np.bincount([p.peer for p in pcs], minlength=N_PEERS)
    assert len(pcs) > 1024 and per_peer.min() > 256
    t = (_lib.SrTensor * 1)(_lib.SrTensor(ROWS, COLS, _lib.SR_DT_U8, 0))
    arr = (_lib.SrPiece * len(pcs))(*pcs)
    opt = _lib.SrPlanOptions(4096, 0, flags, 0)
    h = ctypes.c_void_p()
    _lib.check(L.sr_plan_create(t, 1, t, 1, N_PEERS, arr, len(pcs), ctypes.byref(opt), ctypes.byref(h)),
               "sr_plan_create")
    try:
        peer_bytes, offsets = [], []
        for q in range(N_PEERS):
            b = ctypes.c_uint64()
            _lib.check(L.sr_plan_peer_bytes(h, q, ctypes.byref(b)), "peer_bytes")
            peer_bytes.append(b.value)
        for k in range(len(pcs)):
            o = ctypes.c_uint64()
            _lib.check(L.sr_plan_piece_offset(h, k, ctypes.byref(o)), "piece_offset")
            offsets.append(o.value)

        gen = torch.Generator("cpu").manual_seed(5)
        src_h = torch.randint(0, 256, (ROWS, COLS), dtype=torch.uint8, generator=gen)
        src = src_h.cuda()
        bufs = [torch.full((max(1, n),), POISON, dtype=torch.uint8, device="cuda") for n in peer_bytes]
        stream = torch.cuda.current_stream().cuda_stream
        _lib.check(L.sr_pack(h, _vp([src.data_ptr()]), _vp([b.data_ptr() for b in bufs]), stream), "sr_pack")
        torch.cuda.synchronize()

        host_bufs = [b.cpu().numpy() for b in bufs]
        want = [np.full(max(1, n), POISON, dtype=np.uint8) for n in peer_bytes]
        s = src_h.numpy()
        for k, p in enumerate(pcs):
            payload = s[p.src_row:p.src_row + p.rows, p.src_col:p.src_col + p.cols].reshape(-1)
            want[p.peer][offsets[k]:offsets[k] + payload.size] = payload
        for q in range(N_PEERS):
            np.testing.assert_array_equal(host_bufs[q], want[q], err_msg=f"peer {q} buffer layout")

        for route in ("unpack", "gather"):
            dst = torch.full((ROWS, COLS), POISON, dtype=torch.uint8, device="cuda")
            if route == "unpack":
                rc = L.sr_unpack(h, _vp([b.data_ptr() for b in bufs]), _vp([dst.data_ptr()]), stream)
            else:
                rc = L.sr_gather(h, _vp([src.data_ptr()]), _vp([dst.data_ptr()]), stream)
            _lib.check(rc, route)
            torch.cuda.synchronize()
            assert torch.equal(dst.cpu(), src_h), route
    finally:
        L.sr_plan_destroy(h)


@pytest.mark.gpu
def test_rebind_on_new_pointers_and_stream():
    """A plan reused with other tensors on another stream re-binds its item
    table there (pointer table upload + bind kernel) and stays exact."""
    print("[gpu device-plan] rebind", flush=True)
    L = _lib.lib()
    pcs = _pieces(seed=11)
    t = (_lib.SrTensor * 1)(_lib.SrTensor(ROWS, COLS, _lib.SR_DT_U8, 0))
    arr = (_lib.SrPiece * len(pcs))(*pcs)
    h = ctypes.c_void_p()
    _lib.check(L.sr_plan_create(t, 1, t, 1, N_PEERS, arr, len(pcs), None, ctypes.byref(h)), "sr_plan_create")
    try:
        side = torch.cuda.Stream()
        for i, stream in enumerate([torch.cuda.current_stream(), side, side, torch.cuda.current_stream()]):
            gen = torch.Generator("cpu").manual_seed(100 + i)
            src_h = torch.randint(0, 256, (ROWS, COLS), dtype=torch.uint8, generator=gen)
            with torch.cuda.stream(stream):
                src = src_h.cuda()
                dst = torch.full((ROWS, COLS), POISON, dtype=torch.uint8, device="cuda")
                _lib.check(L.sr_gather(h, _vp([src.data_ptr()]), _vp([dst.data_ptr()]), stream.cuda_stream),
                           "sr_gather")
            stream.synchronize()
            assert torch.equal(dst.cpu(), src_h), i
    finally:
        L.sr_plan_destroy(h)


@pytest.mark.gpu
def test_destroy_right_after_async_launch():
    """sr_plan_destroy directly after sr_gather / sr_pack + sr_unpack, with
    no synchronisation in between: the destroy waits for the plan's own
    launches, so the results are complete and exact."""
    print("[gpu device-plan] destroy after async launch", flush=True)
    L = _lib.lib()
    pcs = _pieces(seed=13)
    t = (_lib.SrTensor * 1)(_lib.SrTensor(ROWS, COLS, _lib.SR_DT_U8, 0))
    arr = (_lib.SrPiece * len(pcs))(*pcs)
    gen = torch.Generator("cpu").manual_seed(21)
    src_h = torch.randint(0, 256, (ROWS, COLS), dtype=torch.uint8, generator=gen)
    src = src_h.cuda()
    stream = torch.cuda.current_stream().cuda_stream
    for route in ("gather", "buffers"):
        h = ctypes.c_void_p()
        _lib.check(L.sr_plan_create(t, 1, t, 1, N_PEERS, arr, len(pcs), None, ctypes.byref(h)), "create")
        dst = torch.full((ROWS, COLS), POISON, dtype=torch.uint8, device="cuda")
        if route == "gather":
            _lib.check(L.sr_gather(h, _vp([src.data_ptr()]), _vp([dst.data_ptr()]), stream), "gather")
        else:
            sizes = []
            for q in range(N_PEERS):
                b = ctypes.c_uint64()
                _lib.check(L.sr_plan_peer_bytes(h, q, ctypes.byref(b)), "peer_bytes")
                sizes.append(b.value)
            bufs = [torch.empty(max(1, n), dtype=torch.uint8, device="cuda") for n in sizes]
            bp = _vp([b.data_ptr() for b in bufs])
            _lib.check(L.sr_pack(h, _vp([src.data_ptr()]), bp, stream), "pack")
            _lib.check(L.sr_unpack(h, bp, _vp([dst.data_ptr()]), stream), "unpack")
        L.sr_plan_destroy(h)
        torch.cuda.synchronize()
        assert torch.equal(dst.cpu(), src_h), route


@pytest.mark.gpu
def test_two_plans_concurrently_on_two_streams():
    """Independent plans own their tables, staging and events: a gather of
    one plan and a pack + unpack of another, issued on two streams without
    synchronisation in between, both come out exact."""
    print("[gpu device-plan] two plans, two streams", flush=True)
    L = _lib.lib()
    t = (_lib.SrTensor * 1)(_lib.SrTensor(ROWS, COLS, _lib.SR_DT_U8, 0))
    plans = []
    for seed in (31, 32):
        pcs = _pieces(seed=seed)
        arr = (_lib.SrPiece * len(pcs))(*pcs)
        h = ctypes.c_void_p()
        _lib.check(L.sr_plan_create(t, 1, t, 1, N_PEERS, arr, len(pcs), None, ctypes.byref(h)), "create")
        plans.append(h)
    try:
        gen = torch.Generator("cpu").manual_seed(41)
        srcs_h = [torch.randint(0, 256, (ROWS, COLS), dtype=torch.uint8, generator=gen) for _ in range(2)]
        srcs = [s.cuda() for s in srcs_h]
        dsts = [torch.full((ROWS, COLS), POISON, dtype=torch.uint8, device="cuda") for _ in range(2)]
        sizes = []
        for q in range(N_PEERS):
            b = ctypes.c_uint64()
            _lib.check(L.sr_plan_peer_bytes(plans[1], q, ctypes.byref(b)), "peer_bytes")
            sizes.append(b.value)
        bufs = [torch.empty(max(1, n), dtype=torch.uint8, device="cuda") for n in sizes]
        torch.cuda.synchronize()
        s0, s1 = torch.cuda.Stream(), torch.cuda.Stream()
        _lib.check(L.sr_gather(plans[0], _vp([srcs[0].data_ptr()]), _vp([dsts[0].data_ptr()]),
                               s0.cuda_stream), "gather")
        bp = _vp([b.data_ptr() for b in bufs])
        _lib.check(L.sr_pack(plans[1], _vp([srcs[1].data_ptr()]), bp, s1.cuda_stream), "pack")
        _lib.check(L.sr_unpack(plans[1], bp, _vp([dsts[1].data_ptr()]), s1.cuda_stream), "unpack")
        torch.cuda.synchronize()
        for i in range(2):
            assert torch.equal(dsts[i].cpu(), srcs_h[i]), i
    finally:
        for h in plans:
            L.sr_plan_destroy(h)


@pytest.mark.gpu
def test_plan_tables_reused_across_threads_and_sizes():
    """Destroyed plans hand their table memory and events to a per-process
    cache; new plans of other sizes reuse them.  Four host threads, each on
    its own stream, create, run and destroy plans of different sizes
    concurrently; every result stays exact."""
    import threading
    print("[gpu device-plan] table cache, 4 threads", flush=True)
    L = _lib.lib()
    errors = []

    def worker(tid):
        try:
            stream = torch.cuda.Stream()
            gen = torch.Generator("cpu").manual_seed(200 + tid)
            for it in range(6):
                rows = [ROWS, 700, 1500][(tid + it) % 3]
                pcs = [p for p in _pieces(seed=50 + tid * 10 + it) if p.src_row + p.rows <= rows]
                # keep the destination covered: whole rows of the kept pieces only
                covered = {p.src_row + r for p in pcs for r in range(p.rows)}
                pcs = [p for p in pcs if all(p.src_row + r in covered for r in range(p.rows))]
                pcs += [_lib.SrPiece(_lib.SR_PIECE_COPY, 0, 0, 0, -1, 0, 1, COLS, r, 0, r, 0)
                        for r in range(rows) if r not in covered]
                t = (_lib.SrTensor * 1)(_lib.SrTensor(rows, COLS, _lib.SR_DT_U8, 0))
                arr = (_lib.SrPiece * len(pcs))(*pcs)
                h = ctypes.c_void_p()
                _lib.check(L.sr_plan_create(t, 1, t, 1, N_PEERS, arr, len(pcs), None, ctypes.byref(h)), "create")
                src_h = torch.randint(0, 256, (rows, COLS), dtype=torch.uint8, generator=gen)
                with torch.cuda.stream(stream):
                    src = src_h.cuda()
                    dst = torch.full((rows, COLS), POISON, dtype=torch.uint8, device="cuda")
                    _lib.check(L.sr_gather(h, _vp([src.data_ptr()]), _vp([dst.data_ptr()]), stream.cuda_stream),
                               "gather")
                L.sr_plan_destroy(h)
                stream.synchronize()
                if not torch.equal(dst.cpu(), src_h):
                    errors.append((tid, it, rows))
        except Exception as e:   # reported below with the thread and iteration
            errors.append((tid, repr(e)))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors

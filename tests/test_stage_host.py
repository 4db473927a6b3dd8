"""The host half of staging (sr_pack_host) and the host-memory route's
checks, on the CPU.

``sr_pack_host`` copies every piece's source region from host memory into
host peer buffers with the library's host threads, window by window; the
bytes must be those of the plan's layout (``sr_plan_piece_offset``) packed
with numpy, and unpacking them with numpy must give the oracle's shards.
``sr_stage_pack`` runs the same filling code into pinned windows on the GPU
(tests/test_gpu_host_sources.py).
"""
import ctypes

import numpy as np
import pytest
import torch

from suika_amd import _lib, execute_param_transfer
from suika_amd.meta import TensorMeta, TransferOp
from suika_amd.plan import ReshardPlan
from tests import cases
from tests.harness import (global_state, index_state, np2t, oracle_dest, payload_spans, simulate_pack,
                           simulate_unpack, source_shards)

SMALL = cases.all_small_cases()


def _esize(code):
    return {_lib.SR_DT_U8: 1, _lib.SR_DT_BF16: 2, _lib.SR_DT_F16: 2, _lib.SR_DT_F32: 4,
            _lib.SR_DT_F64: 8, _lib.SR_DT_I32: 4, _lib.SR_DT_I64: 8}[code]


def _host_sources(w, srcs):
    dt = w.dtypes
    return {r: {n: {f: np2t(a, dt[f]) for f, a in e.items()} for n, e in sd.items()} for r, sd in srcs.items()}


def _plan(ops, fake, fields, recast=None):
    return ReshardPlan.from_sources(ops, lambda r: fake[r], fields, torch.device("cuda", 0), recast=recast,
                                    rank=0, host_ok=True)


def _pack_host(plan, src_ptrs, skip=()):
    bufs = [np.full(max(1, n), 0xCD, dtype=np.uint8) for n in plan.peer_bytes]
    ptrs = [0 if i in skip else b.ctypes.data for i, b in enumerate(bufs)]
    plan.pack_host_ptrs(np.asarray(src_ptrs, dtype=np.uint64), ptrs)
    return bufs


def _check_payloads(plan, got, want, skip=()):
    n = 0
    for peer, off, nbytes in payload_spans(plan, _esize):
        if peer in skip:
            assert (got[peer][off:off + nbytes] == 0xCD).all(), "a skipped peer's buffer was written"
            continue
        np.testing.assert_array_equal(got[peer][off:off + nbytes], want[peer][off:off + nbytes],
                                      err_msg=f"peer {peer} payload at {off}")
        n += nbytes
    return n


@pytest.mark.parametrize("w", SMALL, ids=[w.key for w in SMALL])
@pytest.mark.parametrize("payload", ["seeded", "index"])
def test_pack_host_matches_layout_and_oracle(w, payload):
    spl, _ = w.layouts()
    names = {n for metas in spl.layout.values() for n in metas}
    glob = (global_state if payload == "seeded" else index_state)(w, names)
    srcs = source_shards(w, sorted(spl.layout), glob)
    fake = _host_sources(w, srcs)
    plan, src_ptrs = _plan(w.ops(), fake, [f for f in w.src_fields], recast=w.recast_map)
    try:
        got = _pack_host(plan, src_ptrs)
        _check_payloads(plan, got, simulate_pack(plan, srcs, _esize))
        out = simulate_unpack(plan, got, _esize)
        want = oracle_dest(w, srcs)
        for (name, f), arr in out.items():
            np.testing.assert_array_equal(arr, want[name][f], err_msg=f"{name}/{f}")
    finally:
        plan.close()


def _wide_ops():
    """88 MB of pieces, more than the pinned window ring holds: a dim -1
    split (one run per row), a dim 0 split (one contiguous range) and a
    replicated tensor, from two source ranks."""
    ops = []
    col = TensorMeta(name="row", dtype=torch.float32, shape=(2048, 8192), tp_meta=(-1, 0, 1))
    for r in (0, 1):
        src = TensorMeta(name="row", dtype=torch.float32, shape=(2048, 8192), tp_meta=(-1, r, 2))
        piece = TensorMeta(name="row", dtype=torch.float32, shape=(2048, 8192), tp_meta=(-1, r, 2))
        ops.append(TransferOp("row", r, 0, src, piece, dst_shard_meta=col))
    row = TensorMeta(name="col", dtype=torch.bfloat16, shape=(6000, 2000), tp_meta=(0, 0, 1))
    for r in (0, 1):
        src = TensorMeta(name="col", dtype=torch.bfloat16, shape=(6000, 2000), tp_meta=(0, r, 2))
        ops.append(TransferOp("col", r, 0, src, src, dst_shard_meta=row))
    rep = TensorMeta(name="rep", dtype=torch.float32, shape=(777,))
    ops.append(TransferOp("rep", 1, 0, rep, rep))
    return ops


def _wide_sources(seed=5):
    g = torch.Generator().manual_seed(seed)
    fake = {}
    for r in (0, 1):
        fake[r] = {"row": {"param": torch.randn(2048, 4096, generator=g)},
                   "col": {"param": torch.randn(3000, 2000, generator=g).to(torch.bfloat16)},
                   "rep": {"param": torch.randn(777, generator=g)}}
    return fake


@pytest.mark.parametrize("threads", [1, 3, 16])
def test_pack_host_splits_windows_over_threads(threads):
    """Window tasks start and end inside rows and inside pieces; every
    thread count gives the same bytes, and a null buffer skips its peer."""
    fake = _wide_sources()
    srcs = {r: {n: {f: t.view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32).numpy()
                    for f, t in e.items()} for n, e in sd.items()} for r, sd in fake.items()}
    L = _lib.lib()
    assert L.sr_set_host_threads(threads) == _lib.SR_OK
    try:
        plan, src_ptrs = _plan(_wide_ops(), fake, ["param"])
        try:
            want = simulate_pack(plan, srcs, _esize)
            assert _check_payloads(plan, _pack_host(plan, src_ptrs), want) == \
                2 * (2048 * 4096 * 4 + 3000 * 2000 * 2) + 777 * 4
            skip = (plan.peers.index(1),)
            _check_payloads(plan, _pack_host(plan, src_ptrs, skip=skip), want, skip=skip)
        finally:
            plan.close()
    finally:
        assert L.sr_set_host_threads(0) == _lib.SR_OK


def test_pack_host_rejects_bad_pointers():
    fake = _wide_sources()
    plan, src_ptrs = _plan(_wide_ops(), fake, ["param"])
    L = _lib.lib()
    try:
        bufs = [np.zeros(n + 16, dtype=np.uint8) for n in plan.peer_bytes]
        ptrs = [b.ctypes.data for b in bufs]
        bad = np.asarray(src_ptrs, dtype=np.uint64).copy()
        bad[0] = 0
        with pytest.raises(AssertionError, match=r"sr_pack_host: SR_EINVAL: src_ptrs\[0\] is null"):
            plan.pack_host_ptrs(bad, ptrs)
        odd = [p + (1 if i == 0 else 0) for i, p in enumerate(ptrs)]
        with pytest.raises(AssertionError, match="SR_EALIGN"):
            plan.pack_host_ptrs(np.asarray(src_ptrs, dtype=np.uint64), odd)
        assert L.sr_pack_host(None, None, None) == _lib.SR_EINVAL
    finally:
        plan.close()
    assert L.sr_set_host_threads(-1) == _lib.SR_EINVAL
    assert L.sr_set_host_threads(257) == _lib.SR_EINVAL
    c = _lib.stage_counters()
    assert c.host_bytes_up >= c.host_piece_bytes


def test_host_sources_fail_loudly_without_gpu():
    """No CPU reshard: a host result, and host sources, need the GPU."""
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    fake = _wide_sources()
    with pytest.raises(RuntimeError, match="no GPU is available"):
        execute_param_transfer(_wide_ops(), {}, "cpu", [("param", "normal")], rank=0,
                               fake_source_state_dicts=fake)
    with pytest.raises(AssertionError, match="GPU or in host memory"):
        execute_param_transfer(_wide_ops(), {}, "meta", [("param", "normal")], rank=0,
                               fake_source_state_dicts=fake)


def test_download_argument_checks():
    L = _lib.lib()
    assert L.sr_download(None, None, None, 0, None) == _lib.SR_OK
    assert L.sr_download(None, None, None, -1, None) == _lib.SR_EINVAL
    assert L.sr_download(None, None, None, 2, None) == _lib.SR_EINVAL
    zero = (ctypes.c_uint64 * 1)(0)
    nul = (ctypes.c_void_p * 1)(None)
    assert L.sr_download(nul, nul, zero, 1, None) == _lib.SR_OK   # nothing to copy: no device needed


def test_stage_groups_cut_whole_tensors_by_bytes():
    from suika_amd.migration import STAGE_GROUP_MAX, STAGE_GROUP_MIN, _stage_groups
    assert [g.tolist() for g in _stage_groups(np.zeros(0, dtype=np.int64))] == [[]]
    small = np.full(10, 1 << 20, dtype=np.int64)          # 10 MiB in all: one group
    assert [g.tolist() for g in _stage_groups(small)] == [list(range(10))]
    big = np.full(64, 256 << 20, dtype=np.int64)           # 16 GiB: groups of 1 GiB (4 tensors)
    groups = _stage_groups(big)
    assert all(len(g) == 4 for g in groups) and len(groups) == 16
    mixed = np.array([3 << 30, 1, 1, 40 << 20, 1 << 20, 1 << 20], dtype=np.int64)
    groups = _stage_groups(mixed)
    assert np.concatenate(groups).tolist() == list(range(6))   # every tensor once, in order
    assert groups[0].tolist() == [0]                            # a tensor above the bound stands alone
    total = int(mixed.sum())
    target = max(STAGE_GROUP_MIN, min(STAGE_GROUP_MAX, total // 16))
    for g in groups[:-1]:
        assert mixed[g].sum() >= target

"""The library's transfer scheduler (``sr_schedule``, include/suika_planner.h)
behind ``schedule_param_transfer``, checked on the CPU against the oracle's
restatement of the reference schedule (Suika/migration.py:322-381):

* randomised layouts (every shard kind, TP/PP/DP on both sides, uneven
  stages), whole schedules for every destination rank, both peer-reuse modes;
* layout dict orders the reference iterates (rank order, tensor order), a
  source rank holding no tensor, ties between equally loaded owners;
* the reference's error behaviour (no owner, slice-dim mismatch, an empty
  source layout) and the raw C call's table-size contract.

The committed reference schedules (tests/golden/schedule_vectors.json.gz) are
checked in tests/test_golden.py.
"""
import ctypes
import random

import numpy as np
import pytest
import torch

from oracle import reshard_oracle as O
from suika_amd import ParamLayout, TensorMeta, _lib, schedule_param_transfer
from suika_amd.meta import _encode_layout
from tests.harness import to_olayout
from tests.test_fuzz import random_case


def _sig(op):
    m = op.dst_meta
    return (op.param_name, op.src_rank, op.dst_rank, tuple(m.tp_meta) if m.tp_meta else None, m.rows)


def _osig(o):
    m = o.dst_meta
    return (o.name, o.src, o.dst, tuple(m.tp) if m.tp else None, m.rows)


def _same_as_oracle(spl, tpl, min_peers):
    ours = schedule_param_transfer(spl, tpl, minimum_est_peers=min_peers)
    ref = O.schedule(to_olayout(spl), to_olayout(tpl), minimum_est_peers=min_peers)
    assert [_sig(op) for op in ours] == [_osig(o) for o in ref]
    # the ops read the layouts' own metas
    for op in ours:
        assert op.src_meta is spl.layout[op.src_rank][op.param_name]
        assert op.dst_shard_meta is tpl.layout[op.dst_rank][op.param_name]
    return ours


@pytest.mark.parametrize("min_peers", [1, 2])
@pytest.mark.parametrize("seed", range(0, 200, 2))
def test_fuzz_schedule_matches_oracle(seed, min_peers):
    w = random_case(seed + min_peers - 1)
    spl, tpl = w.layouts()
    _same_as_oracle(spl, tpl, min_peers)


def _shuffled(pl: ParamLayout, rng: random.Random) -> ParamLayout:
    ranks = list(pl.layout)
    rng.shuffle(ranks)
    out = ParamLayout()
    for r in ranks:
        items = list(pl.layout[r].items())
        rng.shuffle(items)
        out.layout[r] = dict(items)
    return out


@pytest.mark.parametrize("seed", range(20))
def test_dict_orders_are_followed(seed):
    """Owners are tried in the layout's rank order and targets are visited in
    its dict order, whatever those orders are."""
    rng = random.Random(1000 + seed)
    w = random_case(seed)
    spl, tpl = w.layouts()
    _same_as_oracle(_shuffled(spl, rng), _shuffled(tpl, rng), rng.choice([1, 2]))


def _m(name, shape, tp=None, dtype=torch.float32, **kw):
    return TensorMeta(name=name, dtype=dtype, shape=shape, tp_meta=tp, **kw)


def test_source_rank_without_tensors():
    """A source rank holding nothing still counts in the load vector."""
    spl = ParamLayout.from_metas({0: {}, 1: {"a": _m("a", (8, 4), (0, 0, 2))},
                                  2: {"a": _m("a", (8, 4), (0, 1, 2))}})
    tpl = ParamLayout.from_metas({5: {"a": _m("a", (8, 4), (0, 0, 1))}})
    ops = _same_as_oracle(spl, tpl, 1)
    assert [(op.src_rank, op.dst_meta.tp_meta) for op in ops] == [(1, (0, 0, 2)), (2, (0, 1, 2))]


def test_ties_go_to_the_first_owner_in_rank_order():
    """Equal loads: the first owner in the layout's rank order wins, as
    Python's min does."""
    rep = {r: {"w": _m("w", (4, 4))} for r in (3, 1, 0, 2)}
    spl = ParamLayout()
    spl.layout = rep
    tpl = ParamLayout.from_metas({9: {"w": _m("w", (4, 4))}, 8: {"w": _m("w", (4, 4))}})
    ops = _same_as_oracle(spl, tpl, 1)
    assert [op.src_rank for op in ops] == [3, 1]


def test_vocab_pieces_and_padding_only_shards():
    """vocab_pad targets are cut at source shard boundaries; a shard of
    padding only is one empty piece."""
    V, H = 10, 4
    def vp(idx, deg):
        return _m("e", (V, H), (0, idx, deg), kind="vocab_pad", kind_args=(4,))
    spl = ParamLayout.from_metas({r: {"e": vp(r, 3)} for r in range(3)})
    tpl = ParamLayout.from_metas({r: {"e": vp(r, 4)} for r in range(4)})
    ops = _same_as_oracle(spl, tpl, 2)
    rows = [(op.dst_rank, op.dst_meta.rows) for op in ops]
    # padded to 12 rows at degree 3 (4 per rank) and 16 at degree 4: rank 3
    # of the target holds rows [12, 16), all padding
    assert rows == [(0, (0, 4)), (1, (4, 8)), (2, (8, 10)), (3, (12, 12))]


def test_log_func_names_remote_pieces():
    spl = ParamLayout.from_metas({0: {"a": _m("a", (4, 4), (0, 0, 2))}, 1: {"a": _m("a", (4, 4), (0, 1, 2))}})
    tpl = ParamLayout.from_metas({0: {"a": _m("a", (4, 4), (0, 0, 1))}})
    lines = []
    schedule_param_transfer(spl, tpl, log_func=lines.append)
    assert lines == ["schedule_param_transfer: 1 > 0 transfer a"]


def test_missing_owner_names_the_tensor():
    spl = ParamLayout.from_metas({0: {"a": _m("a", (4, 4), (0, 0, 2))}})
    tpl = ParamLayout.from_metas({0: {"a": _m("a", (4, 4), (0, 1, 2))}})
    with pytest.raises(AssertionError, match=r"illegal transfer, target param a .*not present in any source"):
        schedule_param_transfer(spl, tpl)


def test_slice_dim_mismatch_is_an_assertion():
    spl = ParamLayout.from_metas({0: {"a": _m("a", (4, 4), (0, 0, 2))}, 1: {"a": _m("a", (4, 4), (0, 1, 2))}})
    tpl = ParamLayout.from_metas({0: {"a": _m("a", (4, 4), (-1, 0, 2))}})
    with pytest.raises(AssertionError, match="slice dim mismatch 0 vs -1"):
        schedule_param_transfer(spl, tpl)
    with pytest.raises(AssertionError, match="slice dim mismatch"):
        O.schedule(to_olayout(spl), to_olayout(tpl))


def test_empty_source_layout_raises_like_the_reference():
    tpl = ParamLayout.from_metas({0: {"a": _m("a", (4, 4))}})
    with pytest.raises(ValueError):
        schedule_param_transfer(ParamLayout.from_metas({0: {}}), tpl)


def test_raw_call_reports_the_needed_table_size():
    """Too small an op table: SR_EINVAL, nothing trusted, *n_ops = the
    schedule's length so the caller can retry."""
    spl = ParamLayout.from_metas({0: {"a": _m("a", (8, 4), (0, 0, 2))}, 1: {"a": _m("a", (8, 4), (0, 1, 2))}})
    tpl = ParamLayout.from_metas({0: {"a": _m("a", (8, 4), (0, 0, 1))}, 1: {"a": _m("a", (8, 4), (0, 0, 1))}})
    names = {}
    src = _encode_layout(spl, names, [])
    dst = _encode_layout(tpl, names, [])
    L = _lib.lib()
    n = ctypes.c_int64(-1)
    ops = np.zeros((3, _lib.SR_OP_WORDS), dtype=np.int64)
    rc = L.sr_schedule(_lib.as_int64_ptr(src), len(src), 2, _lib.as_int64_ptr(dst), len(dst), len(names), 1,
                       _lib.as_int64_ptr(ops), 3, ctypes.byref(n))
    assert rc == _lib.SR_EINVAL and n.value == 4 and "do not fit" in _lib.last_error()
    ops = np.zeros((4, _lib.SR_OP_WORDS), dtype=np.int64)
    rc = L.sr_schedule(_lib.as_int64_ptr(src), len(src), 2, _lib.as_int64_ptr(dst), len(dst), len(names), 1,
                       _lib.as_int64_ptr(ops), 4, ctypes.byref(n))
    assert rc == _lib.SR_OK and n.value == 4
    # (name, src_rank, dst_rank, src_meta row, dst_shard row, piece index, piece deg, rows)
    assert ops.tolist() == [[0, 0, 0, 0, 0, 0, 2, -1, -1], [0, 1, 0, 1, 0, 1, 2, -1, -1],
                            [0, 0, 1, 0, 1, 0, 2, -1, -1], [0, 1, 1, 1, 1, 1, 2, -1, -1]]


@pytest.mark.parametrize("bad, match", [
    ({"rank": 7}, "source rank 7 outside"),
    ({"name": 5}, "name id 5 outside"),
    ({"ndim": 9}, "ndim 9 outside"),
    ({"kind": 3}, "unknown shard kind"),
    ({"slice_dim": 2}, "slice_dim 2 of a 2-D tensor"),
    ({"row0": 3}, "row interval"),
    ({"tp_deg": 1 << 40}, "degree at most 65536"),
])
def test_malformed_tables_are_rejected(bad, match):
    spl = ParamLayout.from_metas({0: {"a": _m("a", (8, 4), (0, 0, 2))}, 1: {"a": _m("a", (8, 4), (0, 1, 2))}})
    tpl = ParamLayout.from_metas({0: {"a": _m("a", (8, 4), (0, 0, 1))}})
    names = {}
    src = _encode_layout(spl, names, [])
    dst = _encode_layout(tpl, names, [])
    col = {"rank": 0, "name": 1, "ndim": 3, "slice_dim": 12, "tp_deg": 14, "kind": 15, "row0": 19}
    src[1, col[next(iter(bad))]] = next(iter(bad.values()))
    L = _lib.lib()
    n = ctypes.c_int64()
    ops = np.zeros((8, _lib.SR_OP_WORDS), dtype=np.int64)
    rc = L.sr_schedule(_lib.as_int64_ptr(src), len(src), 2, _lib.as_int64_ptr(dst), len(dst), len(names), 1,
                       _lib.as_int64_ptr(ops), 8, ctypes.byref(n))
    assert rc == _lib.SR_EINVAL
    assert match in _lib.last_error()


def _corrupt(table, rng, n_cells):
    t = table.copy()
    for _ in range(n_cells):
        i = rng.randrange(t.shape[0])
        j = rng.randrange(t.shape[1])
        t[i, j] = rng.choice([-(1 << 62), -7, -1, 0, 1, 2, 3, 9, 1 << 20, 1 << 62, int(t[i, j]) + 1])
    return t


@pytest.mark.parametrize("seed", range(120))
def test_planner_rejects_corrupted_tables_without_crashing(seed):
    """Random cells of valid sr_meta / sr_op / sr_src_spec tables replaced by
    extreme or off-by-one values: sr_schedule and sr_lower return a status
    (and the tables they accept still lower), never crash or read outside the
    tables."""
    rng = random.Random(seed)
    w = random_case(seed)
    spl, tpl = w.layouts()
    names = {}
    src = _encode_layout(spl, names, [])
    dst = _encode_layout(tpl, names, [])
    L = _lib.lib()
    n = ctypes.c_int64()
    cap = 4 * len(dst) * 16
    ops = np.zeros((cap, _lib.SR_OP_WORDS), dtype=np.int64)
    for trial in range(10):
        s2 = _corrupt(src, rng, rng.randint(1, 3))
        d2 = _corrupt(dst, rng, rng.randint(0, 2))
        rc = L.sr_schedule(_lib.as_int64_ptr(s2), len(s2), len(spl.layout), _lib.as_int64_ptr(d2), len(d2),
                           len(names), 1, _lib.as_int64_ptr(ops), cap, ctypes.byref(n))
        assert rc in (_lib.SR_OK, _lib.SR_EINVAL, _lib.SR_ENOMEM)
    # lower one rank's valid schedule with corrupted ops / specs
    rc = L.sr_schedule(_lib.as_int64_ptr(src), len(src), len(spl.layout), _lib.as_int64_ptr(dst), len(dst),
                       len(names), 1, _lib.as_int64_ptr(ops), cap, ctypes.byref(n))
    assert rc == _lib.SR_OK
    sched = ops[:n.value].copy()
    sched = sched[sched[:, 2] == sched[0, 2]]
    metas = np.concatenate([src, dst])
    sched[:, 4] += len(src)
    nf = 2
    specs = np.zeros((len(sched) * nf, _lib.SR_SPEC_WORDS), dtype=np.int64)
    for k, row in enumerate(sched):
        m = src[row[3]]
        nd = int(m[3])
        shape = m[4:4 + nd].copy()
        if m[14] > 0 and m[15] == 0:
            d = int(m[12]) % nd
            shape[d] //= m[14]
        for f in range(nf):
            specs[k * nf + f, :2] = (_lib.SR_DT_F32, nd)
            specs[k * nf + f, 2:2 + nd] = shape
    recast = np.array([0, 0], dtype=np.int64)
    low = ctypes.POINTER(_lib.SrLowering)()
    for trial in range(10):
        o2 = _corrupt(sched, rng, rng.randint(1, 3))
        m2 = _corrupt(metas, rng, rng.randint(0, 2))
        s2 = _corrupt(specs, rng, rng.randint(0, 2))
        rc = L.sr_lower(_lib.as_int64_ptr(m2), len(m2), _lib.as_int64_ptr(o2), len(o2), _lib.as_int64_ptr(s2),
                        nf, _lib.as_int64_ptr(recast), ctypes.byref(low))
        assert rc in (_lib.SR_OK, _lib.SR_EINVAL, _lib.SR_ENOMEM), rc
        if rc == _lib.SR_OK:
            lw = low.contents
            h = ctypes.c_void_p()
            rc2 = L.sr_plan_create(lw.src, lw.n_src, lw.dst, lw.n_dst, lw.n_peers, lw.pieces, lw.n_pieces, None,
                                   ctypes.byref(h))
            assert rc2 <= 0
            L.sr_plan_destroy(h)
            L.sr_lowering_destroy(low)


def test_qkv_rows_must_match_heads():
    """A qkv_heads row whose rows are not (n_q + 2 n_kv) * head_dim is
    rejected, as TensorMeta's constructor does for Python callers."""
    m = _m("qkv", (24, 5), (0, 0, 2), kind="qkv_heads", kind_args=(4, 2, 3))
    names = {}
    spl = ParamLayout.from_metas({0: {"qkv": m}})
    src = _encode_layout(spl, names, [])
    dst = src.copy()
    src[0, 16] = 5            # n_q 5: (5 + 4) * 3 = 27 rows, not 24
    L = _lib.lib()
    n = ctypes.c_int64()
    ops = np.zeros((8, _lib.SR_OP_WORDS), dtype=np.int64)
    rc = L.sr_schedule(_lib.as_int64_ptr(src), 1, 1, _lib.as_int64_ptr(dst), 1, 1, 1, _lib.as_int64_ptr(ops), 8,
                       ctypes.byref(n))
    assert rc == _lib.SR_EINVAL and "qkv_heads rows 24" in _lib.last_error()

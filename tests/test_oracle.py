"""Pins of the CPU oracle (oracle/reshard_oracle.py) before it is trusted.

* chunk / cat against torch.chunk / torch.cat, the library routines the
  reference calls (Suika/migration.py:310, 536);
* bf16 rounding against torch's CPU conversion, special values included;
* shard_index against a brute-force per-element map;
* the oracle's reshard (schedule + fake-source execute) against the closed
  form ``shard_of(G, destination)`` on seeded and index-coded state, for every
  small case -- so a wrong piece order, index or ownership fails here;
* the reference's deferred-self-transfer order (hazard H1) is shown to differ
  from the closed form, which is why the build follows ascending order.
"""
import numpy as np
import pytest
import torch

from oracle import reshard_oracle as O
from tests import cases
from tests.harness import (expected_dest, global_state, index_state, oracle_dest, source_shards,
                           t2np)

SMALL = cases.all_small_cases()


@pytest.mark.parametrize("n,chunks", [(12, 4), (12, 5), (7, 3), (5, 8), (1, 2), (16, 16), (13, 1)])
@pytest.mark.parametrize("axis", [0, 1])
def test_chunk_matches_torch(n, chunks, axis):
    shape = (n, 3) if axis == 0 else (3, n)
    a = np.arange(np.prod(shape), dtype=np.int64).reshape(shape)
    ours = O.chunk(a, chunks, axis)
    ref = torch.from_numpy(a).chunk(chunks, dim=axis)
    assert len(ours) == len(ref)
    for x, y in zip(ours, ref):
        np.testing.assert_array_equal(x, y.numpy())


def test_cat_matches_torch():
    parts = [np.arange(6).reshape(2, 3) + 10 * i for i in range(3)]
    for axis in (0, 1, -1):
        np.testing.assert_array_equal(O.cat(parts, axis),
                                      torch.cat([torch.from_numpy(p) for p in parts], axis).numpy())


def test_rne_matches_torch_special_values():
    specials = np.array([0x00000000, 0x80000000, 0x3F800000, 0x3F808000, 0x3F818000, 0x3F80FFFF,
                         0x3F7F8000, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F800000, 0xFF800000, 0x7FC00000,
                         0xFFC00001, 0x7F800001, 0x00000001, 0x00008000, 0x00018000, 0x807FFFFF,
                         0x7F7F8000, 0x7F7F7FFF], dtype=np.uint32)
    ref = torch.from_numpy(specials.view(np.float32)).to(torch.bfloat16)
    ref_bits = t2np(ref)
    ours = O.rne_bf16(specials)
    finite = ~np.isnan(specials.view(np.float32))
    np.testing.assert_array_equal(ours[finite], ref_bits[finite])
    # NaN: torch's element conversion (a strided tensor) gives the quiet NaN
    # 0x7FC0 for every sign and payload, and so does the oracle; torch's
    # vectorised loop over a contiguous tensor gives 0xFFFF, also a quiet NaN
    assert np.all(np.isnan(ref.float().numpy()[~finite]))
    assert np.all(ours[~finite] == 0x7FC0)
    flat = torch.from_numpy(specials.view(np.float32).copy())
    elementwise = t2np(torch.stack([flat, flat], 1)[:, 0].to(torch.bfloat16))
    np.testing.assert_array_equal(ours, elementwise)


def test_rne_matches_torch_random():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=200_000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    # every pattern, NaNs included, against torch's element conversion
    flat = torch.from_numpy(f.copy())
    np.testing.assert_array_equal(O.rne_bf16(bits), t2np(torch.stack([flat, flat], 1)[:, 0].to(torch.bfloat16)))
    keep = ~np.isnan(f)
    ref = t2np(torch.from_numpy(f[keep].copy()).to(torch.bfloat16))
    np.testing.assert_array_equal(O.rne_bf16(bits[keep]), ref)
    # ties: low half exactly 0x8000 rounds to even
    ties = (rng.integers(0, 2 ** 15, size=5000).astype(np.uint32) << 16) | 0x8000
    ties = ties[~np.isnan(ties.view(np.float32))]
    ref = t2np(torch.from_numpy(ties.view(np.float32).copy()).to(torch.bfloat16))
    np.testing.assert_array_equal(O.rne_bf16(ties), ref)


@pytest.mark.parametrize("kind,shape,tp,args", [
    ("chunk", (8, 6), (0, 1, 4), ()),
    ("chunk", (8, 6), (-1, 2, 3), ()),
    ("chunk", (12,), (0, 3, 4), ()),
    ("qkv_heads", (24, 5), (0, 1, 2), (4, 2, 3)),
    ("vocab_pad", (10, 3), (0, 1, 2), (4,)),
    ("vocab_pad", (10, 3), (0, 2, 4), (2,)),
])
def test_shard_index_brute_force(kind, shape, tp, args):
    m = O.OMeta("t", 4, shape, tp, kind, args)
    got = O.shard_index(m)
    flat = np.arange(int(np.prod(shape))).reshape(shape)
    sd, idx, deg = tp
    # brute force: enumerate every global element and decide where it lives
    want = {}
    if kind == "chunk":
        d = sd % len(shape)
        n = shape[d] // deg
        for pos in np.ndindex(*shape):
            if idx * n <= pos[d] < (idx + 1) * n:
                lpos = list(pos)
                lpos[d] -= idx * n
                want[tuple(lpos)] = flat[pos]
    elif kind == "qkv_heads":
        nq, nkv, hd = args
        q, kv = nq // deg * hd, nkv // deg * hd
        for pos in np.ndindex(*shape):
            r = pos[0]
            if idx * q <= r < (idx + 1) * q:
                lr = r - idx * q
            elif nq * hd + idx * kv <= r < nq * hd + (idx + 1) * kv:
                lr = q + r - nq * hd - idx * kv
            elif (nq + nkv) * hd + idx * kv <= r < (nq + nkv) * hd + (idx + 1) * kv:
                lr = q + kv + r - (nq + nkv) * hd - idx * kv
            else:
                continue
            want[(lr,) + pos[1:]] = flat[pos]
    else:
        V = shape[0]
        Vp = int(np.ceil(V / (args[0] * deg))) * args[0] * deg
        n = Vp // deg
        for lr in range(n):
            for c in range(shape[1]):
                g = idx * n + lr
                want[(lr, c)] = flat[g, c] if g < V else -1
    assert got.size == len(want)
    for pos, v in want.items():
        assert got[pos] == v, (pos, got[pos], v)


@pytest.mark.parametrize("w", SMALL, ids=[w.key for w in SMALL])
def test_oracle_matches_closed_form_seeded(w):
    glob = global_state(w, _all_names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    got = oracle_dest(w, srcs)
    want = expected_dest(w, glob)
    assert set(got) == set(want)
    for name in want:
        for f in want[name]:
            np.testing.assert_array_equal(got[name][f], want[name][f], err_msg=f"{name}/{f}")


@pytest.mark.parametrize("w", SMALL[::3], ids=[w.key for w in SMALL[::3]])
def test_oracle_matches_closed_form_index_coded(w):
    glob = index_state(w, _all_names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    got = oracle_dest(w, srcs)
    want = expected_dest(w, glob)
    for name in want:
        for f in want[name]:
            np.testing.assert_array_equal(got[name][f], want[name][f], err_msg=f"{name}/{f}")


def test_reference_self_order_hazard():
    """TP4 -> TP2 where the destination rank also holds the leading piece:
    the reference's deferred self transfers put it last (wrong bytes)."""
    w = cases.scaled_configs()["llama7b_tp4pp2_tp2pp2"]
    glob = global_state(w, _all_names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = expected_dest(w, glob)
    good = oracle_dest(w, srcs)
    bad = oracle_dest(w, srcs, self_rank=w.dst_rank)
    name = "h.0.self_attn.q_proj.weight"
    np.testing.assert_array_equal(good[name]["master"], want[name]["master"])
    assert not np.array_equal(bad[name]["master"], want[name]["master"])


def test_oracle_kind_table_matches_inventory():
    """The product inventory assigns the reference's kind to every name."""
    from suika_amd.inventory import COL, QKV, REPL, ROW, VOCAB, rank_params
    from suika_amd.workloads import CONFIGS
    label = {COL: "col", ROW: "row", REPL: "repl", VOCAB: "vocab", QKV: "qkv"}
    for w in list(CONFIGS.values()) + SMALL:
        for rank in range(w.src.world):
            for p in rank_params(w.model, w.src, rank):
                assert label[p.kind] == O.kind_of_name(p.name, w.model.vocab_parallel), p.name


def _all_names(w):
    spl, _ = w.layouts()
    names = set()
    for metas in spl.layout.values():
        names |= set(metas)
    return names

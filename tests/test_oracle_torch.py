"""The torch-CPU restatement timed as the CPU baseline (oracle/torch_ref.py)
equals the numpy oracle on every small case."""
import numpy as np
import pytest

from oracle import reshard_oracle as O
from oracle.torch_ref import execute_torch_cpu
from tests import cases
from tests.harness import global_state, np2t, oracle_dest, source_shards, t2np, to_olayout

SMALL = cases.all_small_cases()


@pytest.mark.parametrize("w", SMALL[::2], ids=[w.key for w in SMALL[::2]])
def test_torch_restatement_matches_oracle(w):
    spl, tpl = w.layouts()
    names = {n for metas in spl.layout.values() for n in metas}
    glob = global_state(w, names)
    srcs = source_shards(w, sorted(spl.layout), glob)
    want = oracle_dest(w, srcs)
    ops = O.schedule(to_olayout(spl), to_olayout(tpl))
    dt = w.dtypes
    tsrc = {r: {n: {f: np2t(a, dt[f]) for f, a in e.items()} for n, e in sd.items()}
            for r, sd in srcs.items()}
    got = execute_torch_cpu(ops, w.dst_rank, tsrc, list(w.src_fields), w.recast_map)
    for name, e in want.items():
        for f, a in e.items():
            np.testing.assert_array_equal(t2np(got[name][f]), a, err_msg=f"{name}/{f}")

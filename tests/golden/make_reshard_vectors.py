#!/usr/bin/env python3
"""Write the committed reshard fixtures: tiny source shards and the expected
destination shards, as raw bit patterns, for every case of
``tests.cases.golden_cases()`` in two payload styles:

* ``seeded``: the seeded state recipe (torch CPU generator, N(0, 0.02) master,
  N(0, 1e-3) exp_avg, |N(0, 1e-6)| exp_avg_sq, bf16 param = RNE(master));
* ``index``:  element bits derived from (tensor, field, global flat index).

Expected outputs come from the closed form ``shard_of(G, destination)`` and
are cross-checked here against both the numpy oracle and the torch-CPU
restatement before anything is written.  Output:
tests/golden/reshard_vectors.npz: ``blob`` (all arrays' bytes) and
``manifest`` (JSON: key -> [byte offset, numpy dtype, shape]); keys are
``payload|case|src|rank|name|field`` and ``payload|case|dst|name|field``.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))


def main() -> int:
    from oracle import reshard_oracle as O
    from oracle.torch_ref import execute_torch_cpu
    from tests import cases
    from tests.harness import (expected_dest, global_state, index_state, np2t, oracle_dest,
                               source_shards, t2np, to_olayout)

    arrays = {}
    for key, w in cases.golden_cases().items():
        spl, tpl = w.layouts()
        names = {n for metas in spl.layout.values() for n in metas}
        for payload, make in (("seeded", global_state), ("index", index_state)):
            glob = make(w, names)
            srcs = source_shards(w, sorted(spl.layout), glob)
            want = expected_dest(w, glob)
            got = oracle_dest(w, srcs)
            ops = O.schedule(to_olayout(spl), to_olayout(tpl))
            dt = w.dtypes
            tsrc = {r: {n: {f: np2t(a, dt[f]) for f, a in e.items()} for n, e in sd.items()}
                    for r, sd in srcs.items()}
            tgot = execute_torch_cpu(ops, w.dst_rank, tsrc, list(w.src_fields), w.recast_map)
            for name, ent in want.items():
                for f, a in ent.items():
                    assert np.array_equal(got[name][f], a), (key, payload, name, f, "oracle")
                    assert np.array_equal(t2np(tgot[name][f]), a), (key, payload, name, f, "torch")
                    arrays[f"{payload}|{key}|dst|{name}|{f}"] = a
            used = {op.src for op in ops if op.dst == w.dst_rank}
            for r in sorted(used):
                for name, ent in srcs[r].items():
                    for f, a in ent.items():
                        arrays[f"{payload}|{key}|src|{r}|{name}|{f}"] = a
    # one byte blob + a JSON manifest (key -> offset, dtype, shape)
    manifest, parts, off = {}, [], 0
    for k in sorted(arrays):
        a = np.ascontiguousarray(arrays[k])
        manifest[k] = [off, a.dtype.str, list(a.shape)]
        parts.append(a.reshape(-1).view(np.uint8))
        off += a.nbytes
    blob = np.concatenate(parts)
    meta = np.frombuffer(json.dumps(manifest, separators=(",", ":")).encode(), dtype=np.uint8)
    dest = Path(__file__).resolve().parent / "reshard_vectors.npz"
    np.savez_compressed(dest, blob=blob, manifest=meta)
    print(f"wrote {dest} ({len(arrays)} arrays, {dest.stat().st_size} bytes)")
    return 0


if __name__ == "__main__":
    sys.exit(main())

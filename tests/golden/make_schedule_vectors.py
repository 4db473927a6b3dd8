#!/usr/bin/env python3
"""Write golden vectors of the reference's ``schedule_param_transfer``.

Runs in the development container only (it reads /root/reference, which the
GPU box does not have).  The greedy choice of a source rank among several
owners (Suika/migration.py:335-379) is the one part of the reshard path that
no closed form pins, so this script imports the reference's own
``Suika/migration.py`` -- registering a bare ``Suika`` package that points at
the reference directory, so that the package ``__init__`` (engines,
schedulers, models) is not imported -- and records, for every case, the op
list it produces: (name, src rank, dst rank, piece tp_meta); for the
full-size workloads only the ops of their destination rank are kept.

Layouts use the reference's kinds only: a vocabulary-parallel ``wte`` is
recorded as replicated (the reference never splits ``nn.Embedding``) and a
fused ``qkv_proj`` as a column-parallel chunk (same nesting).  The output is
tests/golden/schedule_vectors.json.gz; tests/test_golden.py replays the product
and oracle schedules on the same layouts and compares.
"""
from __future__ import annotations

import gzip
import importlib
import json
import os
import sys
import types
from dataclasses import replace
from pathlib import Path

REF = Path("/root/reference")
ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))


def load_reference_migration():
    pkg = types.ModuleType("Suika")
    pkg.__path__ = [str(REF / "Suika")]
    sys.modules["Suika"] = pkg
    return importlib.import_module("Suika.migration")


def reference_kind_workload(w):
    """The same workload with only the reference's shard kinds."""
    return replace(w, model=replace(w.model, vocab_parallel=False, fused_qkv=False))


def main() -> int:
    import torch

    from suika_amd.workloads import CONFIG_ORDER, CONFIGS
    from tests import cases

    mig = load_reference_migration()

    def ref_layout(pl):
        layout = mig.ParamLayout()
        for rank, metas in pl.layout.items():
            d = {}
            for name, m in metas.items():
                rm = mig.TensorMeta(dtype=m.dtype, shape=tuple(m.shape), name=name,
                                    tp_meta=m.tp_meta)
                if m.tp_meta is None:
                    rm.tp_meta = None   # as TensorMeta(tensor) sets it for a plain tensor
                d[name] = rm
            layout.layout[rank] = d
        return layout

    workloads = cases.all_small_cases() + [CONFIGS[k] for k in CONFIG_ORDER]
    names = {}
    out = {"source": "Suika/migration.py schedule_param_transfer (reference, imported)",
           "format": "op = [name id, src rank, dst rank, piece tp_meta]", "names": None,
           "cases": {}}
    for w in workloads:
        wr = reference_kind_workload(w)
        spl, tpl = wr.layouts()
        for ib in ("0", "1"):
            os.environ["NCCL_IB_DISABLE"] = ib
            ops = mig.schedule_param_transfer(ref_layout(spl), ref_layout(tpl))
            if w.key in CONFIGS:
                # full-size plans: this workload's destination rank only (the
                # greedy state still comes from all earlier destination ranks)
                ops = [op for op in ops if op.dst_rank == w.dst_rank]
            out["cases"][f"{w.key}|ib_disable={ib}"] = [
                [names.setdefault(op.param_name, len(names)), op.src_rank, op.dst_rank,
                 list(op.dst_meta.tp_meta) if op.dst_meta.tp_meta is not None else None]
                for op in ops]
    os.environ.pop("NCCL_IB_DISABLE", None)
    out["names"] = sorted(names, key=names.get)
    dest = Path(__file__).resolve().parent / "schedule_vectors.json.gz"
    with gzip.open(dest, "wt") as fh:
        fh.write(json.dumps(out, separators=(",", ":")) + "\n")
    n = sum(len(v) for v in out["cases"].values())
    print(f"wrote {dest} ({len(out['cases'])} cases, {n} ops)")
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Committed golden vectors (tests/golden/):

* schedule_vectors.json.gz -- op lists produced by the reference's own
  ``schedule_param_transfer`` (imported once in the development container by
  tests/golden/make_schedule_vectors.py); the product schedule and the
  oracle's restatement must reproduce every op, source choice included;
* reshard_vectors.npz -- tiny source shards and expected destination shards
  (seeded and index-coded); the oracle and the numpy simulation of the
  product plan must reproduce them bit for bit.
"""
from dataclasses import replace

import numpy as np
import pytest

from oracle import reshard_oracle as O
from suika_amd import schedule_param_transfer
from suika_amd.plan import ReshardPlan, SlotSpec
from suika_amd.workloads import CONFIGS
from tests import cases
from tests.harness import (load_reshard_vectors, load_schedule_vectors, simulate_plan, to_olayout)
from tests.test_plan import _esize

SCHED = load_schedule_vectors()
WORKLOADS = {w.key: w for w in cases.all_small_cases()}
WORKLOADS.update(CONFIGS)
VECTORS = load_reshard_vectors()
GOLDEN = cases.golden_cases()


def _ref_kinds(w):
    return replace(w, model=replace(w.model, vocab_parallel=False, fused_qkv=False))


@pytest.mark.parametrize("case", sorted(SCHED["cases"]))
def test_schedule_matches_reference_vectors(case, monkeypatch):
    key, ib = case.split("|")
    w = _ref_kinds(WORKLOADS[key])
    monkeypatch.setenv("NCCL_IB_DISABLE", ib.split("=")[1])
    names = SCHED["names"]
    want = [(names[n], s, d, tuple(tp) if tp is not None else None) for n, s, d, tp in SCHED["cases"][case]]
    spl, tpl = w.layouts()
    ours = schedule_param_transfer(spl, tpl)
    ref = O.schedule(to_olayout(spl), to_olayout(tpl))
    if key in CONFIGS:
        ours = [op for op in ours if op.dst_rank == w.dst_rank]
        ref = [op for op in ref if op.dst == w.dst_rank]
    got = [(op.param_name, op.src_rank, op.dst_rank,
            tuple(op.dst_meta.tp_meta) if op.dst_meta.tp_meta is not None else None) for op in ours]
    assert got == want
    assert [(o.name, o.src, o.dst, o.dst_meta.tp) for o in ref] == want


@pytest.mark.parametrize("payload", ["seeded", "index"])
@pytest.mark.parametrize("case", sorted(GOLDEN))
def test_oracle_reproduces_reshard_vectors(payload, case):
    w = GOLDEN[case]
    srcs, want = VECTORS[payload][case]
    spl, tpl = w.layouts()
    ops = O.schedule(to_olayout(spl), to_olayout(tpl))
    got = O.execute_fake_source(ops, w.dst_rank, srcs, list(w.src_fields), recast=w.recast_map)
    assert set(got) == set(want)
    for name, ent in want.items():
        for f, a in ent.items():
            np.testing.assert_array_equal(got[name][f], a, err_msg=f"{case}: {name}/{f}")


@pytest.mark.parametrize("payload", ["seeded", "index"])
@pytest.mark.parametrize("case", sorted(GOLDEN))
def test_plan_simulation_reproduces_reshard_vectors(payload, case):
    w = GOLDEN[case]
    srcs, want = VECTORS[payload][case]
    ops = w.ops()
    dt = w.dtypes
    specs = {(op.src_rank, op.param_name, f): SlotSpec(tuple(op.src_meta.actual_shape()), dt[f])
             for op in ops for f in w.src_fields}
    plan = ReshardPlan(ops, specs, list(w.src_fields), recast=w.recast_map)
    got = simulate_plan(plan, srcs, _esize)
    assert {k[0] for k in got} == set(want)
    for (name, f), a in got.items():
        np.testing.assert_array_equal(a, want[name][f], err_msg=f"{case}: {name}/{f}")
    plan.close()

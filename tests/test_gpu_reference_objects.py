"""The drop-in operators on the reference's own plan objects, on the GPU.

``execute_param_transfer`` runs the TransferOps recorded from the reference's
``schedule_param_transfer``, rebuilt as objects with only the reference's
attributes (tests/refshaped.py), on both routes and into a destination
arena; ``schedule_and_execute_param_transfer`` (Suika/migration.py:558-598)
schedules and executes from layouts of such metas and of this build's own,
with the peer shards passed through its keyword arguments.  Every result
must equal the oracle's reshard of the same seeded shards, bit for bit.
"""
import numpy as np
import pytest
import torch

from suika_amd import execute_param_transfer, schedule_and_execute_param_transfer
from tests.harness import (global_state, oracle_dest, poisoned_allocations, source_shards, t2np,
                           to_device)
from tests.refshaped import ref_layout
from tests.test_reference_objects import SMALL_CASES, _ref_ops

pytestmark = pytest.mark.gpu


def _state(w):
    spl, _ = w.layouts()
    glob = global_state(w, {n for metas in spl.layout.values() for n in metas})
    srcs = source_shards(w, sorted(spl.layout), glob)
    return srcs, oracle_dest(w, srcs)


def _compare(case, out, want):
    assert set(out) == set(want), case
    for name, ent in want.items():
        for f, a in ent.items():
            np.testing.assert_array_equal(t2np(out[name][f]), a, err_msg=f"{case}: {name}/{f}")


@pytest.mark.parametrize("route", ["direct", "buffers"])
@pytest.mark.parametrize("case", SMALL_CASES)
def test_execute_reference_ops_matches_oracle(case, route):
    w, _, _, ref_ops = _ref_ops(case, omit_tp=True)
    print(f"[gpu ref objects] {case} route={route}", flush=True)
    srcs, want = _state(w)
    fake = to_device(srcs, w, "cuda")
    with poisoned_allocations() as poisoned:
        out = execute_param_transfer(ref_ops, {}, torch.device("cuda"), [(f, "normal") for f in w.src_fields],
                                     rank=w.dst_rank, fake_source_state_dicts=fake, recast=w.recast_map,
                                     route=route, arena=case == SMALL_CASES[0])
    torch.cuda.synchronize()
    assert poisoned["tensors"] >= sum(len(e) for e in out.values())
    _compare(case, out, want)


@pytest.mark.parametrize("shape", ["reference", "own"])
@pytest.mark.parametrize("case", SMALL_CASES[::4])
def test_schedule_and_execute_matches_oracle(case, shape):
    """Schedule, execute and synchronise in one call; the peer shards and the
    executing rank go through the keyword arguments it passes on."""
    w, rspl, rtpl, _ = _ref_ops(case)
    if shape == "own":
        spl, tpl = w.layouts()
    else:
        spl, tpl = rspl, rtpl
    print(f"[gpu schedule_and_execute] {case} layouts={shape}", flush=True)
    srcs, want = _state(w)
    fake = to_device(srcs, w, "cuda")
    own = dict(fake.get(w.dst_rank, {}))
    ctx = {"expected_sub_fields": [(f, "normal") for f in w.src_fields]}
    with poisoned_allocations():
        out = schedule_and_execute_param_transfer(spl, tpl, own, ctx, torch.device("cuda"), None, None, False,
                                                  rank=w.dst_rank, fake_source_state_dicts=fake,
                                                  recast=w.recast_map)
    assert own == {}, "source_state_dict is cleared in place"
    _compare(case, out, want)


def test_reference_layouts_without_tp_meta_schedule_and_execute():
    """Replicated metas built the reference's way from dtype and shape alone
    carry no tp_meta attribute at all."""
    case = SMALL_CASES[0]
    w, _, _, _ = _ref_ops(case)
    spl, tpl = w.layouts()
    rspl, rtpl = ref_layout(spl, omit_tp=True), ref_layout(tpl, omit_tp=True)
    srcs, want = _state(w)
    fake = to_device(srcs, w, "cuda")
    ctx = {"expected_sub_fields": [(f, "normal") for f in w.src_fields]}
    out = schedule_and_execute_param_transfer(rspl, rtpl, {}, ctx, "cuda", None, None, False,
                                              rank=w.dst_rank, fake_source_state_dicts=fake)
    _compare(case, out, want)

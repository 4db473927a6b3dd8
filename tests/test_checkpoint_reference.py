"""A checkpoint written by the reference's own code, resumed here.

tests/golden/ref_checkpoint_tp2pp2/ was written by
tests/golden/make_reference_checkpoint.py with the reference's ``ParamLayout``,
``TensorMeta`` and ``merge_model_and_optimizer_state_dict``, exactly as its
``checkpoint_save`` writes (Suika/migration.py:1156-1184).  It holds a TP2 x
PP2 world of a small Llama model with seeded parameters and AdamW state.
This build reads its pickled layout and context with
``torch.load(weights_only=True)``: the reference's class paths are allowlisted
to attribute holders, so loading runs none of the file's code.  It then
reshards it on the GPU, bit for bit against the closed form of the same
seeded global tensors.
"""
import shutil
from pathlib import Path

import pytest
import torch

from suika_amd import checkpoint_load
from suika_amd.checkpoint import (ReferenceParamLayout, ReferenceTensorMeta, _context_from_reference,
                                  layout_from_reference, load_reference_object)
from suika_amd.inventory import Parallel, build_layout, build_module
from suika_amd.meta import TensorMeta, schedule_param_transfer
from suika_amd.workloads import shard_global
from tests.golden.make_reference_checkpoint import CONTEXT, SAVE_PAR, global_tensors, ref_model

FIXTURE = Path(__file__).resolve().parent / "golden" / "ref_checkpoint_tp2pp2"


def test_reference_layout_and_context_load_without_running_code():
    raw = load_reference_object(FIXTURE / "param_layout.pt")
    assert type(raw) is ReferenceParamLayout
    assert all(type(m) is ReferenceTensorMeta for metas in raw.layout.values() for m in metas.values())
    layout = layout_from_reference(raw)
    want = build_layout(ref_model(), Parallel(*SAVE_PAR), torch.float32)
    assert list(layout.layout) == list(want.layout)
    for r, metas in want.layout.items():
        assert list(layout.layout[r]) == list(metas), f"rank {r}: names / order"
        for name, m in metas.items():
            got = layout.layout[r][name]
            assert got == m and got.tp_meta == m.tp_meta and got.name == name, name
    ctx = _context_from_reference(load_reference_object(FIXTURE / "other_context.pt"))
    assert ctx["other_context"] == CONTEXT
    fields = dict(ctx["expected_sub_fields"])
    assert list(fields) == ["param", "step", "exp_avg", "exp_avg_sq"]
    assert fields["param"] == "normal" and isinstance(fields["step"], TensorMeta) and fields["step"].numel() == 1
    assert len(ctx["param_groups"]) == 1


def test_plain_weights_only_load_refuses_the_reference_classes():
    """Without the allowlist the safe loader refuses the file: the holders
    are what make it load, and nothing else is allowed."""
    with pytest.raises(Exception, match="Suika.migration"):
        torch.load(FIXTURE / "param_layout.pt", weights_only=True)


def test_reference_state_dicts_hold_the_closed_form_shards():
    glob = global_tensors()
    par = Parallel(*SAVE_PAR)
    metas = build_layout(ref_model(), par, torch.float32).layout
    for r in range(par.world):
        sd = torch.load(FIXTURE / f"state_dict_{r}.pt", weights_only=True)
        assert list(sd) == list(metas[r])
        for name, ent in sd.items():
            assert list(ent) == ["param", "step", "exp_avg", "exp_avg_sq"]
            for f in ("param", "exp_avg", "exp_avg_sq"):
                assert torch.equal(ent[f], shard_global(glob[name][f], metas[r][name])), f"{r} {name}/{f}"
            assert float(ent["step"]) == r + 3


def _check(model, opt, par, rank):
    glob = global_tensors()
    metas = build_layout(ref_model(), par, torch.float32).layout[rank]
    src = layout_from_reference(load_reference_object(FIXTURE / "param_layout.pt"))
    first_src = {}
    for op in schedule_param_transfer(src, build_layout(ref_model(), par, torch.float32)):
        if op.dst_rank == rank:
            first_src.setdefault(op.param_name, op.src_rank)
    state = opt.state_dict()["state"]
    for idx, (name, p) in enumerate(model.named_parameters()):
        assert torch.equal(p.detach().cpu(), shard_global(glob[name]["param"], metas[name])), name
        for f in ("exp_avg", "exp_avg_sq"):
            assert torch.equal(state[idx][f].cpu(), shard_global(glob[name][f], metas[name])), f"{name}/{f}"
        assert float(state[idx]["step"]) == first_src[name] + 3


@pytest.mark.gpu
def test_resume_reference_checkpoint_into_one_rank(tmp_path):
    """TP2 x PP2 (written by the reference) -> TP1: one process holds it all."""
    print("[gpu reference checkpoint] tp1", flush=True)
    ckpt = tmp_path / "ckpt"
    shutil.copytree(FIXTURE, ckpt)
    model = build_module(ref_model(), Parallel(1), 0, torch.float32, "cuda")
    opt, ctx = checkpoint_load(model, lambda: torch.optim.AdamW(model.parameters(), lr=1e-3), str(ckpt))
    assert ctx == CONTEXT
    _check(model, opt, Parallel(1), 0)
    assert not (ckpt / "param_layout.pt").exists(), "rank 0 removes the checkpoint, as the reference does"


def _load_worker(rank, world, port, ckpt, tp, pp):
    import torch.distributed as dist
    dist.init_process_group("gloo", init_method=f"tcp://127.0.0.1:{port}", rank=rank, world_size=world)
    try:
        torch.cuda.set_device(0)
        par = Parallel(tp, pp)
        model = build_module(ref_model(), par, rank, torch.float32, "cuda")
        opt, ctx = checkpoint_load(model, lambda: torch.optim.AdamW(model.parameters(), lr=1e-3), ckpt,
                                   world=dist.group.WORLD)
        assert ctx == CONTEXT
        _check(model, opt, par, rank)
    finally:
        dist.destroy_process_group()


@pytest.mark.gpu
def test_resume_reference_checkpoint_in_a_tp4_world(tmp_path):
    """TP2 x PP2 (written by the reference) -> TP4: four ranks, a gloo world
    of processes sharing the GPU, each checking its own shard."""
    import socket

    import torch.multiprocessing as mp
    print("[gpu reference checkpoint] tp4 world", flush=True)
    ckpt = tmp_path / "ckpt"
    shutil.copytree(FIXTURE, ckpt)
    with socket.socket() as s_:
        s_.bind(("127.0.0.1", 0))
        port = s_.getsockname()[1]
    mp.spawn(_load_worker, args=(4, port, str(ckpt), 4, 1), nprocs=4, join=True)

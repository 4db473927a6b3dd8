#!/usr/bin/env python3
"""Write a checkpoint with the reference's own classes, and check that the
reference reads the checkpoints this build writes.

Runs in the development container only (it reads /root/reference, which the
GPU box does not have).  It imports the reference's ``Suika/migration.py``
through a bare ``Suika`` package (as make_schedule_vectors.py does):

1. A TP2 x PP2 world of a small Llama stage model: each rank's module shard
   (this build's inventory, with the reference's TP attributes), seeded
   parameters and AdamW state (``checkpoint_state``).  The files are written
   exactly as the reference's ``checkpoint_save`` writes them
   (migration.py:1156-1184): ``torch.save`` of the reference's ``ParamLayout``
   of ``TensorMeta(tensor=param)`` objects, of the ``other_context_dict`` that
   the reference's ``merge_model_and_optimizer_state_dict`` returns (its
   ``expected_sub_fields`` hold reference ``TensorMeta`` objects), and of each
   rank's merged state dict.  Output: tests/golden/ref_checkpoint_tp2pp2/.
2. ``suika_amd.checkpoint_save`` writes a one-rank checkpoint into a
   temporary directory. The reference's loader (``torch.load(...,
   weights_only=False)`` with the real ``Suika.migration`` imported, as its
   ``checkpoint_load`` does) must then build its own ``ParamLayout`` and
   ``TensorMeta`` objects from it, with the right attributes, and its
   ``schedule_param_transfer`` must run on them.  The script fails otherwise.

tests/test_checkpoint_reference.py resumes the fixture here (CPU: files and
layouts; GPU: the reshard against the closed form).
"""
from __future__ import annotations

import importlib
import shutil
import sys
import tempfile
import types
from pathlib import Path

import torch

REF = Path("/root/reference")
ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
OUT = Path(__file__).resolve().parent / "ref_checkpoint_tp2pp2"

SEED = 37
SAVE_PAR = (2, 2)      # tp, pp
CONTEXT = {"iteration": 11, "tag": "written by the reference"}


def ref_model():
    from suika_amd.inventory import ModelSpec
    return ModelSpec("llama", n_layer=4, hidden=16, n_head=4, ffn=32, vocab=48)


def global_tensors(seed=SEED):
    """Seeded global tensors of every parameter (torch CPU generator, sorted
    names; param ~ N(0, 0.02), exp_avg ~ N(0, 1e-3), exp_avg_sq = |N(0, 1e-6)|)."""
    from suika_amd.inventory import Parallel, build_layout
    metas = {}
    for ms in build_layout(ref_model(), Parallel(1), torch.float32).layout.values():
        metas.update(ms)
    gen = torch.Generator("cpu").manual_seed(seed)
    out = {}
    for name in sorted(metas):
        shape = tuple(int(s) for s in metas[name].shape)
        out[name] = {"param": torch.randn(shape, generator=gen) * 0.02,
                     "exp_avg": torch.randn(shape, generator=gen) * 1e-3,
                     "exp_avg_sq": (torch.randn(shape, generator=gen) * 1e-6).abs()}
    return out


def checkpoint_state(par, rank: int, glob):
    """Rank ``rank``'s module shard and AdamW state, cut from ``glob`` by this
    build's shard geometry; step = rank + 3."""
    from suika_amd.inventory import build_layout, build_module
    from suika_amd.workloads import shard_global
    mod = build_module(ref_model(), par, rank, torch.float32, "cpu")
    metas = build_layout(ref_model(), par, torch.float32).layout[rank]
    opt = torch.optim.AdamW(mod.parameters(), lr=1e-3)
    for name, p in mod.named_parameters():
        with torch.no_grad():
            p.copy_(shard_global(glob[name]["param"], metas[name]))
        opt.state[p] = {"step": torch.tensor(float(rank + 3)),
                        "exp_avg": shard_global(glob[name]["exp_avg"], metas[name]),
                        "exp_avg_sq": shard_global(glob[name]["exp_avg_sq"], metas[name])}
    return mod, opt


def _reference_migration():
    pkg = types.ModuleType("Suika")
    pkg.__path__ = [str(REF / "Suika")]
    sys.modules["Suika"] = pkg
    return importlib.import_module("Suika.migration")


def main() -> int:
    from suika_amd import checkpoint_save
    from suika_amd.inventory import Parallel
    mig = _reference_migration()

    # 1. the reference writes a TP2 x PP2 checkpoint
    par = Parallel(*SAVE_PAR)
    glob = global_tensors()
    if OUT.exists():
        shutil.rmtree(OUT)
    OUT.mkdir(parents=True)
    layout = mig.ParamLayout()
    for rank in range(par.world):
        mod, opt = checkpoint_state(par, rank, glob)
        layout.layout[rank] = mig.get_param_tensor_meta(mod)
        state_dict, other_context_dict = mig.merge_model_and_optimizer_state_dict(mod, opt, CONTEXT)
        if rank == 0:
            ctx0 = other_context_dict
        torch.save(state_dict, OUT / f"state_dict_{rank}.pt")
    torch.save(layout, OUT / "param_layout.pt")
    torch.save(ctx0, OUT / "other_context.pt")
    total = sum(f.stat().st_size for f in OUT.iterdir())
    print(f"wrote {OUT} ({total} bytes)")

    # 2. the reference reads a checkpoint written by this build
    tmp = Path(tempfile.mkdtemp())
    try:
        mod, opt = checkpoint_state(Parallel(1), 0, glob)
        checkpoint_save(mod, opt, CONTEXT, str(tmp))
        pl = torch.load(tmp / "param_layout.pt", weights_only=False, map_location="cpu")
        ctx = torch.load(tmp / "other_context.pt", weights_only=False, map_location="cpu")
        assert type(pl) is mig.ParamLayout, type(pl)
        metas = pl.layout[0]
        assert list(metas) == [n for n, _ in mod.named_parameters()]
        for name, p in mod.named_parameters():
            m = metas[name]
            want = mig.TensorMeta(tensor=p, name=name)
            assert type(m) is mig.TensorMeta and m == want and m.tp_meta == want.tp_meta and m.name == name, name
        step_meta = dict(ctx["expected_sub_fields"])["step"]
        assert type(step_meta) is mig.TensorMeta and step_meta.numel() == 1
        assert ctx["other_context"] == CONTEXT
        ops = mig.schedule_param_transfer(pl, layout)   # the reference schedules on the loaded layout
        assert len(ops) > 0
        print(f"the reference read this build's checkpoint: {len(metas)} TensorMeta objects of its own "
              f"class, {len(ops)} ops scheduled from them")
    finally:
        shutil.rmtree(tmp)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""checkpoint_save / checkpoint_load (and migration_* with checkpoint_resume),
end to end through the reference-shaped API.

A checkpoint is written by a gloo world of CPU processes, each holding its
rank's module shard (names, TP attributes and AdamW state as a Suika stage
exposes them); it is then loaded under another TP/PP layout and resharded on
the GPU.  Expected values are the oracle's closed-form shards of the seeded
global tensors.
"""
import socket

import numpy as np
import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

from oracle import reshard_oracle as O
from suika_amd import checkpoint_load, checkpoint_save, migration_load, migration_save, schedule_param_transfer
from suika_amd.checkpoint import (layout_from_plain, layout_from_reference, layout_to_plain,
                                  load_reference_object)
from suika_amd.inventory import ModelSpec, Parallel, build_layout, build_module
from tests.harness import t2np, to_ometa

MODEL = ModelSpec("llama", n_layer=4, hidden=32, n_head=4, ffn=64, vocab=100, vocab_parallel=True,
                  pad_multiple=4)
SAVE_PAR = (2, 2)     # tp, pp of the writing world
SEED = 31


def global_tensors(seed=SEED):
    metas = {}
    for ms in build_layout(MODEL, Parallel(1), torch.float32).layout.values():
        metas.update(ms)
    gen = torch.Generator("cpu").manual_seed(seed)
    out = {}
    for name in sorted(metas):
        shape = tuple(int(s) for s in metas[name].shape)
        out[name] = {"param": (torch.randn(shape, generator=gen) * 0.02).numpy(),
                     "exp_avg": (torch.randn(shape, generator=gen) * 1e-3).numpy(),
                     "exp_avg_sq": (torch.randn(shape, generator=gen) * 1e-6).abs().numpy()}
    return out


def rank_state(par: Parallel, rank: int, glob, device="cpu"):
    mod = build_module(MODEL, par, rank, torch.float32, device)
    metas = build_layout(MODEL, par, torch.float32).layout[rank]
    opt = torch.optim.AdamW(mod.parameters(), lr=1e-3)
    for name, p in mod.named_parameters():
        om = to_ometa(metas[name])
        p.data.copy_(torch.from_numpy(np.ascontiguousarray(O.shard_of(glob[name]["param"], om))))
        opt.state[p] = {
            "step": torch.tensor(float(rank + 3)),
            "exp_avg": torch.from_numpy(np.ascontiguousarray(O.shard_of(glob[name]["exp_avg"], om))),
            "exp_avg_sq": torch.from_numpy(np.ascontiguousarray(O.shard_of(glob[name]["exp_avg_sq"], om))),
        }
    return mod, opt


def _save_worker(rank, world, port, ckpt, save_par=SAVE_PAR):
    dist.init_process_group("gloo", init_method=f"tcp://127.0.0.1:{port}", rank=rank, world_size=world)
    try:
        mod, opt = rank_state(Parallel(*save_par), rank, global_tensors())
        checkpoint_save(mod, opt, {"iteration": 7, "tag": "ckpt"}, ckpt)
        dist.barrier()
    finally:
        dist.destroy_process_group()


def _free_port():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def write_checkpoint(ckpt, save_par=SAVE_PAR):
    par = Parallel(*save_par)
    mp.spawn(_save_worker, args=(par.world, _free_port(), str(ckpt), save_par), nprocs=par.world, join=True)


def test_layout_plain_roundtrip():
    pl = build_layout(MODEL, Parallel(2, 2), torch.bfloat16)
    back = layout_from_plain(layout_to_plain(pl))
    assert list(back.layout) == list(pl.layout)
    for r in pl.layout:
        assert list(back.layout[r]) == list(pl.layout[r])
        for n, m in pl.layout[r].items():
            b = back.layout[r][n]
            assert b == m and b.tp_meta == m.tp_meta and tuple(b.actual_shape()) == tuple(m.actual_shape())


def test_checkpoint_save_files(tmp_path):
    """A gloo world of 4 CPU ranks writes the reference's files; every shard
    holds the closed-form slice of the global state."""
    write_checkpoint(tmp_path)
    par = Parallel(*SAVE_PAR)
    layout = layout_from_reference(load_reference_object(tmp_path / "param_layout.pt"))
    want = build_layout(MODEL, par, torch.float32)
    assert layout_to_plain(layout) == layout_to_plain(want)
    ctx = load_reference_object(tmp_path / "other_context.pt")
    assert ctx["other_context"] == {"iteration": 7, "tag": "ckpt"}
    assert [f for f, _ in ctx["expected_sub_fields"]] == ["param", "step", "exp_avg", "exp_avg_sq"]
    glob = global_tensors()
    metas = build_layout(MODEL, par, torch.float32).layout
    for r in range(par.world):
        sd = torch.load(tmp_path / f"state_dict_{r}.pt", weights_only=True)
        assert list(sd) == list(metas[r])
        for name, ent in sd.items():
            om = to_ometa(metas[r][name])
            for f in ("param", "exp_avg", "exp_avg_sq"):
                np.testing.assert_array_equal(ent[f].numpy(), O.shard_of(glob[name][f], om))
            assert float(ent["step"]) == r + 3


def test_migration_api_matches_the_reference_signatures():
    """migration_save / migration_load take the reference's parameters, in
    its order and with its defaults (Suika/migration.py:1357-1366,
    1546-1554); the launcher's placeholder has the reference's keys
    (:1314-1318).  An option of this build's own comes after them,
    keyword-only."""
    import inspect

    from suika_amd import dummy_migration_IPC_state_dict
    save = inspect.signature(migration_save).parameters
    load = inspect.signature(migration_load).parameters
    ref_save = ["IPC_queues", "model", "optimizer", "other_context", "device", "world", "log_func",
                "checkpoint_resume"]
    ref_load = ["IPC_queues", "model", "optimizer", "device", "world", "log_func", "checkpoint_resume"]
    assert list(save) == ref_save + ["handoff_mode", "wave_bytes"]
    assert list(load) == ref_load + ["wait_for_release", "return_before_release"]
    for params, ref in ((save, ref_save), (load, ref_load)):
        for name in list(params)[2:]:
            if name in ref:
                assert params[name].default is None, name
            else:
                assert params[name].kind is inspect.Parameter.KEYWORD_ONLY, name
    assert load["return_before_release"].default is False
    assert dummy_migration_IPC_state_dict == {"source_param_layout": None, "source_state_dict": {},
                                              "other_context_dict": {}}


def _check_loaded(model, opt, par, rank, glob, save_par=SAVE_PAR):
    metas = build_layout(MODEL, par, torch.float32).layout[rank]
    src_layout = build_layout(MODEL, Parallel(*save_par), torch.float32)
    ops = [op for op in schedule_param_transfer(src_layout, build_layout(MODEL, par, torch.float32))
           if op.dst_rank == rank]
    first_src = {}
    for op in ops:
        first_src.setdefault(op.param_name, op.src_rank)
    state = opt.state_dict()["state"]
    for idx, (name, p) in enumerate(model.named_parameters()):
        om = to_ometa(metas[name])
        np.testing.assert_array_equal(t2np(p.data), O.shard_of(glob[name]["param"], om).view(np.uint32),
                                      err_msg=name)
        for f in ("exp_avg", "exp_avg_sq"):
            np.testing.assert_array_equal(t2np(state[idx][f]),
                                          O.shard_of(glob[name][f], om).view(np.uint32), err_msg=f"{name}/{f}")
        assert float(state[idx]["step"]) == first_src[name] + 3


@pytest.mark.gpu
@pytest.mark.parametrize("route", ["direct", "buffers"])
def test_checkpoint_reshard_to_tp1(tmp_path, route):
    """TP2xPP2 checkpoint -> one rank holding everything (stages merged,
    TP shards concatenated, padded vocabulary rows dropped)."""
    print(f"[gpu checkpoint] tp1 route={route}", flush=True)
    write_checkpoint(tmp_path)
    par = Parallel(1)
    model = build_module(MODEL, par, 0, torch.float32, "cuda")
    opt, ctx = checkpoint_load(model, lambda: torch.optim.AdamW(model.parameters(), lr=1e-3),
                               str(tmp_path), route=route)
    assert ctx == {"iteration": 7, "tag": "ckpt"}
    _check_loaded(model, opt, par, 0, global_tensors())
    assert not (tmp_path / "param_layout.pt").exists(), "rank 0 removes the checkpoint"


@pytest.mark.gpu
def test_migration_load_checkpoint_resume_tp4_stage(tmp_path):
    """migration_load(checkpoint_resume=...) into rank 0 of a TP4 layout,
    with an Optimizer instance (not a provider)."""
    print("[gpu checkpoint] migration_load tp4", flush=True)
    write_checkpoint(tmp_path)
    par = Parallel(4)
    model = build_module(MODEL, par, 0, torch.float32, "cuda")
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3)
    ctx = migration_load(None, model, opt, checkpoint_resume=str(tmp_path))
    assert ctx == {"iteration": 7, "tag": "ckpt"}
    _check_loaded(model, opt, par, 0, global_tensors())


@pytest.mark.gpu
def test_checkpoint_tp1_to_tp4_stages_only_piece_bytes(tmp_path):
    """A TP1 checkpoint loaded by rank 0 of TP4: the state files stay in host
    memory (memory-mapped) and only this rank's pieces -- a quarter of every
    split tensor -- go to HBM, which is exactly the new shard's bytes."""
    from suika_amd import _lib
    print("[gpu checkpoint] tp1 -> tp4 staged bytes", flush=True)
    write_checkpoint(tmp_path, save_par=(1, 1))
    par = Parallel(4)
    model = build_module(MODEL, par, 0, torch.float32, "cuda")
    before = _lib.stage_counters()
    opt, ctx = checkpoint_load(model, lambda: torch.optim.AdamW(model.parameters(), lr=1e-3), str(tmp_path))
    after = _lib.stage_counters()
    assert ctx == {"iteration": 7, "tag": "ckpt"}
    _check_loaded(model, opt, par, 0, global_tensors(), save_par=(1, 1))
    shard_bytes = 3 * sum(p.numel() * p.element_size() for p in model.parameters())   # param, exp_avg, exp_avg_sq
    whole_bytes = 3 * sum(int(np.prod(m.shape)) * 4
                          for m in build_layout(MODEL, Parallel(1), torch.float32).layout[0].values())
    assert after.host_piece_bytes - before.host_piece_bytes == shard_bytes
    assert after.device_piece_bytes == before.device_piece_bytes, "no source was on the device"
    staged = after.host_bytes_up - before.host_bytes_up
    assert shard_bytes <= staged <= shard_bytes + 256 * 3 * len(list(model.parameters()))
    assert staged < whole_bytes / 3, (staged, whole_bytes)


@pytest.mark.gpu
def test_checkpoint_missing_returns_fresh_optimizer(tmp_path):
    model = build_module(MODEL, Parallel(1), 0, torch.float32, "cuda")
    opt, ctx = checkpoint_load(model, lambda: torch.optim.AdamW(model.parameters()), str(tmp_path / "none"))
    assert ctx is None and isinstance(opt, torch.optim.AdamW)


def _load_worker(rank, world, port, ckpt, tp, pp):
    # a failure propagates to mp.spawn in the parent with this rank's traceback
    dist.init_process_group("gloo", init_method=f"tcp://127.0.0.1:{port}", rank=rank, world_size=world)
    try:
        torch.cuda.set_device(0)
        par = Parallel(tp, pp)
        model = build_module(MODEL, par, rank, torch.float32, "cuda")
        opt, ctx = checkpoint_load(model, lambda: torch.optim.AdamW(model.parameters(), lr=1e-3), ckpt,
                                   world=dist.group.WORLD)
        assert ctx == {"iteration": 7, "tag": "ckpt"}
        _check_loaded(model, opt, par, rank, global_tensors())
    finally:
        dist.destroy_process_group()


@pytest.mark.gpu
def test_checkpoint_load_two_ranks_share_the_gpu(tmp_path):
    """TP2xPP2 checkpoint -> TP1xPP2, loaded by a gloo world of two ranks that
    share the one GPU: rank 1 (the second stage) resolves its own pieces, the
    layout is all-gathered over gloo, and rank 0 removes the files only after
    both have loaded."""
    print("[gpu checkpoint] two ranks tp1 pp2", flush=True)
    write_checkpoint(tmp_path)
    mp.spawn(_load_worker, args=(2, _free_port(), str(tmp_path), 1, 2), nprocs=2, join=True)
    assert not (tmp_path / "param_layout.pt").exists()

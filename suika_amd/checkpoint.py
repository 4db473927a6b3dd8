"""Checkpoint-resume resharding on the GPU engine.

Same names, arguments, files and control flow as the reference's
``checkpoint_save`` / ``checkpoint_load`` (Suika/migration.py:1156-1305):

* save: every rank writes ``state_dict_{rank}.pt`` (its merged model +
  optimizer state); rank 0 writes ``param_layout.pt`` and
  ``other_context.pt``;
* load: the target layout is gathered from the new model, the transfer is
  scheduled against the saved layout, the shards this rank needs are loaded
  from disk, resharded, split back into model and optimizer state and loaded.

The reference reshards on the CPU (``execute_param_transfer`` with
``device="cpu"``, migration.py:1235-1244); here the source files are
memory-mapped and handed to ``execute_param_transfer`` in host memory, which
sends only the bytes of this rank's pieces to HBM (packed by host threads
into the peer-buffer layout) and unpacks them on the GPU straight into the
new state on ``device``.

The files are the reference's: ``param_layout.pt`` is a pickled
``Suika.migration.ParamLayout`` of ``Suika.migration.TensorMeta`` objects and
``other_context.pt`` holds such metas in ``expected_sub_fields``
(migration.py:1175-1177).  Both are read with ``torch.load(weights_only=True)``:
the two class paths are allowlisted to attribute holders of this module
(``ReferenceParamLayout`` / ``ReferenceTensorMeta``), so loading a file runs
none of its code, and the holders are then turned into this build's
``ParamLayout`` / ``TensorMeta``.  ``checkpoint_save`` writes the same two
class paths, so the reference's ``checkpoint_load`` reads them into its own
classes.  This build's extra shard kinds ride along as ``kind`` /
``kind_args`` attributes, which the reference does not read.  Layout files of
the plain-dict format written by earlier versions of this module are still
read.
"""
from __future__ import annotations

import os
import pickle
import types
from collections import OrderedDict
from typing import Any, Callable, Dict, Optional, Union

import torch
import torch.distributed as dist
from torch.nn import Module
from torch.optim import Optimizer

from .meta import CHUNK, ParamLayout, TensorMeta, schedule_param_transfer
from .migration import (execute_param_transfer, merge_model_and_optimizer_state_dict,
                        split_model_and_optimizer_state_dict)

LAYOUT_FILE = "param_layout.pt"
CONTEXT_FILE = "other_context.pt"


def _dtype_name(dt: torch.dtype) -> str:
    return str(dt).replace("torch.", "")


def meta_to_plain(m: TensorMeta) -> Dict[str, Any]:
    return {"name": m.name, "dtype": _dtype_name(m.dtype), "shape": [int(s) for s in m.shape],
            "tp_meta": None if m.tp_meta is None else [int(v) for v in m.tp_meta],
            "kind": m.kind, "kind_args": [int(v) for v in m.kind_args]}


def meta_from_plain(d: Dict[str, Any]) -> TensorMeta:
    return TensorMeta(name=d["name"], dtype=getattr(torch, d["dtype"]), shape=tuple(d["shape"]),
                      tp_meta=None if d["tp_meta"] is None else tuple(d["tp_meta"]),
                      kind=d["kind"], kind_args=tuple(d["kind_args"]))


def layout_to_plain(pl: ParamLayout) -> Dict[int, Dict[str, Dict[str, Any]]]:
    return {int(r): {n: meta_to_plain(m) for n, m in metas.items()} for r, metas in pl.layout.items()}


def layout_from_plain(d: Dict[int, Dict[str, Dict[str, Any]]]) -> ParamLayout:
    return ParamLayout.from_metas({int(r): {n: meta_from_plain(m) for n, m in metas.items()}
                                   for r, metas in d.items()})


class ReferenceTensorMeta:
    """What a checkpoint file stores for a ``Suika.migration.TensorMeta``
    (migration.py:29-58): the attributes ``name``, ``dtype``, ``shape``,
    ``tp_meta`` and, for this build's shard kinds, ``kind`` / ``kind_args``.
    An attribute holder: nothing of it runs when a file is loaded."""


class ReferenceParamLayout:
    """What a checkpoint file stores for a ``Suika.migration.ParamLayout``
    (migration.py:161-170): the attribute ``layout``, {rank: {name: meta}}."""


_REFERENCE_NAMES = {ReferenceTensorMeta: ("Suika.migration", "TensorMeta"),
                    ReferenceParamLayout: ("Suika.migration", "ParamLayout")}
_SAFE_GLOBALS = [(cls, f"{mod}.{name}") for cls, (mod, name) in _REFERENCE_NAMES.items()]


class _ReferencePickler(pickle._Pickler):
    """Pickles the two holders under the reference's class paths (without
    importing the reference): the reference's ``torch.load`` then builds its
    own ``ParamLayout`` / ``TensorMeta`` from their attributes."""

    def save_global(self, obj, name=None):
        ref = _REFERENCE_NAMES.get(obj) if isinstance(obj, type) else None
        if ref is None:
            return super().save_global(obj, name)
        module, qualname = ref
        if self.proto >= 4:
            self.save(module)
            self.save(qualname)
            self.write(pickle.STACK_GLOBAL)
        else:
            self.write(pickle.GLOBAL + f"{module}\n{qualname}\n".encode("utf-8"))
        self.memoize(obj)


_PICKLE_MODULE = types.ModuleType("suika_amd_reference_pickle")
_PICKLE_MODULE.Pickler = _ReferencePickler


def meta_to_reference(m: TensorMeta) -> ReferenceTensorMeta:
    r = ReferenceTensorMeta()
    r.dtype = m.dtype
    r.shape = torch.Size(int(s) for s in m.shape)
    r.tp_meta = None if m.tp_meta is None else tuple(int(v) for v in m.tp_meta)
    r.name = m.name
    if m.kind != CHUNK:
        r.kind = m.kind
        r.kind_args = tuple(int(v) for v in m.kind_args)
    return r


def meta_from_reference(r) -> TensorMeta:
    tp = getattr(r, "tp_meta", None)
    return TensorMeta(name=getattr(r, "name", None), dtype=r.dtype, shape=tuple(r.shape),
                      tp_meta=None if tp is None else tuple(tp), kind=getattr(r, "kind", CHUNK),
                      kind_args=tuple(getattr(r, "kind_args", ())))


def layout_to_reference(pl: ParamLayout) -> ReferenceParamLayout:
    out = ReferenceParamLayout()
    out.layout = {int(r): {n: meta_to_reference(m) for n, m in metas.items()} for r, metas in pl.layout.items()}
    return out


def layout_from_reference(obj) -> ParamLayout:
    if isinstance(obj, dict):                  # the plain-dict format of earlier versions
        return layout_from_plain(obj)
    return ParamLayout.from_metas({int(r): {n: meta_from_reference(m) for n, m in metas.items()}
                                   for r, metas in obj.layout.items()})


def _context_to_reference(ctx: Dict[str, Any]) -> Dict[str, Any]:
    out = dict(ctx)
    out["expected_sub_fields"] = [(f, t if isinstance(t, str) else meta_to_reference(t))
                                  for f, t in ctx["expected_sub_fields"]]
    return out


def _context_from_reference(ctx: Dict[str, Any]) -> Dict[str, Any]:
    out = dict(ctx)
    out["expected_sub_fields"] = [
        (f, t if isinstance(t, str) else (meta_from_plain(t) if isinstance(t, dict) else meta_from_reference(t)))
        for f, t in ctx["expected_sub_fields"]]
    return out


def save_reference_object(obj, path: str) -> None:
    """``torch.save`` with the holders written under the reference's class paths."""
    torch.save(obj, path, pickle_module=_PICKLE_MODULE)


def load_reference_object(path: str):
    """``torch.load(weights_only=True)`` of a layout or context file, the
    reference's class paths allowlisted to the attribute holders."""
    with torch.serialization.safe_globals(_SAFE_GLOBALS):
        return torch.load(path, weights_only=True, map_location="cpu")


def _rank_and_world(world) -> tuple:
    if dist.is_available() and dist.is_initialized():
        return dist.get_rank(world), dist.get_world_size(world)
    return 0, 1


def _gather_layout(model: Module, world) -> ParamLayout:
    layout = ParamLayout()
    if dist.is_available() and dist.is_initialized():
        layout.gather(model, world)
    else:
        from .meta import get_param_tensor_meta
        layout.layout[0] = get_param_tensor_meta(model)
    return layout


def _barrier(world) -> None:
    if dist.is_available() and dist.is_initialized():
        dist.barrier(world)


def checkpoint_save(model: Module, optimizer: Optional[Optimizer], other_context: Any,
                    checkpoint_dir: str, world: Optional[dist.ProcessGroup] = None,
                    log_func: Optional[Callable] = None) -> None:
    """Write this rank's shard and (rank 0) the layout (migration.py:1156-1184)."""
    if log_func is None:
        log_func = lambda msg: None  # noqa: E731
    log_func("checkpoint_save: begin")
    os.makedirs(checkpoint_dir, exist_ok=True)
    layout = _gather_layout(model, world)
    state_dict, other_context_dict = merge_model_and_optimizer_state_dict(model, optimizer, other_context)
    rank, _ = _rank_and_world(world)
    if rank == 0:
        save_reference_object(layout_to_reference(layout), os.path.join(checkpoint_dir, LAYOUT_FILE))
        save_reference_object(_context_to_reference(other_context_dict), os.path.join(checkpoint_dir, CONTEXT_FILE))
    torch.save(state_dict, os.path.join(checkpoint_dir, f"state_dict_{rank}.pt"))
    log_func("checkpoint_save: end")


def checkpoint_load(model: Module, optimizer: Union[Callable[[], Optimizer], Optimizer, None],
                    checkpoint_dir: str, world: Optional[dist.ProcessGroup] = None,
                    log_func: Optional[Callable] = None, *, device: Optional[torch.device] = None,
                    route: str = "direct", remove_files: bool = True):
    """Reshard a checkpoint written under another layout into ``model`` (and
    the optimizer) on the GPU (migration.py:1186-1305).

    Returns ``other_context``, or ``(optimizer, other_context)`` when
    ``optimizer`` is a provider callable; a missing checkpoint returns
    ``None`` / ``(optimizer_provider(), None)`` as the reference does.
    Extensions: ``device`` (default: the current CUDA device), ``route``
    (``"direct"`` or ``"buffers"``), ``remove_files`` (rank 0 deletes the
    checkpoint after loading, as the reference always does).
    """
    if log_func is None:
        log_func = lambda msg: None  # noqa: E731
    log_func("checkpoint_load: begin")
    if device is None:
        device = torch.device("cuda", torch.cuda.current_device())
    elif not isinstance(device, torch.device):
        device = torch.device(device)
    if callable(optimizer) and not isinstance(optimizer, Optimizer):
        optimizer_provider, optimizer = optimizer, None
    elif isinstance(optimizer, Optimizer) or optimizer is None:
        optimizer_provider = None
    else:
        raise TypeError(f"optimizer should be Optimizer or Callable, but got {type(optimizer)}")
    rank, _ = _rank_and_world(world)
    # a fresh process's first-use costs (the library's, torch.optim's) are
    # paid on a thread while this one reads the checkpoint
    from .handoff import _WarmUp
    warm = _WarmUp(device, optimizer_provider is not None)
    warm.start()

    try:
        source_layout = layout_from_reference(load_reference_object(os.path.join(checkpoint_dir, LAYOUT_FILE)))
        other_context_dict = _context_from_reference(
            load_reference_object(os.path.join(checkpoint_dir, CONTEXT_FILE)))
    except FileNotFoundError as e:
        log_func(f"checkpoint_load: [warning] checkpoint file not found, skip loading\n{e}")
        warm.join()
        return (optimizer_provider(), None) if optimizer_provider else None

    target_layout = _gather_layout(model, world)
    ops = schedule_param_transfer(source_layout, target_layout)
    # (source rank -> names) this rank's pieces read; only those tensors go to HBM
    needed: Dict[int, set] = {}
    for op in ops:
        if op.dst_rank == rank:
            needed.setdefault(op.src_rank, set()).add(op.param_name)
    _barrier(world)
    fake = {}
    for src in sorted(needed):
        # memory-mapped and handed over in host memory: the transfer reads
        # only its pieces' bytes (pages) from the file and sends only those to
        # the GPU; the reference loads whole files to the CPU (migration.py:1223-1233)
        sd = torch.load(os.path.join(checkpoint_dir, f"state_dict_{src}.pt"), weights_only=True,
                        map_location="cpu", mmap=True)
        fake[src] = {name: sd[name] for name in needed[src] if name in sd}
        del sd
    self_source = fake.get(rank, {})
    warm.library_done.wait()
    target = execute_param_transfer(
        transfer_ops=ops, source_state_dict=dict(self_source), device=device,
        expected_sub_fields=other_context_dict["expected_sub_fields"], world=world,
        fake_source_state_dicts=fake, log_func=log_func, rank=rank, route=route)
    torch.cuda.synchronize(device)
    del fake

    model_state_dict, optimizer_state_dict, other_context = split_model_and_optimizer_state_dict(
        model, merged_state_dict=target, other_context_dict=other_context_dict)
    model_state_dict = OrderedDict(sorted(model_state_dict.items(), key=lambda x: x[0]))
    on_meta = any(p.is_meta for p in model.parameters())
    model.load_state_dict(model_state_dict, assign=on_meta)
    warm.join()
    if optimizer_provider:
        optimizer = optimizer_provider()
    if optimizer is not None and optimizer_state_dict["param_groups"] is not None:
        # one param group, as the reference (migration.py:1267)
        optimizer_state_dict["param_groups"][0]["params"] = \
            optimizer.state_dict()["param_groups"][0]["params"]
        optimizer.load_state_dict(optimizer_state_dict)

    _barrier(world)
    if remove_files and rank == 0:
        os.remove(os.path.join(checkpoint_dir, LAYOUT_FILE))
        os.remove(os.path.join(checkpoint_dir, CONTEXT_FILE))
        r = 0
        while True:
            try:
                os.remove(os.path.join(checkpoint_dir, f"state_dict_{r}.pt"))
            except FileNotFoundError:
                break
            r += 1
    log_func("checkpoint_load: end")
    return (optimizer, other_context) if optimizer_provider else other_context


def _device(device) -> torch.device:
    """The reference's device argument (migration.py:1367-1372): default the
    current CUDA device, made current."""
    if device is None:
        device = torch.device("cuda", torch.cuda.current_device())
    elif not isinstance(device, torch.device):
        device = torch.device(device)
    if device.type == "cuda":
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        torch.cuda.set_device(device.index)
    return device


def migration_save(IPC_queues, model: Module, optimizer: Optional[Optimizer] = None,
                   other_context: Any = None, device: Optional[torch.device] = None,
                   world: Optional[dist.ProcessGroup] = None, log_func: Optional[Callable] = None,
                   checkpoint_resume: Optional[str] = None, *, handoff_mode: Optional[str] = None,
                   wave_bytes: Optional[int] = None):
    """Suika's save-side migration API (Suika/migration.py:1357-1486).

    With ``checkpoint_resume`` it writes the checkpoint (:1382-1392).
    Otherwise it hands this rank's state to the new plan's processes on the
    same GPU over ``IPC_queues`` (forward, backward), as
    ``suika_amd.handoff.live_save`` describes: the world-size handshake, the
    state packed into exported device allocations, and their release once
    the new world has resharded from them.

    ``handoff_mode`` and ``wave_bytes`` (not in the reference) force the
    hand-off's order: ``"whole"``, or ``"waves"`` of at most ``wave_bytes``
    (default: a third of the free memory); ``None`` moves the state whole
    when the device has room for it beside the old state, else in waves."""
    if log_func is None:
        log_func = lambda msg: None  # noqa: E731
    device = _device(device)
    log_func("migration_save: begin")
    if checkpoint_resume is not None:
        log_func(f"migration_save: checkpoint-resume={checkpoint_resume}")
        return checkpoint_save(model=model, optimizer=optimizer, other_context=other_context,
                               checkpoint_dir=checkpoint_resume, world=world, log_func=log_func)
    from .handoff import live_save
    return live_save(IPC_queues, model, optimizer, other_context, device, world, log_func,
                     mode=handoff_mode, wave_bytes=wave_bytes)


def migration_load(IPC_queues, model: Module,
                   optimizer: Union[Optimizer, Callable[[], Optimizer], None] = None,
                   device: Optional[torch.device] = None, world: Optional[dist.ProcessGroup] = None,
                   log_func: Optional[Callable] = None, checkpoint_resume: Optional[str] = None, *,
                   wait_for_release: Optional[bool] = None, return_before_release: bool = False):
    """Suika's load-side migration API (Suika/migration.py:1546-1727).

    With ``checkpoint_resume`` the checkpoint is resharded into ``model`` on
    the GPU (:1566-1575).  Otherwise the old plan's processes on the same GPU
    hand their state over ``IPC_queues`` and this rank reshards its share
    straight from their memory (``suika_amd.handoff.live_load``).  Returns
    ``other_context``, or ``(optimizer, other_context)`` for an optimizer
    provider; a fresh launch (the launcher's placeholder on the queue)
    returns ``None`` / ``(optimizer_provider(), None)``.

    ``wait_for_release`` (not in the reference) chooses when a whole live
    hand-off allocates its destinations: ``None`` beside the old state when
    the device has room, else after the old world released it; ``True``
    always after.  ``return_before_release`` (not in the reference) returns
    once this world's state is adopted and its optimizer built, without
    waiting for the old world to release its state (the reference's order);
    by default no new rank returns before that release."""
    if log_func is None:
        log_func = lambda msg: None  # noqa: E731
    device = _device(device)
    log_func("migration_load: begin")
    if checkpoint_resume is not None:
        log_func(f"migration_load: checkpoint_resume = {checkpoint_resume}")
        return checkpoint_load(model=model, optimizer=optimizer, checkpoint_dir=checkpoint_resume,
                               world=world, log_func=log_func, device=device)
    if callable(optimizer) and not isinstance(optimizer, Optimizer):
        optimizer_provider, optimizer = optimizer, None
    elif isinstance(optimizer, Optimizer) or optimizer is None:
        optimizer_provider = None
    else:
        raise TypeError(f"optimizer should be Optimizer or Callable, but got {type(optimizer)}")
    from .handoff import live_load
    return live_load(IPC_queues, model, optimizer_provider, optimizer, device, world, log_func, wait_for_release,
                     return_before_release)

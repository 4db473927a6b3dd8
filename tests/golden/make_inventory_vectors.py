#!/usr/bin/env python3
"""Write golden vectors of the reference's layout definers.

Runs in the development container only (it reads /root/reference, which the
GPU box does not have).  It imports the reference's model, tensor-parallel and
plan modules through a bare ``Suika`` package (the package ``__init__`` --
engines, schedulers, cluster -- is not imported) and records what they
define for the state that migration moves:

* for every model and stage below, on every rank of a TP group of the given
  degree: the stage model the reference builds (``SuikaGPT`` / ``SuikaLlama`` /
  ``SuikaQwen``, Suika/models/*_model.py, with embedding and lm_head, on the
  meta device), converted by the reference's own ``parallelize_tp``
  (tensor_parallel.py:486-606, ``slice_dim="column"`` as TPEngine's default,
  engine.py:51) in a gloo world of that many CPU processes, then read by the
  reference's ``get_param_tensor_meta`` (migration.py:147-151): parameter
  names in registration order, global shapes, tp meta, and the local shard
  shape;
* ``get_uniform_plan_config``'s layer partition and rank mesh
  (cluster/plan_config.py:477-541, 248-250) for a few plan shapes.

The installed transformers (5.15) no longer gives LlamaAttention /
Qwen2Attention the ``num_heads`` attribute that ``parallelize_tp`` divides by
the TP degree for the attention forward pass (``div_by_tp_deg``,
tensor_parallel.py:567-576; the reference pins transformers 5.1.0).  That
step changes no parameter, so for those two families this script removes the
``div_by_tp_deg`` hint from the attention modules before calling
``parallelize_tp``; everything else runs as the reference wrote it.

The output is tests/golden/inventory_vectors.json.gz; tests/test_inventory_reference.py
compares ``suika_amd.inventory`` (and the oracle's kind table) with it.
"""
from __future__ import annotations

import gzip
import importlib
import json
import os
import socket
import sys
import tempfile
import types
from pathlib import Path

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent / "inventory_vectors.json.gz"

# (key, family, config kwargs, total layers, stages [(layer_index, n_layer)], tp degrees)
MODELS = [
    ("gpt_test", "gpt", {"spec": "GPT-TEST"}, 4, [(0, 4), (0, 2), (2, 2), (1, 2)], [1, 2, 4]),
    ("llama_test", "llama", {"spec": "Llama-TEST"}, 2, [(0, 2), (0, 1), (1, 1)], [1, 2, 4]),
    ("qwen2_test", "qwen", {"spec": "Qwen2-TEST"}, 8, [(0, 8), (0, 4), (4, 4), (2, 3)], [1, 2]),
    ("gpt125m_2l", "gpt", {"vocab_size": 50304, "n_embd": 768, "n_head": 12, "n_layer": 2}, 2,
     [(0, 2), (0, 1), (1, 1)], [2, 4]),
    ("llama7b_2l", "llama", {"hidden_size": 4096, "intermediate_size": 11008, "num_attention_heads": 32,
                             "vocab_size": 32000, "num_hidden_layers": 2}, 2, [(0, 2), (0, 1), (1, 1)], [2, 4]),
    ("llama13b_2l", "llama", {"hidden_size": 5120, "intermediate_size": 13824, "num_attention_heads": 40,
                              "vocab_size": 32000, "num_hidden_layers": 2}, 2, [(0, 2), (1, 1)], [4, 8]),
    ("gpt6.7b_2l", "gpt", {"vocab_size": 50304, "n_embd": 4096, "n_head": 32, "n_layer": 2}, 2,
     [(0, 2), (0, 1)], [8]),
    ("qwen2_7b_2l", "qwen", {"hidden_size": 3584, "intermediate_size": 18944, "num_attention_heads": 28,
                             "num_key_value_heads": 4, "vocab_size": 152064, "num_hidden_layers": 2},
     2, [(0, 2), (1, 1)], [2, 4]),
]

PLANS = [(32, 2, 1, 4), (40, 2, 1, 4), (40, 1, 1, 8), (32, 4, 1, 1), (28, 1, 1, 2), (12, 1, 1, 2),
         (7, 3, 2, 2), (5, 2, 2, 1), (4, 4, 1, 2), (2, 2, 2, 2)]


def _bare_suika():
    pkg = types.ModuleType("Suika")
    pkg.__path__ = [str(REF / "Suika")]
    sys.modules["Suika"] = pkg


def _config(family, kw):
    if family == "gpt":
        gm = importlib.import_module("Suika.models.gpt_model")
        return gm.GPT_specs[kw["spec"]] if "spec" in kw else gm.GPTConfig(**kw), gm.SuikaGPT
    if family == "llama":
        lm = importlib.import_module("Suika.models.llama_model")
        return lm.Llama_specs[kw["spec"]] if "spec" in kw else lm.LlamaConfig(**kw), lm.SuikaLlama
    qm = importlib.import_module("Suika.models.qwen_model")
    return qm.Qwen_specs[kw["spec"]] if "spec" in kw else qm.QwenConfig(**kw), qm.SuikaQwen


def _config_record(family, cfg):
    if family == "gpt":
        return {"hidden": cfg.n_embd, "n_head": cfg.n_head, "n_kv_head": cfg.n_head,
                "ffn": cfg.n_inner or 4 * cfg.n_embd, "vocab": cfg.vocab_size, "n_layer": cfg.n_layer}
    return {"hidden": cfg.hidden_size, "n_head": cfg.num_attention_heads,
            "n_kv_head": cfg.num_key_value_heads, "ffn": cfg.intermediate_size, "vocab": cfg.vocab_size,
            "n_layer": cfg.num_hidden_layers}


def _worker(rank: int, world: int, port: int, outdir: str) -> None:
    import torch
    import torch.distributed as dist
    _bare_suika()
    os.environ.update(MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port))
    dist.init_process_group("gloo", rank=rank, world_size=world)
    tpm = importlib.import_module("Suika.tensor_parallel")
    dm = importlib.import_module("Suika.device_mesh")
    mig = importlib.import_module("Suika.migration")
    mesh = dm.DeviceMesh1D(list(range(world)))
    out = {}
    for key, family, kw, _, stages, tps in MODELS:
        if world not in tps:
            continue
        cfg, cls = _config(family, kw)
        for li, nl in stages:
            model = cls(cfg, li, nl, add_embedding_and_lm_head=True, init_on_meta=True)
            if family != "gpt":
                for mod in model.modules():
                    if hasattr(mod, "div_by_tp_deg") and hasattr(mod, "q_proj"):
                        del mod.div_by_tp_deg
            model = tpm.parallelize_tp(model, torch.device("cpu"), mesh, "column", init_on_meta=True)
            params = dict(mig.get_named_parameters_and_persistent_buffers(model))
            rows = []
            for name, m in mig.get_param_tensor_meta(model).items():
                tp = getattr(m, "tp_meta", None)
                rows.append([name, [int(s) for s in m.shape], None if tp is None else [int(v) for v in tp],
                             [int(s) for s in params[name].shape]])
            out[f"{key}|{li}:{nl}|tp{world}"] = rows
    with open(os.path.join(outdir, f"tp{world}_rank{rank}.json"), "w") as fh:
        json.dump(out, fh)
    dist.barrier()
    dist.destroy_process_group()


def _free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def main() -> int:
    import torch.multiprocessing as mp
    _bare_suika()
    pc = importlib.import_module("Suika.cluster.plan_config")
    record = {"source": "Suika/models/{gpt,llama,qwen}_model.py + tensor_parallel.parallelize_tp + "
                        "migration.get_param_tensor_meta + cluster/plan_config.py (reference, imported)",
              "format": "stage rows per TP rank: [name, global shape, tp_meta, local shape]",
              "models": {}, "plans": {}}
    for key, family, kw, n_layer, stages, tps in MODELS:
        cfg, _ = _config(family, kw)
        rec = _config_record(family, cfg)
        assert rec["n_layer"] == n_layer, key
        record["models"][key] = {"family": family, "config": rec, "stages": {}}
    with tempfile.TemporaryDirectory() as tmp:
        for world in sorted({t for m in MODELS for t in m[5]}):
            mp.start_processes(_worker, args=(world, _free_port(), tmp), nprocs=world, join=True,
                               start_method="spawn")
            for rank in range(world):
                with open(os.path.join(tmp, f"tp{world}_rank{rank}.json")) as fh:
                    part = json.load(fh)
                for k, rows in part.items():
                    key, stage, tpk = k.split("|")
                    st = record["models"][key]["stages"].setdefault(stage, {}).setdefault(tpk, [None] * world)
                    st[rank] = rows
    for n, pp, dp, tp in PLANS:
        c = pc.get_uniform_plan_config("H100", (pp, dp, tp), gbs=8 * dp, n_layer=n, n_mb=1)
        rm = c.set_rank_mesh()
        record["plans"][f"{n},{pp},{dp},{tp}"] = {
            "layer_partition": [int(v) for v in c.layer_partition],
            "rank": [[[int(rm.get_rank((p, d, t))) for t in range(tp)] for d in range(dp)] for p in range(pp)]}
    with gzip.open(OUT, "wt") as fh:
        json.dump(record, fh, separators=(",", ":"))
    n_rows = sum(len(r) for m in record["models"].values() for s in m["stages"].values() for t in s.values()
                 for r in t)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {n_rows} parameter rows)")
    return 0


if __name__ == "__main__":
    sys.exit(main())

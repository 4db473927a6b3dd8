"""The layout definers pinned against the reference's own model code.

tests/golden/inventory_vectors.json.gz holds what the reference's modules
produce, recorded in the development container by
tests/golden/make_inventory_vectors.py. It covers:

* the stage models of GPT-TEST, Llama-TEST, Qwen2-TEST and two-layer models
  of the five benchmark families. They are converted by the reference's
  ``parallelize_tp`` on every rank of a TP group and read by its
  ``get_param_tensor_meta``. Each yields parameter names in registration
  order, global shapes, tp meta and local shard shapes;
* ``get_uniform_plan_config``'s layer partitions and rank meshes.

``suika_amd.inventory`` (names, order, shapes, kinds, embedding / lm_head /
norm placement, stage partition, rank order) must reproduce every row, with
the reference's kinds (no extensions). The oracle's kind table
(``REFERENCE_KINDS`` / ``kind_of_name``) must label every recorded parameter
the way its recorded tp meta says. Planted mistakes in the oracle's table
(an ``o_proj`` marked column-parallel, a row bias marked split) must be
caught.
"""
import gzip
import json
from pathlib import Path

import pytest
import torch

from oracle import reshard_oracle as O
from suika_amd.inventory import ModelSpec, Parallel, layer_partition, param_meta, stage_params

VEC = json.load(gzip.open(Path(__file__).resolve().parent / "golden" / "inventory_vectors.json.gz", "rt"))
MODELS = VEC["models"]
STAGES = [(key, stage, tpk) for key, m in sorted(MODELS.items()) for stage in sorted(m["stages"])
          for tpk in sorted(m["stages"][stage])]


def _spec(key) -> ModelSpec:
    m = MODELS[key]
    c = m["config"]
    return ModelSpec(m["family"], n_layer=c["n_layer"], hidden=c["hidden"], n_head=c["n_head"], ffn=c["ffn"],
                     vocab=c["vocab"], n_kv_head=c["n_kv_head"], vocab_parallel=False, fused_qkv=False,
                     positions=0, embeddings=True)


def _kind_label(tp_meta):
    if tp_meta is None:
        return "repl"
    return "col" if tp_meta[0] == 0 else "row"


def test_fixture_covers_every_family_and_stage_kind():
    fams = {m["family"] for m in MODELS.values()}
    assert fams == {"gpt", "llama", "qwen"}
    names = {row[0] for m in MODELS.values() for s in m["stages"].values() for t in s.values() for r in t
             for row in r}
    for must in ("wte.weight", "lm_head.weight", "lm_head.bias", "norm.weight", "h.0.self_attn.q_proj.bias",
                 "h.1.attn.c_proj.linear.bias", "h.3.mlp.c_proj.linear.weight"):
        assert must in names, must
    # middle stages carry neither the embedding nor the head
    rows = MODELS["gpt_test"]["stages"]["1:2"]["tp2"][0]
    assert [r[0] for r in rows][0] == "h.1.ln_1.weight" and not any(r[0].startswith(("wte", "lm_head"))
                                                                  for r in rows)


@pytest.mark.parametrize("key,stage,tpk", STAGES)
def test_inventory_reproduces_reference_stage(key, stage, tpk):
    m = _spec(key)
    li, nl = (int(v) for v in stage.split(":"))
    tp = int(tpk[2:])
    specs = stage_params(m, li, nl)
    for tp_i, rows in enumerate(MODELS[key]["stages"][stage][tpk]):
        ours = [param_meta(s, tp, tp_i, torch.float32) for s in specs]
        assert [o.name for o in ours] == [r[0] for r in rows], f"{key} {stage} {tpk}: names / order"
        for o, (name, gshape, tp_meta, lshape) in zip(ours, rows):
            assert list(o.shape) == gshape, f"{name}: global shape"
            assert (None if o.tp_meta is None else list(o.tp_meta)) == tp_meta, f"{name}: tp meta"
            assert list(o.actual_shape()) == lshape, f"{name}: local shape"


@pytest.mark.parametrize("key,stage,tpk", STAGES)
def test_oracle_kind_table_matches_reference(key, stage, tpk):
    for rows in MODELS[key]["stages"][stage][tpk]:
        for name, _, tp_meta, _ in rows:
            assert O.kind_of_name(name, vocab_parallel=False) == _kind_label(tp_meta), name


def test_planted_kind_table_mistakes_are_caught(monkeypatch):
    """A wrong entry in the oracle's table fails the comparison above."""
    rows = [row for key, stage, tpk in STAGES for r in MODELS[key]["stages"][stage][tpk] for row in r]

    def mismatches():
        return sum(O.kind_of_name(n, False) != _kind_label(tp) for n, _, tp, _ in rows)

    assert mismatches() == 0
    for suffix, wrong in (("self_attn.o_proj.weight", "col"), ("attn.c_proj.linear.bias", "row"),
                          ("lm_head.weight", "repl"), ("self_attn.k_proj.bias", "repl")):
        table = dict(O.REFERENCE_KINDS)
        table[suffix] = wrong
        monkeypatch.setattr(O, "REFERENCE_KINDS", table)
        assert mismatches() > 0, suffix
        monkeypatch.undo()


@pytest.mark.parametrize("plan", sorted(VEC["plans"]))
def test_partition_and_rank_order_match_plan_config(plan):
    n, pp, dp, tp = (int(v) for v in plan.split(","))
    rec = VEC["plans"][plan]
    assert layer_partition(n, pp) == rec["layer_partition"]
    par = Parallel(tp=tp, pp=pp, dp=dp)
    assert [[[par.rank(p, t, d) for t in range(tp)] for d in range(dp)] for p in range(pp)] == rec["rank"]
    for r in range(par.world):
        p, d, t = par.coord(r)
        assert rec["rank"][p][d][t] == r

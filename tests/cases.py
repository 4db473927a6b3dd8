"""Small reshard cases shared by the CPU and GPU suites.

* the reference's own test shapes -- GPT-TEST (gpt_model.py:152-158),
  Llama-TEST (llama_model.py:169-176), Qwen2-TEST (qwen_model.py:178-189) --
  under TP 1<->2<->4<->8 and PP 1<->2<->4 changes;
* the five benchmark workloads at a small shape with the same plan change,
  kinds and fields (vocab sizes chosen so padded rows appear);
* Qwen2-TEST at TP2: ``down_proj [1024, 2028]`` split along the last dim gives
  1014-element rows (4056 B f32 / 2028 B bf16) at an 8112 / 4056 B stride --
  not multiples of 16 bytes -- so the kernels' narrow-vector paths run.
"""
from __future__ import annotations

from dataclasses import replace
from typing import Dict, List

import torch

from suika_amd.inventory import ModelSpec, Parallel
from suika_amd.meta import vocab_padded
from suika_amd.workloads import CONFIGS, Workload, scaled

_F32_3 = (("param", torch.float32), ("exp_avg", torch.float32), ("exp_avg_sq", torch.float32))
_BF16_4 = (("param", torch.bfloat16), ("master", torch.float32),
           ("exp_avg", torch.float32), ("exp_avg_sq", torch.float32))

GPT_TEST = ModelSpec("gpt", n_layer=4, hidden=16, n_head=4, ffn=64, vocab=128)
LLAMA_TEST = ModelSpec("llama", n_layer=2, hidden=16, n_head=4, ffn=64, vocab=128)
QWEN2_TEST = ModelSpec("qwen", n_layer=2, hidden=1024, n_head=4, n_kv_head=2, head_dim=256,
                       ffn=2028, vocab=1024)


def _w(key, model, src, dst, dst_pp, dst_tp, fields=_BF16_4, recast=(), seed=0,
       param_dtype=torch.bfloat16) -> Workload:
    src_fields = tuple(f for f, _ in fields if f not in dict(recast))
    return Workload(key=key, model=model, src=src, dst=dst, dst_pp=dst_pp, dst_tp=dst_tp,
                    src_fields=src_fields, field_dtypes=fields, recast=tuple(recast), seed=seed,
                    param_dtype=param_dtype)


def reference_test_cases() -> List[Workload]:
    out = []
    for (stp, spp), (dtp, dpp) in [((1, 1), (2, 1)), ((2, 1), (4, 1)), ((4, 1), (2, 1)),
                                   ((4, 1), (1, 1)), ((2, 2), (4, 1)), ((1, 4), (2, 2)),
                                   ((2, 1), (1, 2))]:
        for dtp_i in sorted({0, dtp - 1}):
            for dpp_i in sorted({0, dpp - 1}):
                out.append(_w(f"gpt_test_tp{stp}pp{spp}_tp{dtp}pp{dpp}_d{dpp_i}.{dtp_i}",
                              GPT_TEST, Parallel(stp, spp), Parallel(dtp, dpp), dpp_i, dtp_i,
                              fields=_F32_3, param_dtype=torch.float32, seed=11))
    for (stp, spp), (dtp, dpp) in [((4, 1), (2, 1)), ((2, 1), (4, 1)), ((1, 2), (4, 1)),
                                   ((4, 2), (1, 1))]:
        for dtp_i in sorted({0, dtp - 1}):
            out.append(_w(f"llama_test_tp{stp}pp{spp}_tp{dtp}pp{dpp}_d0.{dtp_i}",
                          LLAMA_TEST, Parallel(stp, spp), Parallel(dtp, dpp), 0, dtp_i, seed=12))
    return out


def dp_cases() -> List[Workload]:
    """Data-parallel replicas on either side: every piece has several owners
    holding identical bytes, so the schedule's greedy choice among them (self
    first, least accumulated volume, reuse of connected peers:
    Suika/migration.py:355-379) decides which peer sends it."""
    out = []
    for model, (src, dst, dpp_i, ddp_i, dtp_i), fields, seed in [
            (GPT_TEST, ((2, 1, 2), (1, 2, 2), 1, 1, 0), _F32_3, 41),
            (GPT_TEST, ((4, 1, 2), (2, 2, 1), 0, 0, 1), _F32_3, 42),
            (LLAMA_TEST, ((2, 2, 2), (4, 1, 2), 0, 1, 3), _BF16_4, 43),
            (LLAMA_TEST, ((1, 1, 4), (2, 1, 2), 0, 1, 1), _BF16_4, 44)]:
        s, d = Parallel(*src), Parallel(*dst)
        key = (f"{model.family}_test_tp{s.tp}pp{s.pp}dp{s.dp}_tp{d.tp}pp{d.pp}dp{d.dp}"
               f"_d{dpp_i}.{ddp_i}.{dtp_i}")
        w = _w(key, model, s, d, dpp_i, dtp_i, fields=fields, seed=seed,
               param_dtype=torch.float32 if fields is _F32_3 else torch.bfloat16)
        out.append(replace(w, dst_dp=ddp_i))
    return out


def alignment_cases() -> List[Workload]:
    return [
        _w("qwen2_test_tp2_tp1", QWEN2_TEST, Parallel(2), Parallel(1), 0, 0, seed=13),
        _w("qwen2_test_tp1_tp2_d1", QWEN2_TEST, Parallel(1), Parallel(2), 0, 1, seed=14),
        _w("qwen2_test_tp1_tp2_recast", QWEN2_TEST, Parallel(1), Parallel(2), 0, 0,
           fields=(("master", torch.float32), ("exp_avg", torch.float32),
                   ("exp_avg_sq", torch.float32), ("param", torch.bfloat16)),
           recast=(("param", "master"),), seed=15),
    ]


def scaled_configs() -> Dict[str, Workload]:
    """The five benchmark plan changes at a shape the oracle runs in seconds."""
    c = CONFIGS
    return {
        "gpt125m_tp2_tp4": scaled(c["gpt125m_tp2_tp4"], n_layer=3, hidden=64, ffn=256, vocab=1000,
                                  n_head=4),
        "llama7b_tp4pp2_tp2pp2": scaled(c["llama7b_tp4pp2_tp2pp2"], n_layer=4, hidden=64, ffn=176,
                                        vocab=1000, n_head=8),
        "llama13b_tp8_tp4pp2": scaled(c["llama13b_tp8_tp4pp2"], n_layer=4, hidden=64, ffn=128,
                                      vocab=1000, n_head=8),
        "gpt6.7b_tp1pp4_tp8": scaled(c["gpt6.7b_tp1pp4_tp8"], n_layer=4, hidden=64, ffn=256,
                                     vocab=1000, n_head=8, positions=32),
        "qwen7b_tp2_tp4": scaled(c["qwen7b_tp2_tp4"], n_layer=2, hidden=64, ffn=96, vocab=1000,
                                 n_head=8, n_kv_head=4, head_dim=8),
    }


def padded_vocab_cases() -> List[Workload]:
    """Vocab-parallel tables whose padding shows up on both sides."""
    m = ModelSpec("llama", n_layer=2, hidden=32, n_head=4, ffn=64, vocab=712, vocab_parallel=True,
                  pad_multiple=64)
    out = []
    for stp, dtp in [(2, 4), (4, 2), (1, 8), (8, 1), (2, 8)]:
        # last destination rank that still holds vocabulary rows (a shard of
        # padding only is rejected by the schedule)
        per = vocab_padded(m.vocab, dtp, m.pad_multiple) // dtp
        last = (m.vocab - 1) // per
        for d in sorted({0, last}):
            out.append(_w(f"vocab_pad_tp{stp}_tp{dtp}_d{d}", m, Parallel(stp), Parallel(dtp), 0, d,
                          seed=16))
    return out


def all_small_cases() -> List[Workload]:
    return (reference_test_cases() + dp_cases() + alignment_cases()
            + list(scaled_configs().values()) + padded_vocab_cases())


def golden_cases() -> Dict[str, Workload]:
    """Tiny cases whose inputs and expected outputs are committed under
    tests/golden/ (a few KB): every kind, a TP merge and split, a PP move, an
    all-padding vocabulary shard, the bf16 recast and rows that are not a
    multiple of 16 bytes."""
    gpt = ModelSpec("gpt", n_layer=2, hidden=8, n_head=2, ffn=16, vocab=24)
    llama_v = ModelSpec("llama", n_layer=2, hidden=8, n_head=2, ffn=12, vocab=20,
                        vocab_parallel=True, pad_multiple=4)
    qkv = ModelSpec("llama", n_layer=1, hidden=8, n_head=4, n_kv_head=2, head_dim=2, ffn=8,
                    vocab=16, fused_qkv=True)
    vocab = ModelSpec("llama", n_layer=1, hidden=4, n_head=2, ffn=8, vocab=12,
                      vocab_parallel=True, pad_multiple=5)
    qwen = ModelSpec("qwen", n_layer=1, hidden=8, n_head=2, n_kv_head=2, ffn=8, vocab=12)
    odd = ModelSpec("llama", n_layer=1, hidden=6, n_head=2, ffn=10, vocab=14)
    recast = (("master", torch.float32), ("exp_avg", torch.float32),
              ("exp_avg_sq", torch.float32), ("param", torch.bfloat16))
    return {
        "gpt_tp1_tp2_d1": _w("gpt_tp1_tp2_d1", gpt, Parallel(1), Parallel(2), 0, 1, fields=_F32_3,
                             param_dtype=torch.float32, seed=21),
        "llama_tp2pp1_tp1pp2_d1": _w("llama_tp2pp1_tp1pp2_d1", llama_v, Parallel(2), Parallel(1, 2),
                                     1, 0, seed=22),
        "llama_tp1pp2_tp2pp1_d0": _w("llama_tp1pp2_tp2pp1_d0", llama_v, Parallel(1, 2), Parallel(2),
                                     0, 0, seed=23),
        "qkv_tp1_tp2_d1": _w("qkv_tp1_tp2_d1", qkv, Parallel(1), Parallel(2), 0, 1, seed=24),
        "qkv_tp2_tp1": _w("qkv_tp2_tp1", qkv, Parallel(2), Parallel(1), 0, 0, seed=25),
        "vocab_tp2_tp4_d2": _w("vocab_tp2_tp4_d2", vocab, Parallel(2), Parallel(4), 0, 2, seed=26),
        "vocab_tp2_tp4_d3": _w("vocab_tp2_tp4_d3", vocab, Parallel(2), Parallel(4), 0, 3, seed=27),
        "qwen_recast_tp2_tp1": _w("qwen_recast_tp2_tp1", qwen, Parallel(2), Parallel(1), 0, 0,
                                  fields=recast, recast=(("param", "master"),), seed=28),
        "odd_rows_tp2_tp1": _w("odd_rows_tp2_tp1", odd, Parallel(2), Parallel(1), 0, 0, seed=29),
    }

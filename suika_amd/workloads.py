"""The reshard workloads: which plan change, which destination share, which
state fields -- and a device-side generator of their synthetic source state.

``CONFIGS`` holds the five benchmark shapes (GPT-125M, Llama2-7B, Llama2-13B,
GPT-6.7B, Qwen2-7B).  ``scaled`` derives a small variant with the same plan
change and kinds, for parity tests that a CPU oracle finishes in seconds.

State per parameter: ``param`` (bf16, or f32 for the GPT-125M case),
``master`` f32, ``exp_avg`` f32, ``exp_avg_sq`` f32.  Values are drawn on the
global tensor and then sharded, so replicas agree: master ~ N(0, 0.02),
exp_avg ~ N(0, 1e-3), exp_avg_sq = |N(0, 1e-6)|, param = bf16(master)
(round to nearest even), pad rows 0.
"""
from __future__ import annotations

from dataclasses import dataclass, replace
from typing import Dict, Iterable, List, Optional, Tuple

import torch

from .geometry import segments, view_axis
from .inventory import ModelSpec, Parallel, build_layout
from .meta import ParamLayout, TensorMeta, TransferOp, schedule_param_transfer

FIELD_STD = {"master": 0.02, "param": 0.02, "exp_avg": 1e-3, "exp_avg_sq": 1e-6}


@dataclass(frozen=True)
class Workload:
    key: str
    model: ModelSpec
    src: Parallel
    dst: Parallel
    dst_pp: int
    dst_tp: int
    src_fields: Tuple[str, ...]               # normal sub-fields held by the sources
    field_dtypes: Tuple[Tuple[str, torch.dtype], ...]
    recast: Tuple[Tuple[str, str], ...] = ()  # (bf16 target field, f32 source field)
    seed: int = 0
    param_dtype: torch.dtype = torch.bfloat16  # TensorMeta dtype (schedule volumes)
    description: str = ""
    dst_dp: int = 0                           # data-parallel replica of the destination

    @property
    def dst_rank(self) -> int:
        return self.dst.rank(self.dst_pp, self.dst_tp, self.dst_dp)

    @property
    def dtypes(self) -> Dict[str, torch.dtype]:
        return dict(self.field_dtypes)

    @property
    def recast_map(self) -> Dict[str, str]:
        return dict(self.recast)

    def layouts(self) -> Tuple[ParamLayout, ParamLayout]:
        src_dtype = self.dtypes.get("param", torch.float32)
        return (build_layout(self.model, self.src, src_dtype),
                build_layout(self.model, self.dst, self.param_dtype))

    def ops(self, minimum_est_peers: Optional[int] = None) -> List[TransferOp]:
        """The schedule's ops landing on this workload's destination rank."""
        spl, tpl = self.layouts()
        sched = schedule_param_transfer(spl, tpl, minimum_est_peers=minimum_est_peers)
        return [op for op in sched if op.dst_rank == self.dst_rank]


_BF16_4 = (("param", torch.bfloat16), ("master", torch.float32),
           ("exp_avg", torch.float32), ("exp_avg_sq", torch.float32))
_F32_3 = (("param", torch.float32), ("exp_avg", torch.float32), ("exp_avg_sq", torch.float32))
_F32_MASTER_3 = (("master", torch.float32), ("exp_avg", torch.float32),
                 ("exp_avg_sq", torch.float32), ("param", torch.bfloat16))

CONFIGS: Dict[str, Workload] = {
    "gpt125m_tp2_tp4": Workload(
        key="gpt125m_tp2_tp4",
        model=ModelSpec("gpt", n_layer=12, hidden=768, n_head=12, ffn=3072, vocab=50304),
        src=Parallel(tp=2), dst=Parallel(tp=4), dst_pp=0, dst_tp=0,
        src_fields=("param", "exp_avg", "exp_avg_sq"), field_dtypes=_F32_3, seed=0,
        param_dtype=torch.float32,
        description="GPT-125M fp32 param+m+v, TP2->TP4, dest tp0"),
    "llama7b_tp4pp2_tp2pp2": Workload(
        key="llama7b_tp4pp2_tp2pp2",
        model=ModelSpec("llama", n_layer=32, hidden=4096, n_head=32, ffn=11008, vocab=32000,
                        vocab_parallel=True),
        src=Parallel(tp=4, pp=2), dst=Parallel(tp=2, pp=2), dst_pp=0, dst_tp=0,
        src_fields=("param", "master", "exp_avg", "exp_avg_sq"), field_dtypes=_BF16_4, seed=1,
        description="Llama2-7B bf16 param + f32 master/m/v, TP4PP2->TP2PP2, dest (pp0,tp0)"),
    "llama13b_tp8_tp4pp2": Workload(
        key="llama13b_tp8_tp4pp2",
        model=ModelSpec("llama", n_layer=40, hidden=5120, n_head=40, ffn=13824, vocab=32000,
                        fused_qkv=True, vocab_parallel=True),
        src=Parallel(tp=8), dst=Parallel(tp=4, pp=2), dst_pp=1, dst_tp=2,
        src_fields=("param", "master", "exp_avg", "exp_avg_sq"), field_dtypes=_BF16_4, seed=2,
        description="Llama2-13B fused QKV, TP8PP1->TP4PP2, dest (pp1,tp2)"),
    "gpt6.7b_tp1pp4_tp8": Workload(
        key="gpt6.7b_tp1pp4_tp8",
        model=ModelSpec("gpt", n_layer=32, hidden=4096, n_head=32, ffn=16384, vocab=50304,
                        vocab_parallel=True, positions=2048),
        src=Parallel(tp=1, pp=4), dst=Parallel(tp=8), dst_pp=0, dst_tp=0,
        src_fields=("param", "master", "exp_avg", "exp_avg_sq"), field_dtypes=_BF16_4, seed=3,
        description="GPT-6.7B + wpe, TP1PP4->TP8PP1, dest tp0"),
    "qwen7b_tp2_tp4": Workload(
        key="qwen7b_tp2_tp4",
        model=ModelSpec("qwen", n_layer=28, hidden=3584, n_head=28, n_kv_head=4, head_dim=128,
                        ffn=18944, vocab=152064, vocab_parallel=True),
        src=Parallel(tp=2), dst=Parallel(tp=4), dst_pp=0, dst_tp=3,
        src_fields=("master", "exp_avg", "exp_avg_sq"), field_dtypes=_F32_MASTER_3,
        recast=(("param", "master"),), seed=4,
        description="Qwen2-7B GQA f32 master/m/v + bf16 recast, TP2->TP4, dest tp3"),
}

# Order of the benchmark configurations (GPT-125M, Llama2-7B, Llama2-13B, GPT-6.7B, Qwen2-7B).
CONFIG_ORDER = ["gpt125m_tp2_tp4", "llama7b_tp4pp2_tp2pp2", "llama13b_tp8_tp4pp2",
                "gpt6.7b_tp1pp4_tp8", "qwen7b_tp2_tp4"]
BENCH_CONFIG = "llama7b_tp4pp2_tp2pp2"


def scaled(w: Workload, n_layer: int, hidden: int, ffn: int, vocab: int,
           n_head: Optional[int] = None, n_kv_head: Optional[int] = None,
           head_dim: Optional[int] = None, positions: Optional[int] = None) -> Workload:
    """Same plan change and kinds at a smaller shape."""
    m = replace(w.model, n_layer=n_layer, hidden=hidden, ffn=ffn, vocab=vocab,
                n_head=n_head or w.model.n_head,
                n_kv_head=n_kv_head if n_kv_head is not None else w.model.n_kv_head,
                head_dim=head_dim if head_dim is not None else w.model.head_dim,
                positions=positions if positions is not None else w.model.positions)
    return replace(w, key=w.key + f"_small{n_layer}x{hidden}", model=m)


# ------------------------------------------------------------------ state

def fields_of(w: Workload) -> List[str]:
    """Normal sub-fields moved by the kernels (recast targets excluded)."""
    return list(w.src_fields)


def shard_global(G: torch.Tensor, meta: TensorMeta) -> torch.Tensor:
    """A shard cut from its global tensor on the tensor's device, pad rows 0."""
    view = view_axis(meta)
    segs, pads = segments(meta, view)
    shape = tuple(int(s) for s in meta.actual_shape())
    out = torch.zeros(shape, dtype=G.dtype, device=G.device) if pads else \
        torch.empty(shape, dtype=G.dtype, device=G.device)
    g2 = G.reshape(-1, G.shape[-1]) if (view == 1 and G.dim() > 0) else G.reshape(G.shape[0] if G.dim() else 1, -1)
    o2 = out.reshape(-1, out.shape[-1]) if (view == 1 and out.dim() > 0) else out.reshape(out.shape[0] if out.dim() else 1, -1)
    for s in segs:
        o2[s.l_row:s.l_row + s.rows, s.l_col:s.l_col + s.cols] = \
            g2[s.g_row:s.g_row + s.rows, s.g_col:s.g_col + s.cols]
    return out


def make_source_state(w: Workload, ranks: Iterable[int], device, seed: Optional[int] = None
                      ) -> Dict[int, Dict[str, Dict[str, torch.Tensor]]]:
    """Synthetic source shards of ``ranks`` generated on ``device``.

    Global tensors are drawn per name (sorted) and field, then cut into the
    requested ranks' shards.  Used by the benchmark and smoke runs; parity
    tests build their inputs from the oracle's closed forms instead.
    """
    spl, _ = w.layouts()
    ranks = sorted(set(ranks))
    dt = w.dtypes
    gen = torch.Generator(device=device)
    gen.manual_seed(w.seed if seed is None else seed)
    names = sorted({n for r in ranks for n in spl.layout[r]})
    out: Dict[int, Dict[str, Dict[str, torch.Tensor]]] = {r: {} for r in ranks}
    for name in names:
        holders = [r for r in ranks if name in spl.layout[r]]
        shape = tuple(int(s) for s in spl.layout[holders[0]][name].shape)
        glob: Dict[str, torch.Tensor] = {}
        base = "master" if "master" in w.src_fields else "param"
        for f in ("master", "param", "exp_avg", "exp_avg_sq"):
            if f not in w.src_fields or (f == "param" and base == "master"):
                continue
            g = torch.randn(shape, generator=gen, dtype=torch.float32, device=device)
            g.mul_(FIELD_STD[f])
            if f == "exp_avg_sq":
                g.abs_()
            glob[f] = g
        if "param" in w.src_fields and base == "master":
            glob["param"] = glob["master"].to(dt["param"])
        for r in holders:
            meta = spl.layout[r][name]
            out[r][name] = {f: shard_global(glob[f], meta).to(dt[f]) for f in w.src_fields}
        del glob
    return out

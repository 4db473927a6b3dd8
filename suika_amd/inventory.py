"""Parameter inventory of the model families and their 3-D layouts.

Names, global shapes and TP kinds follow the reference's model definitions:

* GPT   -- Suika/models/gpt_model.py:13-31 (Megatron TP of GPT2Block),
           :87-136 (wte / lm_head), models/utils.py:433-475 (Conv1D replaced
           by ``.linear`` nn.Linear, weight [out, in]);
* Llama -- Suika/models/llama_model.py:16-35, :108-157;
* Qwen2 -- Suika/models/qwen_model.py:17-40, :114-165 (q/k/v biases).

Column-parallel weights and biases split dim 0, row-parallel weights split
the last dim and keep their bias replicated (tensor_parallel.py:189-214,
255-261, 368-390, 435-441).  ``lm_head`` is an ``nn.Linear`` without TP hints,
so ``parallelize_tp``'s default ``slice_dim="column"`` makes it column
parallel (tensor_parallel.py:486-606, engine.py:51).  Layers keep their global
index in names (models/utils.py:375-422).  Stage partition: ``n // pp + (i <
n % pp)`` layers for stage ``i`` (cluster/plan_config.py:497-501, 531-533);
rank = ``pp_i * dp * tp + dp_i * tp + tp_i`` (plan_config.py:505-508).

Build extensions selected per model: ``vocab_parallel`` (wte split over TP
with padding), ``fused_qkv`` (one head-granular ``qkv_proj``), ``positions``
(learned GPT position table ``wpe``).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch

from .meta import QKV_HEADS, VOCAB_PAD, ParamLayout, TensorMeta

COL, ROW, REPL, VOCAB, QKV = "col", "row", "repl", "vocab", "qkv"


@dataclass(frozen=True)
class ModelSpec:
    family: str                      # "gpt" | "llama" | "qwen"
    n_layer: int
    hidden: int
    n_head: int
    ffn: int
    vocab: int
    n_kv_head: Optional[int] = None  # default: n_head
    head_dim: Optional[int] = None   # default: hidden // n_head
    fused_qkv: bool = False
    vocab_parallel: bool = False
    pad_multiple: int = 128
    positions: int = 0               # gpt: rows of a learned wpe table (0: none)
    embeddings: bool = True          # add_embedding_and_lm_head

    @property
    def kv_heads(self) -> int:
        return self.n_kv_head or self.n_head

    @property
    def hd(self) -> int:
        return self.head_dim or self.hidden // self.n_head


@dataclass(frozen=True)
class ParamSpec:
    name: str
    shape: Tuple[int, ...]
    kind: str
    kind_args: Tuple[int, ...] = ()


def layer_params(m: ModelSpec, L: int) -> List[ParamSpec]:
    """One block's parameters in ``named_parameters`` order."""
    H, F = m.hidden, m.ffn
    p = f"h.{L}."
    if m.family == "gpt":
        return [
            ParamSpec(p + "ln_1.weight", (H,), REPL),
            ParamSpec(p + "ln_1.bias", (H,), REPL),
            ParamSpec(p + "attn.c_attn.linear.weight", (3 * H, H), COL),
            ParamSpec(p + "attn.c_attn.linear.bias", (3 * H,), COL),
            ParamSpec(p + "attn.c_proj.linear.weight", (H, H), ROW),
            ParamSpec(p + "attn.c_proj.linear.bias", (H,), REPL),
            ParamSpec(p + "ln_2.weight", (H,), REPL),
            ParamSpec(p + "ln_2.bias", (H,), REPL),
            ParamSpec(p + "mlp.c_fc.linear.weight", (F, H), COL),
            ParamSpec(p + "mlp.c_fc.linear.bias", (F,), COL),
            ParamSpec(p + "mlp.c_proj.linear.weight", (H, F), ROW),
            ParamSpec(p + "mlp.c_proj.linear.bias", (H,), REPL),
        ]
    assert m.family in ("llama", "qwen"), f"unknown family {m.family}"
    q, kv = m.n_head * m.hd, m.kv_heads * m.hd
    bias = m.family == "qwen"
    out: List[ParamSpec] = []
    a = p + "self_attn."
    if m.fused_qkv:
        qkv_args = (m.n_head, m.kv_heads, m.hd)
        out.append(ParamSpec(a + "qkv_proj.weight", (q + 2 * kv, H), QKV, qkv_args))
        if bias:
            out.append(ParamSpec(a + "qkv_proj.bias", (q + 2 * kv,), QKV, qkv_args))
    else:
        for proj, rows in (("q_proj", q), ("k_proj", kv), ("v_proj", kv)):
            out.append(ParamSpec(a + proj + ".weight", (rows, H), COL))
            if bias:
                out.append(ParamSpec(a + proj + ".bias", (rows,), COL))
    out.append(ParamSpec(a + "o_proj.weight", (H, q), ROW))
    out += [
        ParamSpec(p + "mlp.gate_proj.weight", (F, H), COL),
        ParamSpec(p + "mlp.up_proj.weight", (F, H), COL),
        ParamSpec(p + "mlp.down_proj.weight", (H, F), ROW),
        ParamSpec(p + "input_layernorm.weight", (H,), REPL),
        ParamSpec(p + "post_attention_layernorm.weight", (H,), REPL),
    ]
    return out


def stage_params(m: ModelSpec, layer_index: int, n_layer: int) -> List[ParamSpec]:
    """Parameters of the stage holding layers [layer_index, layer_index + n_layer)."""
    out: List[ParamSpec] = []
    for L in range(layer_index, layer_index + n_layer):
        out += layer_params(m, L)
    H, V = m.hidden, m.vocab
    if layer_index == 0 and m.embeddings:
        if m.vocab_parallel:
            out.append(ParamSpec("wte.weight", (V, H), VOCAB, (m.pad_multiple,)))
        else:
            out.append(ParamSpec("wte.weight", (V, H), REPL))
        if m.family == "gpt" and m.positions:
            out.append(ParamSpec("wpe.weight", (m.positions, H), REPL))
    if layer_index + n_layer == m.n_layer and m.embeddings:
        out.append(ParamSpec("lm_head.weight", (V, H), COL))
        if m.family == "gpt":
            out.append(ParamSpec("lm_head.bias", (V,), COL))
        else:
            out.append(ParamSpec("norm.weight", (H,), REPL))
    return out


def layer_partition(n_layer: int, pp: int) -> List[int]:
    """Layers per stage, remainder to the first stages (plan_config.py:497-533)."""
    return [n_layer // pp + (i < n_layer % pp) for i in range(pp)]


@dataclass(frozen=True)
class Parallel:
    tp: int
    pp: int = 1
    dp: int = 1

    @property
    def world(self) -> int:
        return self.tp * self.pp * self.dp

    def rank(self, pp_i: int, tp_i: int, dp_i: int = 0) -> int:
        return pp_i * (self.dp * self.tp) + dp_i * self.tp + tp_i

    def coord(self, rank: int) -> Tuple[int, int, int]:
        """(pp, dp, tp) of a rank (device_mesh.py:11-22 order)."""
        pp_i, rem = divmod(rank, self.dp * self.tp)
        dp_i, tp_i = divmod(rem, self.tp)
        return pp_i, dp_i, tp_i


def param_meta(spec: ParamSpec, tp: int, tp_i: int, dtype: torch.dtype) -> TensorMeta:
    """TensorMeta of one rank's shard (TP attrs are set even at tp=1, as the
    reference does: tensor_parallel.py:495-503)."""
    if spec.kind == REPL:
        return TensorMeta(name=spec.name, dtype=dtype, shape=spec.shape)
    if spec.kind == COL:
        return TensorMeta(name=spec.name, dtype=dtype, shape=spec.shape, tp_meta=(0, tp_i, tp))
    if spec.kind == ROW:
        return TensorMeta(name=spec.name, dtype=dtype, shape=spec.shape, tp_meta=(-1, tp_i, tp))
    if spec.kind == VOCAB:
        return TensorMeta(name=spec.name, dtype=dtype, shape=spec.shape, tp_meta=(0, tp_i, tp),
                          kind=VOCAB_PAD, kind_args=spec.kind_args)
    if spec.kind == QKV:
        return TensorMeta(name=spec.name, dtype=dtype, shape=spec.shape, tp_meta=(0, tp_i, tp),
                          kind=QKV_HEADS, kind_args=spec.kind_args)
    raise AssertionError(f"unknown kind {spec.kind}")


def rank_params(m: ModelSpec, par: Parallel, rank: int) -> List[ParamSpec]:
    pp_i, _, _ = par.coord(rank)
    part = layer_partition(m.n_layer, par.pp)
    return stage_params(m, sum(part[:pp_i]), part[pp_i])


def check_divisible(spec: ParamSpec, tp: int) -> None:
    """A TP split must be exact, as ColumnParallelLinear / RowParallelLinear
    allocate ``features // tp`` rows or columns (tensor_parallel.py:189-204,
    368-381)."""
    if spec.kind == COL:
        assert spec.shape[0] % tp == 0, f"{spec.name}: {spec.shape[0]} rows not divisible by tp {tp}"
    elif spec.kind == ROW:
        assert spec.shape[-1] % tp == 0, f"{spec.name}: {spec.shape[-1]} cols not divisible by tp {tp}"
    elif spec.kind == QKV:
        n_q, n_kv, _ = spec.kind_args
        assert n_q % tp == 0 and n_kv % tp == 0, \
            f"{spec.name}: {n_q} q / {n_kv} kv heads not divisible by tp {tp}"


def build_layout(m: ModelSpec, par: Parallel, dtype: torch.dtype) -> ParamLayout:
    """ParamLayout of every rank of a plan (what ParamLayout.gather collects)."""
    metas: Dict[int, Dict[str, TensorMeta]] = {}
    for rank in range(par.world):
        _, _, tp_i = par.coord(rank)
        specs = rank_params(m, par, rank)
        for s in specs:
            check_divisible(s, par.tp)
        metas[rank] = {s.name: param_meta(s, par.tp, tp_i, dtype) for s in specs}
    return ParamLayout.from_metas(metas)


def set_tp_attrs(param: torch.Tensor, spec: ParamSpec, tp: int, tp_i: int) -> None:
    """The attributes TensorMeta(tensor) reads: the reference's slice_dim /
    tp_index / tp_deg (tensor_parallel.py:255-261, 435-441) and, for the
    build's extra kinds, shard_kind with its arguments."""
    if spec.kind == REPL:
        return
    param.slice_dim = -1 if spec.kind == ROW else 0
    param.tp_index = tp_i
    param.tp_deg = tp
    if spec.kind == VOCAB:
        param.shard_kind = VOCAB_PAD
        param.vocab_size = spec.shape[0]
        param.pad_multiple = spec.kind_args[0]
    elif spec.kind == QKV:
        param.shard_kind = QKV_HEADS
        param.qkv_heads = tuple(spec.kind_args)


def build_module(m: ModelSpec, par: Parallel, rank: int, dtype: torch.dtype = torch.float32,
                 device="cpu") -> "torch.nn.Module":
    """An nn.Module holding one rank's shard of every parameter, with the
    reference's names, registration order and TP attributes -- the state a
    Suika stage model exposes to the migration API (``named_parameters`` /
    ``state_dict``).  Values are uninitialised."""
    import torch.nn as nn

    _, _, tp_i = par.coord(rank)
    root = nn.Module()
    for spec in rank_params(m, par, rank):
        check_divisible(spec, par.tp)
        meta = param_meta(spec, par.tp, tp_i, dtype)
        *path, leaf = spec.name.split(".")
        mod = root
        for part in path:
            child = mod._modules.get(part)
            if child is None:
                child = nn.Module()
                mod.add_module(part, child)
            mod = child
        p = nn.Parameter(torch.empty(tuple(meta.actual_shape()), dtype=dtype, device=device))
        set_tp_attrs(p, spec, par.tp, tp_i)
        mod.register_parameter(leaf, p)
    return root

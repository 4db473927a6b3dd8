"""Every element type the C ABI accepts, through the drop-in operator (GPU)
and through a numpy execution of the product plan (CPU).

A column-parallel [6, 10], a row-parallel [6, 14] (7-element runs, so no
16-byte vectors apply on the strided side) and a replicated [9] tensor are
merged TP2 -> TP1 and split TP1 -> TP2, both routes.  The expected shards
are torch's own ``chunk`` / ``cat`` of the global tensors on the CPU
(Suika/migration.py:304-310, 536), compared bit for bit.
"""
import numpy as np
import pytest
import torch

from suika_amd import ParamLayout, TensorMeta, execute_param_transfer, schedule_param_transfer
from suika_amd.plan import ReshardPlan, SlotSpec
from tests.harness import simulate_plan
from tests.test_plan import _esize

DTYPES = [torch.uint8, torch.int8, torch.bool, torch.bfloat16, torch.float16, torch.float32,
          torch.float64, torch.int32, torch.int64]
SHAPES = {"w_col": ((6, 10), 0), "w_row": ((6, 14), -1), "bias": ((9,), None)}
FIELDS = ("param", "exp_avg")


def _global(dtype, seed):
    gen = torch.Generator("cpu").manual_seed(seed)
    out = {}
    for name, (shape, _) in SHAPES.items():
        ent = {}
        for f in FIELDS:
            if dtype.is_floating_point:
                ent[f] = torch.randn(shape, generator=gen).to(dtype)
            elif dtype == torch.bool:
                ent[f] = torch.randint(0, 2, shape, generator=gen).bool()
            else:
                info = torch.iinfo(dtype)
                ent[f] = torch.randint(max(info.min, -2**31), min(info.max, 2**31 - 1), shape,
                                       generator=gen, dtype=torch.int64).to(dtype)
        out[name] = ent
    return out


def _metas(dtype, tp):
    layout = {}
    for r in range(tp):
        layout[r] = {name: TensorMeta(name=name, dtype=dtype, shape=shape,
                                      tp_meta=None if dim is None else (dim, r, tp))
                     for name, (shape, dim) in SHAPES.items()}
    return ParamLayout.from_metas(layout)


def _shard(t, dim, r, tp):
    return t if dim is None else t.chunk(tp, dim)[r].contiguous()


CASES = [(2, 1, 0), (1, 2, 1)]


@pytest.mark.parametrize("src_tp,dst_tp,dst_rank", CASES)
@pytest.mark.parametrize("dtype", DTYPES, ids=[str(d).replace("torch.", "") for d in DTYPES])
def test_dtype_plan_simulation(dtype, src_tp, dst_tp, dst_rank):
    """The host plan (regions, buffer layout) executed byte-wise with numpy."""
    glob = _global(dtype, seed=src_tp * 10 + dst_tp)
    ops = [op for op in schedule_param_transfer(_metas(dtype, src_tp), _metas(dtype, dst_tp))
           if op.dst_rank == dst_rank]
    srcs = {r: {name: {f: _shard(glob[name][f], SHAPES[name][1], r, src_tp).view(torch.uint8).numpy()
                       for f in FIELDS} for name in SHAPES} for r in range(src_tp)}
    specs = {(op.src_rank, op.param_name, f): SlotSpec(tuple(op.src_meta.actual_shape()), dtype)
             for op in ops for f in FIELDS}
    plan = ReshardPlan(ops, specs, list(FIELDS))
    got = simulate_plan(plan, srcs, _esize)
    plan.close()
    for name, (shape, dim) in SHAPES.items():
        for f in FIELDS:
            want = _shard(glob[name][f], dim, dst_rank, dst_tp).view(torch.uint8).numpy()
            np.testing.assert_array_equal(got[(name, f)].view(np.uint8).reshape(want.shape), want,
                                          err_msg=f"{name}/{f}")


@pytest.mark.gpu
@pytest.mark.parametrize("route", ["direct", "buffers"])
@pytest.mark.parametrize("src_tp,dst_tp,dst_rank", CASES)
@pytest.mark.parametrize("dtype", DTYPES, ids=[str(d).replace("torch.", "") for d in DTYPES])
def test_dtype_reshard(dtype, src_tp, dst_tp, dst_rank, route):
    print(f"[gpu dtypes] {dtype} tp{src_tp}->tp{dst_tp} rank {dst_rank} {route}", flush=True)
    glob = _global(dtype, seed=src_tp * 10 + dst_tp)
    ops = schedule_param_transfer(_metas(dtype, src_tp), _metas(dtype, dst_tp))
    fake = {r: {name: {f: _shard(glob[name][f], SHAPES[name][1], r, src_tp).cuda() for f in FIELDS}
                for name in SHAPES}
            for r in range(src_tp)}
    out = execute_param_transfer(ops, {}, torch.device("cuda", 0), [(f, "normal") for f in FIELDS],
                                 rank=dst_rank, fake_source_state_dicts=fake, route=route)
    torch.cuda.synchronize()
    assert set(out) == set(SHAPES)
    for name, (shape, dim) in SHAPES.items():
        for f in FIELDS:
            want = _shard(glob[name][f], dim, dst_rank, dst_tp)
            got = out[name][f].cpu()
            assert got.dtype == dtype and got.shape == want.shape, (name, f, got.dtype, got.shape)
            assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), (name, f)

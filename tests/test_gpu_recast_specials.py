"""The fused f32 -> bf16 recast on the GPU with IEEE special values.

A bf16 ``param`` is rounded from the f32 ``master`` while both are resharded
TP2 -> TP1 (``recast={"param": "master"}``).  The masters hold the values
where a rounding routine goes wrong: signed zeros, the smallest and largest
subnormals, infinities, quiet and signalling NaNs of both signs with
payloads, the largest finite value and its neighbours (which round to
infinity or stay finite), ties at even and odd mantissas, and mantissa carries
into the exponent.  Three tensors reach both lane widths of the kernel:

* ``w_col`` [8, 64], split by rows: 1 KiB contiguous pieces, 16-byte aligned,
  four f32 per lane;
* ``w_row`` [6, 14], split by columns: strided 7-element (28-byte) runs, one
  f32 per lane;
* ``v_odd`` [37], replicated: a 148-byte piece (not a multiple of 16 bytes),
  one f32 per lane.

Expected bits: torch's CPU ``.to(torch.bfloat16)`` (round to nearest, ties to
even).  Torch converts element by element (a 0-dim or strided tensor) to the
quiet NaN 0x7FC0 for every NaN input, and its vectorised loop over a
contiguous tensor to 0xFFFF; the kernel, like the oracle's ``rne_bf16``,
gives the element conversion's result, so every bit is compared with a
strided conversion and every non-NaN bit with the contiguous one as well.
The f32 copy must keep every bit, NaN payloads included.
"""
import numpy as np
import pytest
import torch

from oracle import reshard_oracle as O
from suika_amd import ParamLayout, TensorMeta, execute_param_transfer, schedule_param_transfer
from tests.harness import t2np

pytestmark = pytest.mark.gpu

SPECIALS = np.array([
    0x00000000, 0x80000000,                          # +0, -0
    0x00000001, 0x80000001, 0x007FFFFF, 0x807FFFFF,  # smallest / largest subnormals
    0x00008000, 0x00018000, 0x00007FFF,              # subnormal ties and below
    0x7F800000, 0xFF800000,                          # +inf, -inf
    0x7FC00000, 0xFFC00000, 0x7FC12345, 0xFFD00001,  # quiet NaNs with payloads
    0x7F800001, 0xFF800001, 0x7FA00000, 0xFFBFFFFF,  # signalling NaNs
    0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F7FFF, 0x7F7F8000,  # max finite and neighbours
    0x7F7F8001, 0x7F7EFFFF,
    0x3F808000, 0x3F818000, 0x3F80FFFF, 0x3F807FFF,  # ties at even / odd, just below / above
    0x3FFFFFFF, 0x3FFF8000, 0x407FFFFF, 0x00FFFFFF,  # mantissa carries into the exponent
    0x3F800000, 0xBF800000, 0x33800000, 0xC0490FDB,  # ordinary values
], dtype=np.uint32)

SHAPES = {"w_col": ((8, 64), 0), "w_row": ((6, 14), -1), "v_odd": ((37,), None)}


def _master(shape, seed):
    """Special values first, then random bit patterns of finite numbers."""
    n = int(np.prod(shape))
    rng = np.random.default_rng(seed)
    fill = rng.integers(0, 2 ** 32, size=n, dtype=np.uint64).astype(np.uint32)
    fill = np.where(np.isfinite(fill.view(np.float32)), fill, np.uint32(0x3F800000))
    k = min(n, len(SPECIALS))
    fill[:k] = SPECIALS[(np.arange(k) + seed) % len(SPECIALS)]
    return fill.reshape(shape)


def _layout(tp):
    return ParamLayout.from_metas({
        r: {name: TensorMeta(name=name, dtype=torch.float32, shape=shape,
                             tp_meta=None if dim is None else (dim, r, tp))
            for name, (shape, dim) in SHAPES.items()} for r in range(tp)})


def _shard(a, dim, r, tp):
    return a if dim is None else np.ascontiguousarray(np.array_split(a, tp, axis=dim)[r])


@pytest.mark.parametrize("route", ["direct", "buffers"])
def test_recast_special_values_both_lane_widths(route):
    print(f"[gpu recast specials] route={route}", flush=True)
    glob = {name: {"master": _master(shape, seed), "exp_avg": _master(shape, seed + 7)}
            for seed, (name, (shape, _)) in enumerate(SHAPES.items())}
    ops = schedule_param_transfer(_layout(2), _layout(1))
    fake = {r: {name: {f: torch.from_numpy(_shard(glob[name][f], dim, r, 2).view(np.int32)).view(torch.float32).cuda()
                       for f in ("master", "exp_avg")}
                for name, (_, dim) in SHAPES.items()} for r in range(2)}
    out = execute_param_transfer(ops, {}, torch.device("cuda"), [("master", "normal"), ("exp_avg", "normal")],
                                 rank=0, fake_source_state_dicts=fake, recast={"param": "master"}, route=route)
    torch.cuda.synchronize()
    seen_nan = 0
    for name in SHAPES:
        master = glob[name]["master"]
        np.testing.assert_array_equal(t2np(out[name]["master"]), master, err_msg=f"{name}/master bits")
        np.testing.assert_array_equal(t2np(out[name]["exp_avg"]), glob[name]["exp_avg"], err_msg=f"{name}/exp_avg")
        got = t2np(out[name]["param"])
        assert out[name]["param"].dtype == torch.bfloat16
        flat = torch.from_numpy(master.reshape(-1).view(np.float32).copy())
        elementwise = t2np(torch.stack([flat, flat], 1)[:, 0].to(torch.bfloat16)).reshape(master.shape)
        contiguous = t2np(flat.to(torch.bfloat16)).reshape(master.shape)
        nan = np.isnan(master.view(np.float32))
        np.testing.assert_array_equal(got, elementwise, err_msg=f"{name}/param vs torch (element conversion)")
        np.testing.assert_array_equal(got[~nan], contiguous[~nan], err_msg=f"{name}/param vs torch (vectorised)")
        np.testing.assert_array_equal(got, O.rne_bf16(master), err_msg=f"{name}/param vs oracle")
        assert np.all(got[nan] == 0x7FC0)
        seen_nan += int(nan.sum())
    assert seen_nan >= 3 * 8, "every tensor carries the NaN patterns"

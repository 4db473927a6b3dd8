"""Full-size benchmark reshards on the GPU, checked by a size-independent
property: every destination element holds the code of its global position.

Sources are index-coded on the GPU from the oracle's closed-form shard maps
(``shard_index``): element bits = f(tensor, field, global flat index), unique
within a tensor.  After pack + unpack, each destination tensor must equal the
codes of its own closed-form index map, pad rows must be zero, and a recast
``param`` must be the bf16 rounding of the destination ``master``.  Any
misrouted, dropped or duplicated element changes a code.  The direct gather
and the drop-in ``execute_param_transfer`` (in launch groups) must then
reproduce the same bytes.
"""
import pytest
import torch

from oracle import reshard_oracle as O
from suika_amd import execute_param_transfer
from suika_amd.plan import ReshardPlan, SlotSpec
from suika_amd.workloads import CONFIG_ORDER, CONFIGS
from tests.harness import poisoned_allocations, to_olayout

pytestmark = pytest.mark.gpu

FIELD_ID = {"param": 0, "master": 1, "exp_avg": 2, "exp_avg_sq": 3}


def code(gidx: torch.Tensor, tid: int, field: str, dtype: torch.dtype) -> torch.Tensor:
    """Index code of a tensor of ``dtype``; pad positions (gidx < 0) are 0."""
    salt = (tid * 7919 + FIELD_ID[field] * 104729) & 0xFFFFFFFF
    pad = gidx < 0
    if dtype.itemsize == 2:
        x = (gidx * 40503 + salt) & 0xFFFF
        x = x - ((x >> 15) << 16)
        out = x.to(torch.int16)
    else:
        x = 0x10000000 + torch.remainder(gidx + salt, 1 << 30)
        out = x.to(torch.int32)
    out.masked_fill_(pad, 0)
    return out.view(dtype)


@pytest.mark.parametrize("key", CONFIG_ORDER)
def test_fullsize_index_coded(key):
    w = CONFIGS[key]
    print(f"[gpu fullsize] {key}: planning", flush=True)
    dev = torch.device("cuda")
    ops = w.ops()
    dt = w.dtypes
    specs = {(op.src_rank, op.param_name, f): SlotSpec(tuple(op.src_meta.actual_shape()), dt[f])
             for op in ops for f in w.src_fields}
    plan = ReshardPlan(ops, specs, list(w.src_fields), recast=w.recast_map)
    spl, tpl = w.layouts()
    osrc, odst = to_olayout(spl), to_olayout(tpl)
    names = sorted({n for metas in spl.layout.values() for n in metas})
    tid = {n: i for i, n in enumerate(names)}

    sources = {}
    for (r, name, f) in plan.src_keys:
        gidx = O.shard_index(osrc[r][name], xp=torch, device=dev)
        sources.setdefault(r, {}).setdefault(name, {})[f] = code(gidx, tid[name], f, dt[f]).contiguous()
        del gidx
    bufs = plan.alloc_buffers(dev)
    dst = plan.alloc_dst(dev)
    for e in dst.values():
        for t in e.values():
            t.view(torch.uint8).fill_(0xA5)
    print(f"[gpu fullsize] {key}: {len(plan.src_keys)} sources, {plan.n_pieces} pieces, "
          f"{sum(plan.peer_bytes) / 1e9:.2f} GB buffers; pack+unpack", flush=True)
    plan.pack(sources, bufs)
    plan.unpack(bufs, dst)
    torch.cuda.synchronize()
    del bufs
    # the direct route into a second destination set must agree bit for bit
    dst2 = plan.alloc_dst(dev)
    for e in dst2.values():
        for t in e.values():
            t.view(torch.uint8).fill_(0x5A)
    plan.gather(sources, dst2)
    torch.cuda.synchronize()

    recast = w.recast_map
    bad = []
    for (name, f) in plan.dst_keys:
        if not torch.equal(dst[name][f].view(torch.uint8), dst2[name][f].view(torch.uint8)):
            bad.append((name, f, "gather"))
    del dst2
    # the drop-in operator (launch groups planned while the GPU runs, poisoned
    # destinations) must agree bit for bit as well
    print(f"[gpu fullsize] {key}: execute_param_transfer", flush=True)
    with poisoned_allocations() as poisoned:
        out = execute_param_transfer(ops, {}, dev, [(f, "normal") for f in w.src_fields],
                                     rank=w.dst_rank, fake_source_state_dicts=sources, recast=recast)
    torch.cuda.synchronize()
    assert poisoned["tensors"] >= sum(len(e) for e in out.values()), "destinations were not poisoned"
    for (name, f) in plan.dst_keys:
        if not torch.equal(dst[name][f].view(torch.uint8), out[name][f].view(torch.uint8)):
            bad.append((name, f, "execute_param_transfer"))
    del out, sources
    for (name, f) in plan.dst_keys:
        gidx = O.shard_index(odst[w.dst_rank][name], xp=torch, device=dev)
        if f in recast:
            master = code(gidx, tid[name], recast[f], torch.float32)
            want = master.to(torch.bfloat16)
            want.masked_fill_(gidx < 0, 0)
        else:
            want = code(gidx, tid[name], f, dt[f])
        got = dst[name][f]
        if not torch.equal(got.view(torch.int16 if got.dtype.itemsize == 2 else torch.int32),
                           want.view(torch.int16 if want.dtype.itemsize == 2 else torch.int32)):
            bad.append((name, f))
        del gidx, want
    plan.close()
    assert not bad, f"{key}: {len(bad)} destination tensors differ, first {bad[:5]}"
    print(f"[gpu fullsize] {key}: {len(plan.dst_keys)} destination tensors exact", flush=True)

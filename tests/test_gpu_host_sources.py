"""Sources in host memory and results for the host, on the GPU engine.

The reference's checkpoint_load calls execute_param_transfer with the loaded
state dicts in host memory as fake sources and ``device="cpu"``
(Suika/migration.py:1235-1244); its fake-source loop slices each host
tensor and moves the piece with ``.to(device)`` (:477-482, 583).  Here the
pieces' bytes are packed by host threads into pinned windows and copied to
HBM peer buffers (sr_stage_pack), the GPU unpacks them, and a host result
comes back through the same windows (sr_download).  Every result must equal
the oracle's reshard of the same seeded shards (or, for the wide synthetic
case, torch.cat of the shards on the CPU), bit for bit.
"""
import numpy as np
import pytest
import torch

from suika_amd import _lib, execute_param_transfer
from suika_amd.meta import TensorMeta
from suika_amd.plan import ReshardPlan, download
from tests.harness import global_state, oracle_dest, payload_spans, source_shards, t2np, to_device
from tests.test_reference_objects import SMALL_CASES, _ref_ops
from tests.test_stage_host import _esize, _wide_ops, _wide_sources

pytestmark = pytest.mark.gpu


def _state(w):
    spl, _ = w.layouts()
    glob = global_state(w, {n for metas in spl.layout.values() for n in metas})
    srcs = source_shards(w, sorted(spl.layout), glob)
    return srcs, oracle_dest(w, srcs)


def _with_step(fake):
    """AdamW's 1-element ``step`` beside every tensor, a different value per
    source rank, as a merged state dict holds it (migration.py:675-711)."""
    for r, sd in fake.items():
        for name, ent in sd.items():
            items = list(ent.items())
            ent.clear()
            ent[items[0][0]] = items[0][1]
            ent["step"] = torch.tensor(float(r + 3))
            ent.update(items[1:])
    return fake


def _sub_fields(w):
    """expected_sub_fields as the reference's merge records them: param,
    step (a TensorMeta: numel 1), then the other normal fields."""
    fields = list(w.src_fields)
    return [(fields[0], "normal"), ("step", TensorMeta(torch.tensor(0.0)))] + [(f, "normal") for f in fields[1:]]


def _compare(case, out, want, device_type):
    assert set(out) == set(want), case
    for name, ent in want.items():
        for f, a in ent.items():
            t = out[name][f]
            assert t.device.type == device_type, f"{case}: {name}/{f} on {t.device}"
            np.testing.assert_array_equal(t2np(t), a, err_msg=f"{case}: {name}/{f}")


@pytest.mark.parametrize("case", SMALL_CASES)
def test_checkpoint_call_with_host_state_and_host_result(case):
    """The call of migration.py:1235-1244 on the reference's own ops: host
    fake sources (self source = this rank's entry), device="cpu", a scalar
    sub-field; the caller's source dict is cleared."""
    w, _, _, ref_ops = _ref_ops(case, omit_tp=True)
    print(f"[gpu host sources] {case} device=cpu", flush=True)
    srcs, want = _state(w)
    fake = _with_step(to_device(srcs, w, "cpu"))
    rank = w.dst_rank
    self_source = fake[rank] if rank in fake else {}
    # the reference's keywords; a workload whose bf16 param is rounded from
    # master also names that recast (this build's extension)
    extra = {"recast": w.recast_map} if w.recast_map else {}
    out = execute_param_transfer(ref_ops, self_source, "cpu", _sub_fields(w), rank=rank,
                                 forcefully_free=False, fake_source_state_dicts=fake, **extra)
    assert self_source == {}, "source_state_dict is cleared in place"
    _compare(case, {n: {f: t for f, t in e.items() if f != "step"} for n, e in out.items()}, want, "cpu")
    first = {}
    for op in ref_ops:
        if op.dst_rank == rank:
            first.setdefault(op.param_name, op.src_rank)
    for name, ent in out.items():
        assert ent["step"].device.type == "cpu" and float(ent["step"]) == first[name] + 3, name
        if not w.recast_map:
            assert list(ent)[:2] == [w.src_fields[0], "step"], "sub-fields keep the merge order"


@pytest.mark.parametrize("route", ["direct", "buffers"])
@pytest.mark.parametrize("case", SMALL_CASES[::3])
def test_host_sources_to_gpu_result(case, route):
    """Host sources with device="cuda" (the on-load of migration.py:583):
    the state arrives in HBM; the route asked for does not matter."""
    w, _, _, ref_ops = _ref_ops(case, omit_tp=True)
    print(f"[gpu host sources] {case} device=cuda route={route}", flush=True)
    srcs, want = _state(w)
    fake = to_device(srcs, w, "cpu")
    before = _lib.stage_counters().host_piece_bytes
    out = execute_param_transfer(ref_ops, {}, torch.device("cuda"), [(f, "normal") for f in w.src_fields],
                                 rank=w.dst_rank, fake_source_state_dicts=fake, route=route,
                                 arena=case == SMALL_CASES[0], recast=w.recast_map)
    torch.cuda.synchronize()
    _compare(case, out, want, "cuda")
    # exactly the pieces' bytes went up: P of this rank's plan
    staged = _lib.stage_counters().host_piece_bytes - before
    plan, _ = ReshardPlan.from_sources([op for op in ref_ops if op.dst_rank == w.dst_rank], lambda r: fake[r],
                                       list(w.src_fields), torch.device("cuda", 0), recast=w.recast_map,
                                       rank=w.dst_rank, host_ok=True)
    try:
        assert staged == plan.info.pack_bytes_read
    finally:
        plan.close()


def test_mixed_residency_sources():
    """One source rank in HBM, the others in host memory: device pieces are
    copied on the device, host pieces staged, in one plan."""
    case = next(c for c in SMALL_CASES if "tp4pp1_tp2pp1" in c or "tp2pp1_tp4pp1" in c)
    w, _, _, ref_ops = _ref_ops(case, omit_tp=True)
    srcs, want = _state(w)
    ranks = sorted(srcs)
    fake = {r: to_device({r: srcs[r]}, w, "cuda" if i == 0 else "cpu")[r] for i, r in enumerate(ranks)}
    for device in ("cuda", "cpu"):
        print(f"[gpu host sources] mixed {case} device={device}", flush=True)
        out = execute_param_transfer(ref_ops, {}, device, [(f, "normal") for f in w.src_fields],
                                     rank=w.dst_rank, fake_source_state_dicts=fake, recast=w.recast_map)
        torch.cuda.synchronize()
        _compare(case, out, want, device)


def test_staged_buffers_equal_the_device_pack():
    """sr_stage_pack from host memory writes every payload byte sr_pack
    writes from the same contents on the device."""
    print("[gpu host sources] stage vs pack buffers", flush=True)
    host = _wide_sources()
    dev = {r: {n: {f: t.cuda() for f, t in e.items()} for n, e in sd.items()} for r, sd in host.items()}
    plan_h, ptrs_h = ReshardPlan.from_sources(_wide_ops(), lambda r: host[r], ["param"], torch.device("cuda", 0),
                                              rank=0, host_ok=True)
    plan_d, ptrs_d = ReshardPlan.from_sources(_wide_ops(), lambda r: dev[r], ["param"], torch.device("cuda", 0),
                                              rank=0)
    try:
        assert plan_h.peer_bytes == plan_d.peer_bytes
        bh = plan_h.alloc_buffers("cuda")
        bd = plan_d.alloc_buffers("cuda")
        before = _lib.stage_counters()
        plan_h.stage_pack_ptrs(ptrs_h, [b.data_ptr() for b in bh])
        plan_d.pack_ptrs(ptrs_d, [b.data_ptr() for b in bd])
        torch.cuda.synchronize()
        after = _lib.stage_counters()
        n = 0
        for peer, off, nbytes in payload_spans(plan_h, _esize):
            assert torch.equal(bh[peer][off:off + nbytes], bd[peer][off:off + nbytes]), (peer, off)
            n += nbytes
        assert after.host_piece_bytes - before.host_piece_bytes == n
        assert n <= after.host_bytes_up - before.host_bytes_up <= n + 256 * len(plan_h.pieces)
        assert after.windows - before.windows >= n // _lib.STAGE_WINDOW_BYTES
    finally:
        plan_h.close()
        plan_d.close()


def _wide_expected(host):
    return {"row": torch.cat([host[0]["row"]["param"], host[1]["row"]["param"]], dim=-1),
            "col": torch.cat([host[0]["col"]["param"], host[1]["col"]["param"]], dim=0),
            "rep": host[1]["rep"]["param"]}


@pytest.mark.parametrize("threads", [1, 0])
@pytest.mark.parametrize("device", ["cpu", "cuda"])
def test_wide_transfer_through_many_windows(device, threads):
    """88 MB of pieces and of results, more than the four 16 MiB windows:
    the ring wraps in both directions; the result equals torch.cat of the
    shards on the CPU."""
    print(f"[gpu host sources] wide device={device} threads={threads}", flush=True)
    host = _wide_sources()
    L = _lib.lib()
    assert L.sr_set_host_threads(threads) == _lib.SR_OK
    try:
        out = execute_param_transfer(_wide_ops(), {}, device, [("param", "normal")], rank=0,
                                     fake_source_state_dicts=host)
        torch.cuda.synchronize()
    finally:
        assert L.sr_set_host_threads(0) == _lib.SR_OK
    for name, t in _wide_expected(host).items():
        got = out[name]["param"]
        assert got.device.type == device
        assert torch.equal(got.cpu(), t), name


def test_download_regions():
    """sr_download: regions of one device allocation (adjacent ones copied
    together) into separate host tensors, larger than the ring."""
    print("[gpu host sources] download regions", flush=True)
    g = torch.Generator(device="cuda").manual_seed(9)
    big = torch.randint(0, 256, (80 << 20,), dtype=torch.uint8, device="cuda", generator=g)
    cuts = [0, 1, 4096, 4096 + 17, 9 << 20, 40 << 20, (40 << 20) + 3, 80 << 20]
    pairs = [(big[a:b], torch.empty(b - a, dtype=torch.uint8)) for a, b in zip(cuts[:-1], cuts[1:])]
    before = _lib.stage_counters().bytes_down
    download(pairs)
    for d, h in pairs:
        assert torch.equal(d.cpu(), h)
    assert _lib.stage_counters().bytes_down - before == 80 << 20


def _extension_cases():
    from tests import cases
    out = list(cases.scaled_configs().values())
    pads = cases.padded_vocab_cases()
    out += [pads[0], pads[-1]]
    gold = cases.golden_cases()
    out += [gold["qkv_tp1_tp2_d1"], gold["qkv_tp2_tp1"], gold["vocab_tp2_tp4_d3"]]
    return out


@pytest.mark.parametrize("w", _extension_cases(), ids=lambda w: w.key)
def test_host_sources_extension_kinds(w):
    """The staged route with the build's own layouts: zero-padded vocabulary
    rows (ZERO pieces), head-granular fused QKV, the bf16 recast and the
    five benchmark plan changes at a small shape, from host-resident shards
    to HBM and back to the host, exact against the oracle."""
    srcs, want = _state(w)
    fake = to_device(srcs, w, "cpu")
    fields = [(f, "normal") for f in w.src_fields]
    for device in ("cuda", "cpu"):
        print(f"[gpu host sources] {w.key} device={device}", flush=True)
        out = execute_param_transfer(w.ops(), {}, device, fields, rank=w.dst_rank,
                                     fake_source_state_dicts=fake, recast=w.recast_map)
        torch.cuda.synchronize()
        _compare(w.key, out, want, device)

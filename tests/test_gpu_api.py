"""Reference-shaped API semantics of the GPU path (Suika/migration.py:397-556)
and the boundary's error handling, which rejects bad input before any launch."""
import numpy as np
import pytest
import torch

from suika_amd import PlanError, TensorMeta, TransferOp, execute_param_transfer
from suika_amd.plan import ReshardPlan, SlotSpec
from tests import cases
from tests.harness import global_state, oracle_dest, source_shards, t2np, to_device

pytestmark = pytest.mark.gpu


def _names(w):
    spl, _ = w.layouts()
    return {n for metas in spl.layout.values() for n in metas}


def test_execute_semantics_step_and_clear():
    w = cases.scaled_configs()["llama7b_tp4pp2_tp2pp2"]
    print(f"[gpu api] {w.key}", flush=True)
    glob = global_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    dev = torch.device("cuda")
    fake = to_device(srcs, w, dev)
    step_meta = TensorMeta(torch.tensor(7.0))
    for r, sd in fake.items():
        for name, e in sd.items():
            e["step"] = torch.tensor(float(r + 10))   # CPU scalar, as AdamW keeps it
    own = fake[w.dst_rank] if w.dst_rank in fake else {}
    own_copy = dict(own)
    fields = [("param", "normal"), ("step", step_meta), ("master", "normal"),
              ("exp_avg", "normal"), ("exp_avg_sq", "normal")]
    out = execute_param_transfer(w.ops(), own_copy, dev, fields, rank=w.dst_rank,
                                 fake_source_state_dicts=fake)
    torch.cuda.synchronize()
    assert own_copy == {}, "source_state_dict is cleared in place"
    for name, e in want.items():
        assert list(out[name]) == ["param", "step", "master", "exp_avg", "exp_avg_sq"]
        for f, a in e.items():
            np.testing.assert_array_equal(t2np(out[name][f]), a, err_msg=f"{name}/{f}")
        assert out[name]["step"].device.type == "cuda" and out[name]["step"].numel() == 1


@pytest.mark.parametrize("route", ["direct", "buffers"])
def test_execute_with_no_ops_for_this_rank(route):
    """A rank the schedule sends nothing to (an empty schedule, or one for
    other ranks only) gets an empty state and its own dict cleared, on both
    routes, and the next call is unaffected."""
    w = cases.scaled_configs()["gpt125m_tp2_tp4"]
    print(f"[gpu api] no ops for this rank, {route}", flush=True)
    dev = torch.device("cuda")
    own = {"x": {"param": torch.zeros(4, device=dev)}}
    assert execute_param_transfer([], own, dev, [("param", "normal")], rank=0, route=route) == {}
    assert own == {}
    others = [op for op in w.ops()]      # every op targets w.dst_rank
    stranger = w.dst_rank + 1000
    assert execute_param_transfer(others, {}, dev, [(f, "normal") for f in w.src_fields], rank=stranger,
                                  route=route) == {}
    glob = global_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    out = execute_param_transfer(w.ops(), {}, dev, [(f, "normal") for f in w.src_fields], rank=w.dst_rank,
                                 fake_source_state_dicts=to_device(srcs, w, "cuda"), route=route)
    torch.cuda.synchronize()
    for name, e in want.items():
        for f, a in e.items():
            np.testing.assert_array_equal(t2np(out[name][f]), a, err_msg=f"{name}/{f}")


def test_execute_rejects_remote_without_exchange():
    w = cases.scaled_configs()["llama7b_tp4pp2_tp2pp2"]
    ops = w.ops()
    glob = global_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    own = to_device({w.dst_rank: srcs[w.dst_rank]}, w, "cuda")[w.dst_rank]
    assert any(op.src_rank != w.dst_rank for op in ops)
    with pytest.raises(NotImplementedError, match="cross-GPU exchange"):
        execute_param_transfer(ops, own, torch.device("cuda"), [(f, "normal") for f in w.src_fields],
                               rank=w.dst_rank)
    # a missing own shard is the reference's assertion (migration.py:436)
    with pytest.raises(AssertionError, match="param missing in source"):
        execute_param_transfer(ops, {}, torch.device("cuda"), [("param", "normal")], rank=w.dst_rank)


def test_execute_checks_source_shapes_and_layout():
    """Sources in host memory take the staged route (the reference slices
    them where they live, migration.py:477-482) and match the oracle; a
    source of the wrong shape or a strided one is rejected by name."""
    w = cases.scaled_configs()["gpt125m_tp2_tp4"]
    glob = global_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    cpu = to_device(srcs, w, "cpu")
    fields = [(f, "normal") for f in w.src_fields]
    got = execute_param_transfer(w.ops(), {}, torch.device("cuda"), fields, rank=w.dst_rank,
                                 fake_source_state_dicts=cpu)
    want = oracle_dest(w, srcs)
    assert set(got) == set(want)
    for name, ent in want.items():
        for f, arr in ent.items():
            assert got[name][f].is_cuda and (t2np(got[name][f]) == arr).all(), f"{name}/{f}"
    gpu = to_device(srcs, w, "cuda")
    r = next(iter(gpu))
    name = next(iter(gpu[r]))
    good = gpu[r][name]["param"]
    gpu[r][name]["param"] = good.reshape(-1)[:-1].clone()
    with pytest.raises(AssertionError, match=f"param {name} - src_tensor shape"):
        execute_param_transfer(w.ops(), {}, torch.device("cuda"), fields, rank=w.dst_rank,
                               fake_source_state_dicts=gpu)
    gpu[r][name]["param"] = good
    # a transposed view of the right shape: strided, so rejected by name
    op2 = next(op for op in w.ops() if gpu[op.src_rank][op.param_name]["param"].dim() == 2
               and min(gpu[op.src_rank][op.param_name]["param"].shape) > 1)
    r2, name2 = op2.src_rank, op2.param_name
    gpu[r2][name2]["param"] = gpu[r2][name2]["param"].t().contiguous().t()
    with pytest.raises(AssertionError, match=f"source {name2}/param of rank {r2} is not contiguous"):
        execute_param_transfer(w.ops(), {}, torch.device("cuda"), fields, rank=w.dst_rank,
                               fake_source_state_dicts=gpu)


@pytest.mark.parametrize("groups", [1, 4])
def test_failed_call_frees_its_destinations(groups, monkeypatch):
    """A launch group that fails after its destination blocks went to the
    helper thread (the lowering rejects a source of the wrong shape) leaves
    no device memory behind: torch's allocated bytes return to where they
    were, and the next call on the same sources is exact."""
    from suika_amd import migration as M
    from tests.harness import round_robin_groups
    monkeypatch.setattr(M, "_pipeline_groups", round_robin_groups(groups))
    w = cases.scaled_configs()["gpt125m_tp2_tp4"]
    print(f"[gpu api] failed call frees its destinations, {groups} group(s)", flush=True)
    glob = global_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    gpu = to_device(srcs, w, "cuda")
    fields = [(f, "normal") for f in w.src_fields]
    ops = w.ops()
    last = ops[-1]                                # in the last group of the round robin
    good = gpu[last.src_rank][last.param_name]["exp_avg"]
    gpu[last.src_rank][last.param_name]["exp_avg"] = good.reshape(-1)[:-1].clone()
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    with pytest.raises(AssertionError, match=f"param {last.param_name} - src_tensor shape"):
        execute_param_transfer(ops, {}, torch.device("cuda"), fields, rank=w.dst_rank,
                               fake_source_state_dicts={r: {n: dict(e) for n, e in sd.items()}
                                                        for r, sd in gpu.items()})
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before
    gpu[last.src_rank][last.param_name]["exp_avg"] = good
    out = execute_param_transfer(ops, {}, torch.device("cuda"), fields, rank=w.dst_rank,
                                 fake_source_state_dicts=gpu)
    torch.cuda.synchronize()
    for name, e in want.items():
        for f, a in e.items():
            np.testing.assert_array_equal(t2np(out[name][f]), a, err_msg=f"{name}/{f}")


def test_execute_rejects_one_tensor_with_two_source_dtypes():
    """The two sources of one tensor hold uint8 and int8: the library sees
    one byte type, so the drop-in call's planner itself checks that the
    torch dtype of a (tensor, field) agrees across sources, and names it."""
    dst = TensorMeta(name="a", dtype=torch.uint8, shape=(64, 32), tp_meta=(0, 0, 1))
    ops = [TransferOp("a", r, 0, TensorMeta(name="a", dtype=torch.uint8, shape=(64, 32), tp_meta=(0, r, 2)),
                      TensorMeta(name="a", dtype=torch.uint8, shape=(64, 32), tp_meta=(0, r, 2)), dst)
           for r in (0, 1)]
    dev = torch.device("cuda")
    fake = {0: {"a": {"param": torch.zeros((32, 32), dtype=torch.uint8, device=dev)}},
            1: {"a": {"param": torch.zeros((32, 32), dtype=torch.int8, device=dev)}}}
    print("[gpu api] two source dtypes", flush=True)
    for route in ("direct", "buffers"):
        with pytest.raises(AssertionError, match="a/param: dtype differs between sources"):
            execute_param_transfer(ops, {}, dev, [("param", "normal")], rank=0, fake_source_state_dicts=fake,
                                   route=route)
    fake[1]["a"]["param"] = torch.ones((32, 32), dtype=torch.uint8, device=dev)
    out = execute_param_transfer(ops, {}, dev, [("param", "normal")], rank=0, fake_source_state_dicts=fake)
    torch.cuda.synchronize()
    want = torch.cat([torch.zeros((32, 32), dtype=torch.uint8), torch.ones((32, 32), dtype=torch.uint8)])
    assert torch.equal(out["a"]["param"].cpu(), want)


def test_boundary_rejects_misaligned_and_null_pointers():
    src = TensorMeta(name="a", dtype=torch.float32, shape=(64, 32), tp_meta=(0, 0, 2))
    dst = TensorMeta(name="a", dtype=torch.float32, shape=(64, 32), tp_meta=(0, 0, 1))
    ops = [TransferOp("a", 0, 0, src, TensorMeta(name="a", dtype=torch.float32, shape=(64, 32),
                                                 tp_meta=(0, 0, 2)), dst),
           TransferOp("a", 1, 0, TensorMeta(name="a", dtype=torch.float32, shape=(64, 32),
                                            tp_meta=(0, 1, 2)),
                      TensorMeta(name="a", dtype=torch.float32, shape=(64, 32), tp_meta=(0, 1, 2)), dst)]
    specs = {(0, "a", "param"): SlotSpec((32, 32), torch.float32),
             (1, "a", "param"): SlotSpec((32, 32), torch.float32)}
    plan = ReshardPlan(ops, specs, ["param"])
    s0 = torch.randn(32, 32, device="cuda")
    s1 = torch.randn(32, 32, device="cuda")
    bufs = plan.alloc_buffers("cuda")
    bp = plan.buf_pointers(bufs)
    with pytest.raises(PlanError, match="aligned"):
        plan.pack_ptrs([s0.data_ptr() + 2, s1.data_ptr()], bp)
    with pytest.raises(PlanError, match="aligned"):
        plan.pack_ptrs([s0.data_ptr(), s1.data_ptr()], [bp[0] + 8, bp[1]])
    with pytest.raises(PlanError, match="null"):
        plan.pack_ptrs([0, s1.data_ptr()], bp)
    # the valid call still works after the rejected ones
    dst_t = plan.alloc_dst("cuda")
    plan.pack({0: {"a": {"param": s0}}, 1: {"a": {"param": s1}}}, bufs)
    plan.unpack(bufs, dst_t)
    torch.cuda.synchronize()
    assert torch.equal(dst_t["a"]["param"], torch.cat([s0, s1], 0))
    plan.close()


@pytest.mark.gpu
@pytest.mark.parametrize("groups", ["one", "many"])
@pytest.mark.parametrize("route", ["direct", "buffers"])
def test_arena_destinations_and_adoption(route, groups, monkeypatch):
    """execute_param_transfer(arena=True): bit-identical to the oracle, every
    destination a view of one allocation -- also when the transfer runs as
    several launch groups -- and a stage module adopting the params with
    load_state_dict(assign=True) keeps them in place (no copy)."""
    if groups == "many":
        from suika_amd import migration
        from tests.harness import round_robin_groups
        monkeypatch.setattr(migration, "_pipeline_groups", round_robin_groups(4))
    from suika_amd.inventory import build_module
    from tests.cases import scaled_configs
    from tests.harness import index_state, oracle_dest, source_shards, t2np, to_device

    w = scaled_configs()["llama7b_tp4pp2_tp2pp2"]
    print(f"[gpu api] arena {w.key} {route}", flush=True)
    names = {n for metas in w.layouts()[0].layout.values() for n in metas}
    srcs = source_shards(w, sorted(w.layouts()[0].layout), index_state(w, names))
    want = oracle_dest(w, srcs)
    out = execute_param_transfer(w.ops(), {}, torch.device("cuda", 0),
                                 [(f, "normal") for f in w.src_fields], rank=w.dst_rank,
                                 fake_source_state_dicts=to_device(srcs, w, "cuda"),
                                 recast=w.recast_map, route=route, arena=True)
    torch.cuda.synchronize()
    storages = {t.untyped_storage().data_ptr() for e in out.values() for t in e.values()}
    assert len(storages) == 1
    for name, ent in want.items():
        for f, a in ent.items():
            np.testing.assert_array_equal(t2np(out[name][f]), a, err_msg=f"{name}/{f}")
    module = build_module(w.model, w.dst, w.dst_rank, w.dtypes["param"], "cuda")
    module.load_state_dict({n: e["param"] for n, e in out.items()}, assign=True)
    for n, p in module.named_parameters():
        assert p.data_ptr() == out[n]["param"].data_ptr(), n


@pytest.mark.gpu
@pytest.mark.parametrize("route", ["direct", "buffers"])
def test_zero_element_tensors(route):
    from tests.test_plan import _empty_case
    print(f"[gpu api] zero-element tensors {route}", flush=True)
    ops = _empty_case(2, 1)
    gen = torch.Generator("cpu").manual_seed(3)
    w = torch.randn((8, 4), generator=gen)
    fake = {r: {"w": {"param": w.chunk(2, 0)[r].contiguous().cuda()},
                "none": {"param": torch.empty(0, device="cuda")},
                "none2d": {"param": torch.empty((0, 2), device="cuda")}} for r in range(2)}
    for arena in (False, True):
        out = execute_param_transfer(ops, {}, torch.device("cuda", 0), [("param", "normal")], rank=0,
                                     fake_source_state_dicts=fake, route=route, arena=arena)
        torch.cuda.synchronize()
        assert torch.equal(out["w"]["param"].cpu(), w)
        assert tuple(out["none"]["param"].shape) == (0,) and tuple(out["none2d"]["param"].shape) == (0, 4)


def _send_case(case):
    """(source meta, piece meta, expected piece from the source tensor)."""
    from oracle import reshard_oracle as O
    from tests.harness import to_ometa
    f32 = torch.float32
    if case in ("rows", "cols"):
        dim = 0 if case == "rows" else -1
        src = TensorMeta(name="w", dtype=f32, shape=(12, 16), tp_meta=(dim, 1, 2))
        piece = TensorMeta(name="w", dtype=f32, shape=(12, 16), tp_meta=(dim, 3, 4))
        # the reference: chunk(dst_deg // src_deg, dim)[dst_idx - src_idx * (dst_deg // src_deg)]
        return src, piece, lambda t: t.chunk(2, dim=dim)[1].contiguous()
    if case == "qkv":
        src = TensorMeta(name="qkv", dtype=f32, shape=(24, 5), tp_meta=(0, 0, 1), kind="qkv_heads",
                         kind_args=(4, 2, 3))
        piece = TensorMeta(name="qkv", dtype=f32, shape=(24, 5), tp_meta=(0, 1, 2), kind="qkv_heads",
                           kind_args=(4, 2, 3))
    else:   # vocab: rows [2, 6) of rank 0's shard of a 10-row table padded to 16 at degree 2
        src = TensorMeta(name="e", dtype=f32, shape=(10, 4), tp_meta=(0, 0, 2), kind="vocab_pad",
                         kind_args=(4,))
        piece = src.with_rows(2, 6)
    G = np.arange(int(np.prod(src.shape)), dtype=np.float32).reshape(tuple(src.shape))
    want = O.shard_of(G, to_ometa(piece)) if piece.rows is None else G[2:6]
    return src, piece, lambda t: torch.from_numpy(np.ascontiguousarray(want)).to(t.device)


@pytest.mark.parametrize("case", ["rows", "cols", "qkv", "vocab"])
def test_get_send_tensor_cuts_the_piece(case):
    """TransferOp.get_send_tensor (migration.py:290-312) on the engine: the
    reference's chunk(...)[k].contiguous() for chunk shards, the closed-form
    piece for the head-granular and vocabulary kinds; a shard at least as
    fine as the piece is sent as the tensor itself."""
    from oracle import reshard_oracle as O
    from tests.harness import to_ometa
    print(f"[gpu api] get_send_tensor {case}", flush=True)
    src, piece, expect = _send_case(case)
    G = np.arange(int(np.prod(src.shape)), dtype=np.float32).reshape(tuple(src.shape))
    t = torch.from_numpy(np.ascontiguousarray(O.shard_of(G, to_ometa(src)))).cuda()
    op = TransferOp(src.name, 0, 1, src, piece)
    got = op.get_send_tensor(t)
    assert got.is_contiguous() and got.data_ptr() != t.data_ptr()
    assert torch.equal(got, expect(t)), case
    assert tuple(got.shape) == tuple(piece.actual_shape())
    # the reverse direction: the finer source is sent whole, without a copy
    if piece.rows is None:
        back = TransferOp(src.name, 0, 1, piece, src)
        t2 = got.clone()
        assert back.get_send_tensor(t2) is t2


def test_execute_on_a_side_stream_waits_for_current_work():
    """stream=...: the kernels run on the given stream but after the work
    already queued on the current stream.  Here the sources are filled by
    device copies queued behind a bounded sleep kernel on the current stream,
    so a gather that did not wait would read the zeros they replace."""
    w = cases.scaled_configs()["gpt125m_tp2_tp4"]
    print(f"[gpu api] side stream {w.key}", flush=True)
    glob = global_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    real = to_device(srcs, w, "cuda")
    fake = {r: {n: {f: torch.zeros_like(t) for f, t in e.items()} for n, e in sd.items()}
            for r, sd in real.items()}
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    torch.cuda._sleep(50_000_000)   # ~20 ms of spinning on the current stream
    for r, sd in fake.items():
        for n, e in sd.items():
            for f, t in e.items():
                t.copy_(real[r][n][f])
    out = execute_param_transfer(w.ops(), {}, torch.device("cuda"), [(f, "normal") for f in w.src_fields],
                                 rank=w.dst_rank, fake_source_state_dicts=fake, stream=side)
    torch.cuda.synchronize()
    for name, e in want.items():
        for f, a in e.items():
            np.testing.assert_array_equal(t2np(out[name][f]), a, err_msg=f"{name}/{f}")


@pytest.mark.parametrize("key", ["gpt_test_tp2pp1_tp4pp1_d0.3", "llama_test_tp4pp1_tp2pp1_d0.1",
                                 "vocab_pad_tp2_tp4_d3"])
def test_forcefully_free_releases_what_the_reference_frees(key):
    """With forcefully_free the reference frees the pieces it received
    (migration.py:539-541), which releases a source only where the piece is
    that tensor or a view of it.  The expected set comes from torch itself:
    the torch restatement of get_send_tensor (oracle/torch_ref.py) runs on
    CPU copies of the sources and a source counts as freed when its piece
    shares its storage.  A 1-element field on the device is freed (sent as
    tensor.to(device), the tensor itself); one on the CPU is not."""
    from oracle import reshard_oracle as O
    from oracle.torch_ref import get_send
    from tests.harness import to_olayout
    w = {c.key: c for c in cases.all_small_cases()}[key]
    print(f"[gpu forcefully_free] {key}", flush=True)
    glob = global_state(w, _names(w))
    spl, tpl = w.layouts()
    srcs = source_shards(w, sorted(spl.layout), glob)
    fake = to_device(srcs, w, "cuda")
    cpu = to_device(srcs, w, "cpu")
    want = set()
    for op in O.schedule(to_olayout(spl), to_olayout(tpl)):
        if op.dst != w.dst_rank:
            continue
        for f in w.src_fields:
            t = cpu[op.src][op.name][f]
            if get_send(op, t).untyped_storage().data_ptr() == t.untyped_storage().data_ptr():
                want.add((op.src, op.name, f))
    for r, sd in fake.items():
        for name, e in sd.items():
            e["step_dev"] = torch.tensor([float(r)], device="cuda")
            e["step_cpu"] = torch.tensor([float(r)])
    kept = {(r, n, f): t for r, sd in fake.items() for n, e in sd.items() for f, t in e.items()}
    fields = [(f, "normal") for f in w.src_fields] + [("step_dev", TensorMeta(torch.tensor([1.0]))),
                                                      ("step_cpu", TensorMeta(torch.tensor([1.0])))]
    out = execute_param_transfer(w.ops(), {}, torch.device("cuda"), fields, rank=w.dst_rank,
                                 fake_source_state_dicts=fake, forcefully_free=True)
    torch.cuda.synchronize()
    for name, e in oracle_dest(w, srcs).items():
        for f, a in e.items():
            np.testing.assert_array_equal(t2np(out[name][f]), a, err_msg=f"{name}/{f}")
    read = {(op.src_rank, op.param_name) for op in w.ops()}
    freed = {k for k, t in kept.items() if t.untyped_storage().nbytes() == 0}
    assert {k for k in freed if k[2] in w.src_fields} == want
    n_read = len(read) * len(w.src_fields)
    if key.startswith("llama"):     # a TP merge sends whole source shards: all are released
        assert len(want) == n_read
    else:                           # row-parallel splits are copies: their sources survive
        assert 0 < len(want) < n_read
    assert {k for k in freed if k[2] == "step_dev"} == {(r, n, "step_dev") for (r, n) in read}
    assert not any(k[2] == "step_cpu" for k in freed)


def _blocks_of(tensors) -> int:
    """Bytes torch's caching allocator counts for one allocation per tensor
    (its request rounded up to 512 bytes; none for an empty tensor)."""
    return sum(-(-t.untyped_storage().nbytes() // 512) * 512 for t in tensors)


def test_fresh_destinations_are_ordinary_independent_tensors():
    """Destinations come from torch's caching allocator like torch.empty:
    the same device, counted by torch's memory statistics, one storage each
    (freeing one leaves the others intact, as Suika's forcefully_free_tensor
    expects)."""
    w = cases.scaled_configs()["gpt125m_tp2_tp4"]
    print(f"[gpu api] fresh destinations {w.key}", flush=True)
    glob = global_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    fake = to_device(srcs, w, "cuda")
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    out = execute_param_transfer(w.ops(), {}, torch.device("cuda"), [(f, "normal") for f in w.src_fields],
                                 rank=w.dst_rank, fake_source_state_dicts=fake)
    torch.cuda.synchronize()
    after = torch.cuda.memory_allocated()
    ref = torch.empty(1, device="cuda")
    tensors = [t for e in out.values() for t in e.values()]
    total = sum(t.untyped_storage().nbytes() for t in tensors)
    # one caching-allocator block per tensor (rounded to 512 bytes) and
    # nothing else left allocated: no block made ahead and left unused
    assert after - before == _blocks_of(tensors) and total > 0
    assert all(t.device == ref.device and t.is_contiguous() for t in tensors)
    assert len({t.untyped_storage().data_ptr() for t in tensors}) == len(tensors)
    assert all(t.untyped_storage().nbytes() == t.numel() * t.element_size() for t in tensors)
    victim = tensors[0]
    victim.untyped_storage().resize_(0)
    for name, e in want.items():
        for f, a in e.items():
            if out[name][f] is not victim:
                np.testing.assert_array_equal(t2np(out[name][f]), a, err_msg=f"{name}/{f}")


@pytest.mark.parametrize("groups", [None, 4])
@pytest.mark.parametrize("key", ["gpt125m_tp2_tp4", "qwen7b_tp2_tp4"])
def test_destination_blocks_made_ahead(key, groups, monkeypatch):
    """The direct route's fresh destinations are allocated on a helper thread
    from the call's prologue on, while the launch groups are planned.  Every
    tensor whose pieces cover it (all but vocabulary shards, which may be
    padded, and empty tensors) and whose element size is its field's in the
    first source the prologue reads is built on such a block, bf16 recast
    copies included; the rest -- here one tensor's exp_avg, float64 among
    float32 ones -- are allocated on the calling thread.  The result matches
    the oracle, each tensor holds one allocation of its own and no block is
    left over."""
    from suika_amd import _lib
    from suika_amd import migration as M
    from tests.harness import round_robin_groups
    if groups:
        monkeypatch.setattr(M, "_pipeline_groups", round_robin_groups(groups))
    w = cases.scaled_configs()[key]
    print(f"[gpu api] blocks ahead {w.key} groups={groups}", flush=True)
    glob = global_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    fake = to_device(srcs, w, "cuda")
    ops = w.ops()
    odd = next(op.param_name for op in ops
               if op.dst_shard_meta.kind == "chunk" and len(op.dst_shard_meta.shape) == 2)
    for sd in fake.values():
        if odd in sd:
            assert sd[odd]["exp_avg"].dtype == torch.float32
            sd[odd]["exp_avg"] = sd[odd]["exp_avg"].double()
    pieces, vocab = {}, set()
    for op in ops:
        pieces[op.param_name] = pieces.get(op.param_name, 0) + op.dst_meta.numel()
        if op.dst_shard_meta.kind == "vocab_pad":
            vocab.add(op.param_name)
    assert bool(vocab) == (key == "qwen7b_tp2_tp4") and bool(w.recast_map) == bool(vocab)
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    taken0, missed0 = _lib.host().blocks_ahead()
    out = execute_param_transfer(ops, {}, torch.device("cuda"), [(f, "normal") for f in w.src_fields],
                                 rank=w.dst_rank, fake_source_state_dicts=fake, recast=w.recast_map)
    torch.cuda.synchronize()
    after = torch.cuda.memory_allocated()
    taken, missed = (a - b for a, b in zip(_lib.host().blocks_ahead(), (taken0, missed0)))
    tensors = [t for e in out.values() for t in e.values()]
    assert after - before == _blocks_of(tensors)
    assert len({t.untyped_storage().data_ptr() for t in tensors if t.numel()}) == sum(1 for t in tensors if t.numel())
    # the element size each field's blocks are made for: the first source's
    first_op = next(op for op in ops if op.dst_rank == w.dst_rank)
    first = fake[first_op.src_rank][first_op.param_name]
    guess = {f: first[f].element_size() for f in w.src_fields}
    guess.update({t: 2 for t in w.recast_map})
    own = sum(1 for n, e in out.items() for f, t in e.items()
              if n in vocab or pieces[n] == 0 or pieces[n] != t.numel() or t.element_size() != guess[f])
    assert own >= 1
    assert (taken, missed) == (len(tensors) - own, own), (taken, missed, own)
    assert out[odd]["exp_avg"].dtype == torch.float64
    for name, e in want.items():
        for f, a in e.items():
            got = out[name][f]
            if name == odd and f == "exp_avg":
                got = got.to(torch.float32)      # exact: float64 copies of float32 values
            np.testing.assert_array_equal(t2np(got), a, err_msg=f"{name}/{f}")


def test_destination_blocks_with_memory_history_recording():
    """With torch's allocator history recording Python stacks, every
    allocation -- the helper thread's too -- takes the GIL to record its
    context.  The calling thread waits for the helper only with the GIL
    released, so the call completes, matches the oracle, and the snapshot
    holds the destinations' allocations."""
    w = cases.scaled_configs()["gpt125m_tp2_tp4"]
    print(f"[gpu api] blocks ahead under memory history {w.key}", flush=True)
    glob = global_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    fake = to_device(srcs, w, "cuda")
    from suika_amd import _lib
    torch.cuda.synchronize()
    taken0 = _lib.host().blocks_ahead()[0]
    torch.cuda.memory._record_memory_history(max_entries=100000, stacks="python")
    try:
        out = execute_param_transfer(w.ops(), {}, torch.device("cuda"), [(f, "normal") for f in w.src_fields],
                                     rank=w.dst_rank, fake_source_state_dicts=fake)
        torch.cuda.synchronize()
        snap = torch.cuda.memory._snapshot()
    finally:
        torch.cuda.memory._record_memory_history(enabled=None)
    assert _lib.host().blocks_ahead()[0] > taken0, "the helper thread made no block"
    ptrs = {t.untyped_storage().data_ptr() for e in out.values() for t in e.values() if t.numel()}
    traced = {ev["addr"] for trace in snap["device_traces"] for ev in trace if ev["action"] == "alloc"}
    assert ptrs <= traced, f"{len(ptrs - traced)} destinations not in the allocator's history"
    for name, e in want.items():
        for f, a in e.items():
            np.testing.assert_array_equal(t2np(out[name][f]), a, err_msg=f"{name}/{f}")


def test_prepare_then_reshard():
    """sr_prepare (a process's first-use costs paid ahead: GPU code, setup
    stream, copy path) succeeds on the current stream and on another one,
    any number of times, and the reshards after it are unchanged."""
    import ctypes

    from suika_amd import _lib
    L = _lib.lib()
    print("[gpu api] sr_prepare", flush=True)
    side = torch.cuda.Stream()
    for stream in (torch.cuda.current_stream(), side, torch.cuda.current_stream()):
        assert L.sr_prepare(ctypes.c_void_p(stream.cuda_stream)) == _lib.SR_OK, _lib.last_error(L)
    w = cases.scaled_configs()["llama7b_tp4pp2_tp2pp2"]
    glob = global_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    out = execute_param_transfer(w.ops(), {}, torch.device("cuda"), [(f, "normal") for f in w.src_fields],
                                 rank=w.dst_rank, fake_source_state_dicts=to_device(srcs, w, "cuda"))
    torch.cuda.synchronize()
    for name, e in want.items():
        for f, a in e.items():
            np.testing.assert_array_equal(t2np(out[name][f]), a, err_msg=f"{name}/{f}")


@pytest.mark.parametrize("w", cases.all_small_cases(), ids=lambda w: w.key)
def test_whole_schedule_and_plain_list_agree(w):
    """The drop-in call given the world's whole schedule (this rank's ops
    taken at the schedule's positions, encoded from its tables) and given
    the same ops as a plain list (every op's attributes read) returns the
    oracle's state both times."""
    from suika_amd import schedule_param_transfer
    from suika_amd.meta import Schedule
    print(f"[gpu api] whole schedule vs list {w.key}", flush=True)
    world = schedule_param_transfer(*w.layouts())
    assert type(world) is Schedule and world.encoding() is not None
    glob = global_state(w, _names(w))
    srcs = source_shards(w, sorted(w.layouts()[0].layout), glob)
    want = oracle_dest(w, srcs)
    for ops in (world, list(world)):
        out = execute_param_transfer(ops, {}, torch.device("cuda"), [(f, "normal") for f in w.src_fields],
                                     rank=w.dst_rank, fake_source_state_dicts=to_device(srcs, w, "cuda"),
                                     recast=w.recast_map)
        torch.cuda.synchronize()
        assert set(out) == set(want), (w.key, type(ops))
        for name, e in want.items():
            for f, a in e.items():
                np.testing.assert_array_equal(t2np(out[name][f]), a, err_msg=f"{w.key} {type(ops)}: {name}/{f}")

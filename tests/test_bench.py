"""bench.py's contract: one GPU only, the CPU baseline sampler, and the JSON
line's keys and arithmetic."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused():
    out = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], cwd=ROOT, capture_output=True,
                         text=True, timeout=120)
    assert out.returncode == 2, out.stdout + out.stderr
    assert "--gpus 2 is not supported" in out.stderr and out.stdout == ""


def test_cpu_baseline_sample():
    """The torch-CPU leg on a one-layer sample of the GPT-125M share: one
    untimed run, then timed runs; bytes are the sample's algorithmic bytes."""
    sys.path.insert(0, str(ROOT))
    import bench
    from suika_amd.workloads import CONFIGS
    t, nbytes, runs, layers, out, b_min = bench.cpu_baseline(CONFIGS["gpt125m_tp2_tp4"], 2, 0.0, layers=1,
                                                             keep_output=True)
    assert t > 0 and runs >= 1 and layers == 1
    assert 0 < nbytes < 4 * 0.835e9       # below the full share's B_alg
    assert 0 < b_min < nbytes             # P + D of the sample, below its 3P + D
    # the sample's output is the oracle's reshard of the same seeded shards
    from dataclasses import replace

    from oracle import reshard_oracle as O
    from suika_amd.workloads import make_source_state
    from tests.harness import t2np, to_olayout
    w = CONFIGS["gpt125m_tp2_tp4"]
    ws = replace(w, model=replace(w.model, n_layer=1))
    spl, tpl = ws.layouts()
    ops = O.schedule(to_olayout(spl), to_olayout(tpl))
    srcs = make_source_state(ws, sorted({op.src for op in ops if op.dst == ws.dst_rank}), "cpu")
    srcs_np = {r: {n: {f: t2np(x) for f, x in e.items()} for n, e in sd.items()} for r, sd in srcs.items()}
    want = O.execute_fake_source(ops, ws.dst_rank, srcs_np, list(ws.src_fields), recast=ws.recast_map)
    assert set(out) == set(want)
    for name, ent in want.items():
        for f, a in ent.items():
            assert (t2np(out[name][f]) == a).all(), f"{name}/{f}"


def test_mismatch_counter():
    sys.path.insert(0, str(ROOT))
    import torch

    import bench
    a = {"x": {"p": torch.arange(6, dtype=torch.float32)}, "y": {"p": torch.zeros(3, dtype=torch.bfloat16)}}
    b = {"x": {"p": torch.arange(6, dtype=torch.float32)}, "y": {"p": torch.zeros(3, dtype=torch.bfloat16)}}
    keys = [("x", "p"), ("y", "p")]
    assert bench.mismatches(keys, a, b) == []
    b["y"]["p"][1] = -0.0             # equal as numbers, different bytes
    assert bench.mismatches(keys, a, b) == ["y/p"]
    b["x"]["p"] = b["x"]["p"].to(torch.float64)
    assert bench.mismatches(keys, a, b) == ["x/p", "y/p"]


@pytest.mark.gpu
def test_bench_json_line(tmp_path):
    """A short run on the smallest workload prints one JSON line with every
    key the driver reads, self-consistent figures and no CPU baseline when
    it is switched off."""
    out_file = tmp_path / "b.json"
    print("[bench test] gpt125m_tp2_tp4", flush=True)
    res = subprocess.run([sys.executable, "bench.py", "--config", "gpt125m_tp2_tp4", "--steps", "3", "--warmup", "1",
                          "--no-cpu-baseline", "--json-out", str(out_file)], cwd=ROOT, capture_output=True,
                         text=True, timeout=240)
    assert res.returncode == 0, res.stderr[-3000:]
    lines = [l for l in res.stdout.splitlines() if l.strip()]
    assert len(lines) == 1, res.stdout
    d = json.loads(lines[0])
    assert json.loads(out_file.read_text()) == d
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
              "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert k in d, k
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 1 and d["unit"] == "GB/s"
    assert d["higher_is_better"] is True and d["vs_baseline"] is None and d["cpu_baseline"] is None
    assert d["config"]["key"] == "gpt125m_tp2_tp4" and "workload" in d["config"]
    b_alg = d["config"]["B_alg_bytes"]
    assert abs(d["value"] - b_alg / (d["ms_per_step"] * 1e-3) / 1e9) <= 0.1 + 1e-3 * d["value"]
    r = d["roofline"]
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert abs(r["frac"] - r["achieved"] / r["peak"]) < 1e-3
    assert r["kernel"] in ("sr_pack_kernel", "sr_unpack_kernel")
    assert 0.2 < r["frac"] < 1.0
    p = d["parity"]
    assert p["mismatched"] == 0 and p["tensors"] > 0, p
    assert set(p["routes"]) == {"gather_vs_pack_unpack", "execute_param_transfer",
                                "execute_param_transfer_arena"}


def test_handoff_closed_form_matches_the_oracle():
    """bench.py's own closed form (which seeds the hand-off leg's old ranks
    and checks its new ranks without the product's geometry) cuts the same
    shard as the oracle's shard_of for every kind: row and column chunks,
    head-granular fused QKV, and zero-padded vocabulary tables."""
    import numpy as np
    import torch

    import bench
    from oracle import reshard_oracle as O
    from tests import cases
    from tests.harness import to_ometa
    ws = list(cases.golden_cases().values()) + list(cases.scaled_configs().values()) + \
        cases.padded_vocab_cases()
    kinds = set()
    for w in ws:
        spl, tpl = w.layouts()
        for layout in (spl, tpl):
            for metas in layout.layout.values():
                for name, m in metas.items():
                    shape = tuple(int(s) for s in m.shape)
                    G = np.arange(int(np.prod(shape)), dtype=np.int64).reshape(shape)
                    got = bench._expected_shard(torch.from_numpy(G), m).numpy()
                    want = O.shard_of(G, to_ometa(m))
                    assert got.shape == want.shape and (got == want).all(), (w.key, name, m.tp_meta)
                    kinds.add(m.kind if m.tp_meta is not None else "replicated")
    assert kinds == {"chunk", "qkv_heads", "vocab_pad", "replicated"}, kinds

"""The whole native path driven from plain C11, with no Python in the
process: layouts -> ``sr_schedule`` -> ``sr_lower`` -> ``sr_plan_create`` ->
``sr_gather`` and ``sr_pack`` + ``sr_unpack`` on hipMalloc'd device memory,
checked byte for byte by the program itself (tests/c/abi_gpu_reshard.c).

This is what a cgo / JNI / N-API binding of the library does.  The program is
built by ``__graft_entry__.build()`` next to the library; on a host without a
GPU its planning half still runs.
"""
import subprocess

import pytest

from suika_amd import build as sb

PLAN_LINES = [
    "schedule ops 4",                          # two names x two source ranks
    "lowered src 4 dst 2 pieces 4 peers 2",
]


def test_c_caller_plans_without_gpu(tmp_path):
    """Build the program into a scratch folder and run it here: the planning
    lines print, then the first HIP call reports that no device is present."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present; the GPU test runs the whole program")
    exe = sb.build_c_check(out=tmp_path / "abi_gpu_reshard")
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    lines = out.stdout.splitlines()
    assert out.returncode == 1 and lines[:2] == PLAN_LINES, out.stdout + out.stderr
    assert lines[2].startswith("hip error"), out.stdout


@pytest.mark.gpu
def test_c_caller_on_gpu():
    exe = sb.C_GPU_BIN
    assert exe.exists(), f"{exe} is missing: run __graft_entry__.build() first"
    print(f"running {exe}", flush=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=90)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.splitlines() == PLAN_LINES + [
        "gather mismatches 0",
        "pack_unpack mismatches 0",
    ], out.stdout

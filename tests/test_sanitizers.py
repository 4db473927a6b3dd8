"""The native host code under AddressSanitizer and UndefinedBehaviorSanitizer.

``suika_amd.build.build_sanitized`` compiles the library's host half (plan
builder, schedule.cpp, lower.cpp, handoff.cpp, stage.cpp and the host side
of reshard.hip; the gfx950 code as usual) and host_bind.cpp with both
sanitizers.  The CPU tests that drive that code -- the C ABI's argument
checks and corrupted-table fuzz, the planner against the reference's
recorded schedules, the host-side staging pack, the host extension's
per-tensor work -- then run in a child process with the sanitizer runtime
preloaded and any report fatal.  The run must pass with no report.
"""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

FILES = ["tests/test_abi.py", "tests/test_schedule.py", "tests/test_plan.py", "tests/test_stage_host.py",
         "tests/test_handoff.py", "tests/test_golden.py", "tests/test_fuzz.py", "tests/test_reference_objects.py",
         "tests/test_checkpoint.py"]


@pytest.mark.slow
def test_host_code_is_clean_under_asan_and_ubsan():
    from suika_amd.build import build_sanitized, sanitizer_runtime
    lib, host = build_sanitized()
    env = dict(os.environ,
               LD_PRELOAD=str(sanitizer_runtime()),
               # Python itself frees nothing at exit; leaks are not what this run checks
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1",
               SUIKA_RESHARD_LIB=str(lib), SUIKA_HOST_LIB=str(host))
    # the two large Qwen2-TEST plan changes run the same host code as the
    # others at 64x the bytes; the recast case stays
    res = subprocess.run([sys.executable, "-m", "pytest", *FILES, "-q", "-m", "not gpu", "-p", "no:cacheprovider",
                          "-k", "not (qwen2_test_tp2_tp1 or qwen2_test_tp1_tp2_d1)", "-n", "6"],
                         cwd=ROOT, env=env, capture_output=True, text=True, timeout=1500)
    out = res.stdout + res.stderr
    reports = [l for l in out.splitlines() if "runtime error:" in l or "AddressSanitizer" in l]
    assert res.returncode == 0 and not reports, "\n".join(reports[:20]) + "\n" + out[-4000:]
    assert " passed" in out.splitlines()[-1], out[-2000:]

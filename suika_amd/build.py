"""Build the in-tree HIP library ``suika_amd/lib/libsuika_reshard.so`` for gfx950.

The library is compiled with ``hipcc`` directly (no torch extension
machinery) so that it stays a plain C-ABI shared object that ``ctypes`` -- or
any other FFI -- can load.  hipcc cross-compiles for gfx950 without a GPU
present.  Sources: ``reshard.hip`` (plan builder and kernels),
``schedule.cpp`` and ``lower.cpp`` (the host-only planner: transfer schedule
and its lowering to region moves), ``handoff.cpp`` (exported device
allocations for the same-GPU state hand-off between processes), ``stage.cpp``
(sources in host memory packed into device buffers, results copied back to
host memory, through pinned windows and a host thread pool).

``build_host`` compiles ``host_bind.cpp`` into ``suika_amd/lib/_suika_host.so``,
the CPython extension (on torch's C++ API) that does the drop-in operator's
per-tensor host work; it is a plain ``g++`` line against the installed torch
and the library (whose sr_lower and sr_plan_create it calls), found beside it.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path
from typing import Tuple

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
SOURCES = [PKG_DIR / "csrc" / "reshard.hip", PKG_DIR / "csrc" / "schedule.cpp",
           PKG_DIR / "csrc" / "lower.cpp", PKG_DIR / "csrc" / "handoff.cpp", PKG_DIR / "csrc" / "stage.cpp"]
INCLUDE = REPO_DIR / "include"
LIB_DIR = PKG_DIR / "lib"
LIB = LIB_DIR / "libsuika_reshard.so"
HOST_SRC = PKG_DIR / "csrc" / "host_bind.cpp"
HOST_LIB = LIB_DIR / "_suika_host.so"

ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # the host extension names the library by this soname, so it binds to
    # whichever copy the process loaded first (the ctypes binding's)
    "-Wl,-soname,libsuika_reshard.so",
    # packed-FP32 instructions stay disabled for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (looked at $HIPCC, PATH, /opt/rocm/bin/hipcc)")


def build(verbose: bool = False, out: Path = LIB, defines=()) -> Path:
    """Compile the library (always recompiles) and return its path.

    ``defines`` are extra ``NAME=VALUE`` macros (kernel tuning knobs such as
    SR_UNROLL / SR_BLOCK) for building variants elsewhere than ``out``."""
    out = Path(out)
    out.parent.mkdir(parents=True, exist_ok=True)
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc_path(), *HIPCC_FLAGS, *[f"-D{d}" for d in defines], f"-I{INCLUDE}", *map(str, SOURCES),
           "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    noise = "packed-fp32-ops"
    msgs = [l for l in (res.stdout + res.stderr).splitlines() if l.strip() and noise not in l]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs), flush=True)
    os.replace(tmp, out)
    return out


C_GPU_SRC = REPO_DIR / "tests" / "c" / "abi_gpu_reshard.c"
C_GPU_BIN = LIB_DIR / "abi_gpu_reshard"


def build_c_check(verbose: bool = False, out: Path = C_GPU_BIN) -> Path:
    """Compile the C11 program that drives the whole native path on the GPU
    (tests/c/abi_gpu_reshard.c) against the library; its GPU test runs it."""
    out = Path(out)
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    cc = os.environ.get("CC") or shutil.which("gcc") or "gcc"
    cmd = [cc, "-std=c11", "-O2", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__", f"-I{INCLUDE}",
           f"-I{rocm / 'include'}", str(C_GPU_SRC), f"-L{LIB_DIR}", "-lsuika_reshard", f"-L{rocm / 'lib'}",
           "-lamdhip64", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{LIB_DIR}", f"-Wl,-rpath,{rocm / 'lib'}", "-o", str(out)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("C check build failed:\n" + (res.stdout + res.stderr)[-4000:])
    return out


def build_host(verbose: bool = False, out: Path = HOST_LIB) -> Path:
    """Compile the torch-facing host extension (always recompiles)."""
    import sysconfig

    import torch
    from torch.utils.cpp_extension import include_paths, library_paths
    out = Path(out)
    out.parent.mkdir(parents=True, exist_ok=True)
    tmp = out.with_suffix(".so.tmp")
    cxx = os.environ.get("CXX") or shutil.which("g++") or "g++"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    libdirs = library_paths()
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-function",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           "-DTORCH_EXTENSION_NAME=_suika_host",
           *[f"-I{p}" for p in include_paths()], f"-I{sysconfig.get_paths()['include']}",
           # the library's TensorMeta arithmetic (sr_meta.h) and the headers it uses
           "-D__HIP_PLATFORM_AMD__", f"-I{INCLUDE}", f"-I{HOST_SRC.parent}",
           f"-I{Path(os.environ.get('ROCM_PATH', '/opt/rocm')) / 'include'}",
           str(HOST_SRC), *[f"-L{p}" for p in libdirs], *[f"-Wl,-rpath,{p}" for p in libdirs],
           "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
           # the library itself (sr_lower, sr_plan_create), found beside the extension
           f"-L{LIB_DIR}", "-lsuika_reshard", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("host extension build failed:\n" + (res.stdout + res.stderr)[-6000:])
    os.replace(tmp, out)
    return out


SANITIZE_DIR = REPO_DIR / "_build" / "sanitize"


def _llvm() -> Path:
    return Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "llvm"


def sanitizer_runtime() -> Path:
    """clang's shared AddressSanitizer runtime (it carries UBSan's handlers
    too), which a sanitized build needs preloaded into the Python process."""
    found = sorted(_llvm().glob("lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not found:
        raise RuntimeError(f"no libclang_rt.asan-x86_64.so under {_llvm()}")
    return found[-1]


def build_sanitized(verbose: bool = False, out_dir: Path = SANITIZE_DIR) -> Tuple[Path, Path]:
    """The library and the host extension with the host code under
    AddressSanitizer and UndefinedBehaviorSanitizer, for CPU runs.

    The library's host half (the plan builder, schedule.cpp, lower.cpp,
    handoff.cpp, stage.cpp and the host side of reshard.hip) is compiled by
    hipcc with each sanitizer flag behind ``-Xarch_host``, so the gfx950 code
    is built as usual; host_bind.cpp is compiled by the same clang so both
    use one sanitizer runtime (``sanitizer_runtime()``).  Both go to
    ``out_dir`` (outside the package, never loaded unless named by
    SUIKA_RESHARD_LIB / SUIKA_HOST_LIB)."""
    import sysconfig

    import torch
    from torch.utils.cpp_extension import include_paths, library_paths
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    lib, host = out_dir / "libsuika_reshard.so", out_dir / "_suika_host.so"
    san = ["-O1", "-g", "-fno-omit-frame-pointer", "-shared-libasan"]
    flags = [f for f in HIPCC_FLAGS if f != "-O3"]
    cmd = [hipcc_path(), *flags, *san, "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           f"-I{INCLUDE}", *map(str, SOURCES), "-o", str(lib)]
    runs = [("sanitized library", cmd)]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    libdirs = library_paths()
    runs.append(("sanitized host extension", [
        str(_llvm() / "bin" / "clang++"), *san, "-fsanitize=address,undefined", "-std=c++17", "-fPIC", "-shared",
        "-Wno-braced-scalar-init", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        "-DTORCH_EXTENSION_NAME=_suika_host", *[f"-I{p}" for p in include_paths()],
        f"-I{sysconfig.get_paths()['include']}", "-D__HIP_PLATFORM_AMD__", f"-I{INCLUDE}", f"-I{HOST_SRC.parent}",
        f"-I{Path(os.environ.get('ROCM_PATH', '/opt/rocm')) / 'include'}", str(HOST_SRC),
        *[f"-L{p}" for p in libdirs], *[f"-Wl,-rpath,{p}" for p in libdirs],
        "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", f"-L{out_dir}", "-lsuika_reshard",
        "-Wl,-rpath,$ORIGIN", "-o", str(host)]))
    for what, c in runs:
        if verbose:
            print(" ".join(c), flush=True)
        res = subprocess.run(c, capture_output=True, text=True)
        if res.returncode != 0:
            msgs = [l for l in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in l]
            raise RuntimeError(f"{what} build failed:\n" + "\n".join(msgs)[-6000:])
    return lib, host


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        print(build_sanitized(verbose="-v" in sys.argv))
        sys.exit(0)
    print(build(verbose="-v" in sys.argv))
    print(build_host(verbose="-v" in sys.argv))
    print(build_c_check(verbose="-v" in sys.argv))

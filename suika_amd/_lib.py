"""ctypes binding of ``libsuika_reshard.so`` (C ABI in include/suika_reshard.h
and include/suika_planner.h).

The binding fails loudly: importing the package never falls back to a CPU or
torch path.  If the library is missing, every entry point raises
``RuntimeError`` telling the caller to run the build.
"""
from __future__ import annotations

import ctypes
import os
from collections import namedtuple
from pathlib import Path
from typing import Optional

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libsuika_reshard.so"
HOST_PATH = Path(__file__).resolve().parent / "lib" / "_suika_host.so"

SR_OK = 0
SR_EINVAL = -1
SR_EBOUNDS = -2
SR_EALIGN = -3
SR_EOVERLAP = -4
SR_EHIP = -5
SR_ENOMEM = -6
SR_EDTYPE = -7

STATUS_NAMES = {
    SR_OK: "SR_OK",
    SR_EINVAL: "SR_EINVAL",
    SR_EBOUNDS: "SR_EBOUNDS",
    SR_EALIGN: "SR_EALIGN",
    SR_EOVERLAP: "SR_EOVERLAP",
    SR_EHIP: "SR_EHIP",
    SR_ENOMEM: "SR_ENOMEM",
    SR_EDTYPE: "SR_EDTYPE",
}

SR_DT_U8, SR_DT_BF16, SR_DT_F16, SR_DT_F32, SR_DT_F64, SR_DT_I32, SR_DT_I64 = range(7)

SR_PIECE_COPY, SR_PIECE_RECAST, SR_PIECE_ZERO = 0, 1, 2

SR_OPT_TEMPORAL = 0x1
SR_OPT_SKIP_COVERAGE = 0x2
SR_OPT_PIECE_ORDER = 0x4
SR_OPT_NO_XCD_INTERLEAVE = 0x8
SR_OPT_NO_ROW_GROUPS = 0x10
SR_OPT_GATHER_ONLY = 0x20

SR_MAX_DIMS = 8
SR_KIND_CHUNK, SR_KIND_VOCAB_PAD, SR_KIND_QKV_HEADS = 0, 1, 2

# Every symbol the header declares; the CPU test-suite checks they resolve.
EXPORTED_SYMBOLS = (
    "sr_abi_version",
    "sr_last_error",
    "sr_selftest",
    "sr_plan_create",
    "sr_plan_peer_bytes",
    "sr_plan_piece_offset",
    "sr_plan_info_get",
    "sr_pack",
    "sr_unpack",
    "sr_gather",
    "sr_gather_noalloc",
    "sr_prepare",
    "sr_stage_pack",
    "sr_pack_host",
    "sr_download",
    "sr_set_host_threads",
    "sr_stage_counters_get",
    "sr_plan_destroy",
    "sr_schedule",
    "sr_lower",
    "sr_lowering_destroy",
    "sr_handoff_alloc",
    "sr_handoff_free",
    "sr_handoff_open",
    "sr_handoff_close",
)

# Largest hand-off allocation (SR_HANDOFF_MAX_BYTES, include/suika_handoff.h).
HANDOFF_MAX_BYTES = 2146435072


class SrIpcHandle(ctypes.Structure):
    """The 64 opaque bytes of an exported hand-off allocation (sr_ipc_handle)."""
    _fields_ = [("bytes", ctypes.c_ubyte * 64)]

ABI_VERSION = 5

# Device bytes per GPU that sr_gather_noalloc keeps its tables in (SR_SCRATCH_BYTES).
SCRATCH_BYTES = 64 << 20

# Pinned staging windows of sr_stage_pack / sr_download (SR_STAGE_WINDOW_BYTES,
# SR_STAGE_WINDOWS).
STAGE_WINDOW_BYTES = 16 << 20
STAGE_WINDOWS = 4


class SrStageCounters(ctypes.Structure):
    """Process totals of the host staging calls (sr_stage_counters)."""
    _fields_ = [
        ("host_bytes_up", ctypes.c_uint64),
        ("host_piece_bytes", ctypes.c_uint64),
        ("device_piece_bytes", ctypes.c_uint64),
        ("bytes_down", ctypes.c_uint64),
        ("windows", ctypes.c_uint64),
    ]


class SrTensor(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_uint64),
        ("cols", ctypes.c_uint64),
        ("dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class SrPiece(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("peer", ctypes.c_int32),
        ("src", ctypes.c_int32),
        ("dst", ctypes.c_int32),
        ("dst2", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("rows", ctypes.c_uint64),
        ("cols", ctypes.c_uint64),
        ("src_row", ctypes.c_uint64),
        ("src_col", ctypes.c_uint64),
        ("dst_row", ctypes.c_uint64),
        ("dst_col", ctypes.c_uint64),
    ]


def _struct_dtype(struct) -> "np.dtype":
    """numpy dtype with the field names, types and offsets of a ctypes struct."""
    import numpy as np
    kinds = {ctypes.c_int32: np.int32, ctypes.c_uint32: np.uint32, ctypes.c_int64: np.int64,
             ctypes.c_uint64: np.uint64}
    names = [n for n, _ in struct._fields_]
    dt = np.dtype({"names": names, "formats": [kinds[t] for _, t in struct._fields_],
                   "offsets": [getattr(struct, n).offset for n in names],
                   "itemsize": ctypes.sizeof(struct)})
    return dt


SR_TENSOR_DTYPE = _struct_dtype(SrTensor)
SR_PIECE_DTYPE = _struct_dtype(SrPiece)
TensorRecord = namedtuple("TensorRecord", [n for n, _ in SrTensor._fields_])
PieceRecord = namedtuple("PieceRecord", [n for n, _ in SrPiece._fields_])


def as_tensors(arr) -> "ctypes.POINTER(SrTensor)":
    """Pointer to a contiguous SR_TENSOR_DTYPE array (kept alive by the caller)."""
    assert arr.dtype == SR_TENSOR_DTYPE and arr.flags["C_CONTIGUOUS"]
    return arr.ctypes.data_as(ctypes.POINTER(SrTensor))


def as_pieces(arr) -> "ctypes.POINTER(SrPiece)":
    """Pointer to a contiguous SR_PIECE_DTYPE array (kept alive by the caller)."""
    assert arr.dtype == SR_PIECE_DTYPE and arr.flags["C_CONTIGUOUS"]
    return arr.ctypes.data_as(ctypes.POINTER(SrPiece))


class SrMeta(ctypes.Structure):
    """One TensorMeta of a layout (sr_meta)."""
    _fields_ = [
        ("rank", ctypes.c_int64),
        ("name", ctypes.c_int64),
        ("itemsize", ctypes.c_int64),
        ("ndim", ctypes.c_int64),
        ("shape", ctypes.c_int64 * SR_MAX_DIMS),
        ("slice_dim", ctypes.c_int64),
        ("tp_index", ctypes.c_int64),
        ("tp_deg", ctypes.c_int64),
        ("kind", ctypes.c_int64),
        ("kind_args", ctypes.c_int64 * 3),
        ("row0", ctypes.c_int64),
        ("row1", ctypes.c_int64),
    ]


class SrOp(ctypes.Structure):
    """One scheduled piece (sr_op)."""
    _fields_ = [
        ("name", ctypes.c_int64),
        ("src_rank", ctypes.c_int64),
        ("dst_rank", ctypes.c_int64),
        ("src_meta", ctypes.c_int64),
        ("dst_shard", ctypes.c_int64),
        ("piece_tp_index", ctypes.c_int64),
        ("piece_tp_deg", ctypes.c_int64),
        ("row0", ctypes.c_int64),
        ("row1", ctypes.c_int64),
    ]


class SrSrcSpec(ctypes.Structure):
    """The tensor a source slot binds to (sr_src_spec)."""
    _fields_ = [
        ("dtype", ctypes.c_int64),
        ("ndim", ctypes.c_int64),
        ("shape", ctypes.c_int64 * SR_MAX_DIMS),
    ]


class SrSlotKey(ctypes.Structure):
    """What a tensor slot of a lowering holds (sr_slot_key)."""
    _fields_ = [
        ("op", ctypes.c_int64),
        ("field", ctypes.c_int64),
        ("recast", ctypes.c_int64),
        ("dtype", ctypes.c_int64),
        ("ndim", ctypes.c_int64),
        ("shape", ctypes.c_int64 * SR_MAX_DIMS),
    ]


class SrLowering(ctypes.Structure):
    """Tables of one sr_lower call (owned by the library)."""
    _fields_ = [
        ("n_src", ctypes.c_int64),
        ("n_dst", ctypes.c_int64),
        ("n_pieces", ctypes.c_int64),
        ("n_peers", ctypes.c_int64),
        ("n_empty", ctypes.c_int64),
        ("src", ctypes.POINTER(SrTensor)),
        ("src_key", ctypes.POINTER(SrSlotKey)),
        ("dst", ctypes.POINTER(SrTensor)),
        ("dst_key", ctypes.POINTER(SrSlotKey)),
        ("pieces", ctypes.POINTER(SrPiece)),
        ("peer_rank", ctypes.POINTER(ctypes.c_int64)),
        ("empty", ctypes.POINTER(SrSlotKey)),
    ]


# These records are all-int64, so tables are plain [n, k] int64 matrices.
SR_META_WORDS = ctypes.sizeof(SrMeta) // 8
SR_OP_WORDS = ctypes.sizeof(SrOp) // 8
SR_SPEC_WORDS = ctypes.sizeof(SrSrcSpec) // 8
SR_KEY_WORDS = ctypes.sizeof(SrSlotKey) // 8


def copy_table(ptr, n: int, dtype) -> "np.ndarray":
    """A numpy copy of ``n`` records of ``dtype`` at a ctypes pointer."""
    import numpy as np
    dtype = np.dtype(dtype)
    if n == 0:
        return np.zeros(0, dtype=dtype)
    addr = ctypes.cast(ptr, ctypes.c_void_p).value
    raw = (ctypes.c_char * (n * dtype.itemsize)).from_address(addr)
    return np.frombuffer(raw, dtype=dtype).copy()


def as_int64_ptr(arr) -> "ctypes.c_void_p":
    """Address of a C-contiguous int64 matrix (kept alive by the caller)."""
    import numpy as np
    assert arr.dtype == np.int64 and arr.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(arr.ctypes.data)


class SrPlanOptions(ctypes.Structure):
    _fields_ = [
        ("tile_bytes", ctypes.c_uint32),
        ("max_blocks", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


class SrPlanInfo(ctypes.Structure):
    _fields_ = [
        ("n_pieces", ctypes.c_int64),
        ("n_peers", ctypes.c_int64),
        ("n_src", ctypes.c_int64),
        ("n_dst", ctypes.c_int64),
        ("pack_tiles", ctypes.c_int64),
        ("unpack_tiles", ctypes.c_int64),
        ("pack_bytes_read", ctypes.c_uint64),
        ("pack_bytes_written", ctypes.c_uint64),
        ("unpack_bytes_read", ctypes.c_uint64),
        ("unpack_bytes_written", ctypes.c_uint64),
        ("buffer_bytes", ctypes.c_uint64),
        ("gather_tiles", ctypes.c_int64),
        ("gather_bytes_read", ctypes.c_uint64),
        ("gather_bytes_written", ctypes.c_uint64),
    ]


class ReshardError(RuntimeError):
    """HIP/runtime failure reported by the library (SR_EHIP, SR_ENOMEM)."""


class PlanError(AssertionError):
    """Invalid plan or argument; an AssertionError like the reference's
    ``assert`` checks (Suika/migration.py:293-294, 311, 356, 436, 441)."""


class HostSourceError(PlanError):
    """A source tensor in host memory where the device route takes only
    tensors on the device; ``execute_param_transfer`` then stages the
    transfer from host memory (``sr_stage_pack``)."""


_lib: Optional[ctypes.CDLL] = None


def _declare(lib: ctypes.CDLL) -> None:
    vp = ctypes.c_void_p
    lib.sr_abi_version.restype = ctypes.c_int
    lib.sr_abi_version.argtypes = []
    lib.sr_last_error.restype = ctypes.c_char_p
    lib.sr_last_error.argtypes = []
    lib.sr_selftest.restype = ctypes.c_int
    lib.sr_selftest.argtypes = []
    lib.sr_plan_create.restype = ctypes.c_int
    lib.sr_plan_create.argtypes = [
        ctypes.POINTER(SrTensor), ctypes.c_int32,
        ctypes.POINTER(SrTensor), ctypes.c_int32,
        ctypes.c_int32,
        ctypes.POINTER(SrPiece), ctypes.c_int32,
        ctypes.POINTER(SrPlanOptions),
        ctypes.POINTER(vp),
    ]
    lib.sr_plan_peer_bytes.restype = ctypes.c_int
    lib.sr_plan_peer_bytes.argtypes = [vp, ctypes.c_int32, ctypes.POINTER(ctypes.c_uint64)]
    lib.sr_plan_piece_offset.restype = ctypes.c_int
    lib.sr_plan_piece_offset.argtypes = [vp, ctypes.c_int32, ctypes.POINTER(ctypes.c_uint64)]
    lib.sr_plan_info_get.restype = ctypes.c_int
    lib.sr_plan_info_get.argtypes = [vp, ctypes.POINTER(SrPlanInfo)]
    lib.sr_pack.restype = ctypes.c_int
    lib.sr_pack.argtypes = [vp, vp, vp, vp]   # pointer arrays: ctypes arrays or addresses
    lib.sr_unpack.restype = ctypes.c_int
    lib.sr_unpack.argtypes = [vp, vp, vp, vp]   # pointer arrays: ctypes arrays or addresses
    lib.sr_gather.restype = ctypes.c_int
    lib.sr_gather.argtypes = [vp, vp, vp, vp]   # pointer arrays: ctypes arrays or addresses
    lib.sr_gather_noalloc.restype = ctypes.c_int
    lib.sr_gather_noalloc.argtypes = [vp, vp, vp, vp]   # pointer arrays: ctypes arrays or addresses
    lib.sr_prepare.restype = ctypes.c_int
    lib.sr_prepare.argtypes = [vp]
    lib.sr_stage_pack.restype = ctypes.c_int
    lib.sr_stage_pack.argtypes = [vp, vp, vp, vp]   # pointer arrays: ctypes arrays or addresses
    lib.sr_pack_host.restype = ctypes.c_int
    lib.sr_pack_host.argtypes = [vp, vp, vp]   # pointer arrays: ctypes arrays or addresses
    lib.sr_download.restype = ctypes.c_int
    lib.sr_download.argtypes = [vp, vp, vp, ctypes.c_int32, vp]
    lib.sr_set_host_threads.restype = ctypes.c_int
    lib.sr_set_host_threads.argtypes = [ctypes.c_int32]
    lib.sr_stage_counters_get.restype = ctypes.c_int
    lib.sr_stage_counters_get.argtypes = [ctypes.POINTER(SrStageCounters)]
    lib.sr_plan_destroy.restype = None
    lib.sr_plan_destroy.argtypes = [vp]
    i64 = ctypes.c_int64
    lib.sr_schedule.restype = ctypes.c_int
    lib.sr_schedule.argtypes = [vp, i64, i64, vp, i64, i64, i64, vp, i64, ctypes.POINTER(i64)]
    lib.sr_lower.restype = ctypes.c_int
    lib.sr_lower.argtypes = [vp, i64, vp, i64, vp, i64, vp, ctypes.POINTER(ctypes.POINTER(SrLowering))]
    lib.sr_lowering_destroy.restype = None
    lib.sr_lowering_destroy.argtypes = [ctypes.POINTER(SrLowering)]
    lib.sr_handoff_alloc.restype = ctypes.c_int
    lib.sr_handoff_alloc.argtypes = [ctypes.c_uint64, ctypes.POINTER(vp), ctypes.POINTER(SrIpcHandle)]
    lib.sr_handoff_free.restype = ctypes.c_int
    lib.sr_handoff_free.argtypes = [vp]
    lib.sr_handoff_open.restype = ctypes.c_int
    lib.sr_handoff_open.argtypes = [ctypes.POINTER(SrIpcHandle), ctypes.POINTER(vp)]
    lib.sr_handoff_close.restype = ctypes.c_int
    lib.sr_handoff_close.argtypes = [vp]


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it is missing."""
    global _lib
    if _lib is None:
        path = Path(os.environ.get("SUIKA_RESHARD_LIB", str(LIB_PATH)))
        if not path.exists():
            raise RuntimeError(
                f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `python suika_amd/build.py`; there is no fallback path")
        handle = ctypes.CDLL(str(path))
        _declare(handle)
        if handle.sr_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{path}: ABI {handle.sr_abi_version()} != expected {ABI_VERSION}")
        _lib = handle
    return _lib


_host = None


def host():
    """Load (once) and return the host extension (per-tensor work of the
    drop-in operator, on torch's C++ API); raise if it is missing."""
    global _host
    if _host is None:
        import importlib.util

        import torch  # noqa: F401  (its libraries back the extension)
        # the extension calls the library: it binds (by soname) to the copy
        # loaded here, so both sides share one instance of its state
        lib()
        path = Path(os.environ.get("SUIKA_HOST_LIB", str(HOST_PATH)))
        if not path.exists():
            raise RuntimeError(
                f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `python suika_amd/build.py`; there is no fallback path")
        spec = importlib.util.spec_from_file_location("_suika_host", str(path))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _host = mod
    return _host


def stage_counters() -> SrStageCounters:
    """The library's staging totals (sr_stage_counters_get)."""
    out = SrStageCounters()
    check(lib().sr_stage_counters_get(ctypes.byref(out)), "sr_stage_counters_get")
    return out


def last_error(handle: Optional[ctypes.CDLL] = None) -> str:
    return (handle or lib()).sr_last_error().decode("utf-8", "replace")


def check(rc: int, what: str, handle: Optional[ctypes.CDLL] = None) -> None:
    """Raise the Python exception matching a library status code."""
    if rc == SR_OK:
        return
    msg = f"{what}: {STATUS_NAMES.get(rc, rc)}: {last_error(handle)}"
    if rc in (SR_EHIP, SR_ENOMEM):
        raise ReshardError(msg)
    raise PlanError(msg)

"""The C ABI library: loads, exports what include/*.h declares, and rejects
invalid plans before anything reaches a GPU (host-only calls)."""
import ctypes
import re
from pathlib import Path

import pytest

from suika_amd import _lib

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("*.h"))


def header_functions():
    found = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        found |= set(re.findall(r"\b(sr_[a-z_0-9]+)\s*\(", text))
    return sorted(found)


def test_library_loads_and_version():
    L = _lib.lib()
    assert L.sr_abi_version() == _lib.ABI_VERSION == 5


def test_every_declared_symbol_is_exported():
    declared = header_functions()
    assert declared, "no declarations parsed"
    assert sorted(_lib.EXPORTED_SYMBOLS) == declared
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared:
        assert hasattr(raw, name), f"{name} not exported"


def test_selftest_division_constants():
    assert _lib.lib().sr_selftest() == 0, _lib.last_error()


def _plan(src, dst, n_peers, pieces, options=None):
    L = _lib.lib()
    s = (_lib.SrTensor * max(1, len(src)))(*[_lib.SrTensor(r, c, d, 0) for r, c, d in src])
    d = (_lib.SrTensor * max(1, len(dst)))(*[_lib.SrTensor(r, c, t, 0) for r, c, t in dst])
    p = (_lib.SrPiece * max(1, len(pieces)))(*pieces)
    h = ctypes.c_void_p()
    opt = ctypes.byref(options) if options is not None else None
    rc = L.sr_plan_create(s, len(src), d, len(dst), n_peers, p, len(pieces), opt, ctypes.byref(h))
    return rc, h


def piece(kind=_lib.SR_PIECE_COPY, peer=0, src=0, dst=0, dst2=-1, rows=4, cols=8,
          sr=0, sc=0, dr=0, dc=0):
    return _lib.SrPiece(kind, peer, src, dst, dst2, 0, rows, cols, sr, sc, dr, dc)


F32, BF16 = _lib.SR_DT_F32, _lib.SR_DT_BF16


def test_valid_plan_and_buffer_layout():
    # dst [4, 16] = two [4, 8] column halves from two sources (a row-parallel merge)
    rc, h = _plan([(4, 8, F32), (4, 8, F32)], [(4, 16, F32)], 2,
                  [piece(src=0, peer=0, dc=0), piece(src=1, peer=1, dc=8)])
    assert rc == 0, _lib.last_error()
    L = _lib.lib()
    b = ctypes.c_uint64()
    assert L.sr_plan_peer_bytes(h, 0, ctypes.byref(b)) == 0 and b.value == 4 * 8 * 4
    info = _lib.SrPlanInfo()
    assert L.sr_plan_info_get(h, ctypes.byref(info)) == 0
    assert info.n_pieces == 2 and info.pack_bytes_read == 256 and info.unpack_bytes_written == 256
    assert info.gather_bytes_read == 256 and info.gather_bytes_written == 256
    off = ctypes.c_uint64()
    assert L.sr_plan_piece_offset(h, 1, ctypes.byref(off)) == 0 and off.value == 0
    L.sr_plan_destroy(h)


def test_buffer_offsets_are_256_aligned():
    pcs = [piece(src=0, peer=0, rows=1, cols=3, sr=i, dr=i) for i in range(4)]
    rc, h = _plan([(4, 3, F32)], [(4, 3, F32)], 1, pcs)
    assert rc == 0, _lib.last_error()
    L = _lib.lib()
    offs = []
    for k in range(4):
        o = ctypes.c_uint64()
        L.sr_plan_piece_offset(h, k, ctypes.byref(o))
        offs.append(o.value)
    assert offs == [0, 256, 512, 768]
    b = ctypes.c_uint64()
    L.sr_plan_peer_bytes(h, 0, ctypes.byref(b))
    assert b.value == 768 + 12
    L.sr_plan_destroy(h)


@pytest.mark.parametrize("bad,code", [
    (dict(sr=1), _lib.SR_EBOUNDS),                 # source rows past the end
    (dict(dc=1), _lib.SR_EBOUNDS),                 # destination cols past the end
    (dict(peer=3), _lib.SR_EINVAL),                # no such peer
    (dict(src=5), _lib.SR_EINVAL),                 # no such source slot
    (dict(rows=0), _lib.SR_EINVAL),                # empty region
    (dict(kind=7), _lib.SR_EINVAL),                # unknown kind
    (dict(dst2=0), _lib.SR_EINVAL),                # COPY with a second target
])
def test_invalid_pieces_rejected(bad, code):
    kw = dict(src=0, peer=0)
    kw.update(bad)
    rc, h = _plan([(4, 8, F32)], [(4, 8, F32)], 1, [piece(**kw)])
    assert rc == code, (rc, _lib.last_error())
    assert not h.value
    assert _lib.last_error()


def test_dtype_mismatch_rejected():
    rc, _ = _plan([(4, 8, F32)], [(4, 8, BF16)], 1, [piece()])
    assert rc == _lib.SR_EDTYPE


def test_overlap_and_holes_rejected():
    rc, _ = _plan([(4, 8, F32)], [(4, 8, F32)], 1, [piece(), piece(rows=1, cols=1, dr=2, dc=2)])
    assert rc == _lib.SR_EOVERLAP and "overlapping" in _lib.last_error()
    rc, _ = _plan([(4, 8, F32)], [(4, 8, F32)], 1, [piece(rows=3)])
    assert rc == _lib.SR_EOVERLAP and "cover" in _lib.last_error()
    opt = _lib.SrPlanOptions(0, 0, _lib.SR_OPT_SKIP_COVERAGE, 0)
    rc, h = _plan([(4, 8, F32)], [(4, 8, F32)], 1, [piece(rows=3)], options=opt)
    assert rc == 0
    _lib.lib().sr_plan_destroy(h)


def test_coverage_checked_per_destination():
    """Coverage is kept per destination slot, whatever order the pieces come in:
    the same region of two slots is no overlap, and a fault in one slot names it."""
    src, dst = [(4, 8, F32)], [(4, 8, F32)] * 3
    halves = lambda d: [piece(dst=d, rows=2), piece(dst=d, rows=2, sr=2, dr=2)]
    # slots interleaved (2, 0, 1, 2, 0, 1), every slot covered once: valid
    pcs = [p for pair in zip(halves(2), halves(0), halves(1)) for p in pair]
    rc, h = _plan(src, dst, 1, pcs)
    assert rc == 0, _lib.last_error()
    _lib.lib().sr_plan_destroy(h)
    # slot 1 gets a third piece over its first half: the overlap names slot 1
    rc, _ = _plan(src, dst, 1, pcs + [piece(dst=1, rows=1, cols=1)])
    assert rc == _lib.SR_EOVERLAP
    assert _lib.last_error().startswith("dst[1]: pieces") and "overlapping" in _lib.last_error()
    # slot 0 has no pieces at all: reported as covering none of its elements
    rc, _ = _plan(src, dst, 1, halves(1) + halves(2))
    assert rc == _lib.SR_EOVERLAP
    assert "dst[0]: pieces cover 0 of 32 elements" in _lib.last_error()
    # the last slot short by a half
    rc, _ = _plan(src, dst, 1, halves(0) + halves(1) + halves(2)[:1])
    assert rc == _lib.SR_EOVERLAP
    assert "dst[2]: pieces cover 16 of 32 elements" in _lib.last_error()


def test_recast_and_zero_rules():
    # f32 source -> f32 dst 0 and bf16 dst 1; zero fill the remaining rows of both
    pcs = [piece(kind=_lib.SR_PIECE_RECAST, dst=0, dst2=1, rows=3),
           piece(kind=_lib.SR_PIECE_ZERO, src=-1, dst=0, rows=1, dr=3),
           piece(kind=_lib.SR_PIECE_ZERO, src=-1, dst=1, rows=1, dr=3)]
    rc, h = _plan([(4, 8, F32)], [(4, 8, F32), (4, 8, BF16)], 1, pcs)
    assert rc == 0, _lib.last_error()
    info = _lib.SrPlanInfo()
    _lib.lib().sr_plan_info_get(h, ctypes.byref(info))
    assert info.unpack_bytes_written == 3 * 8 * 4 + 3 * 8 * 2 + 8 * 4 + 8 * 2
    assert info.gather_bytes_written == info.unpack_bytes_written
    assert info.gather_bytes_read == 3 * 8 * 4
    _lib.lib().sr_plan_destroy(h)
    # bf16 source cannot be recast
    rc, _ = _plan([(4, 8, BF16)], [(4, 8, F32), (4, 8, BF16)], 1,
                  [piece(kind=_lib.SR_PIECE_RECAST, dst=0, dst2=1)])
    assert rc == _lib.SR_EDTYPE
    # ZERO takes no source
    rc, _ = _plan([(4, 8, F32)], [(4, 8, F32)], 1, [piece(kind=_lib.SR_PIECE_ZERO, src=0)])
    assert rc == _lib.SR_EINVAL


def test_options_validation():
    for opt in (_lib.SrPlanOptions(3000, 0, 0, 0), _lib.SrPlanOptions(0, 0, 0x80, 0),
                _lib.SrPlanOptions(0, 0, 0x40, 0), _lib.SrPlanOptions(0, 0, 0, 1)):
        rc, _ = _plan([(4, 8, F32)], [(4, 8, F32)], 1, [piece()], options=opt)
        assert rc == _lib.SR_EINVAL
    every = (_lib.SR_OPT_TEMPORAL | _lib.SR_OPT_SKIP_COVERAGE | _lib.SR_OPT_PIECE_ORDER |
             _lib.SR_OPT_NO_XCD_INTERLEAVE | _lib.SR_OPT_NO_ROW_GROUPS | _lib.SR_OPT_GATHER_ONLY)
    rc, h = _plan([(4, 8, F32)], [(4, 8, F32)], 1, [piece()], options=_lib.SrPlanOptions(0, 0, every, 0))
    assert rc == _lib.SR_OK, _lib.last_error()
    _lib.lib().sr_plan_destroy(h)


def test_gather_only_plan_refuses_pack_and_unpack():
    """A gather-only plan keeps the buffer layout it reports but builds no
    pack / unpack phase; those calls fail before touching any pointer."""
    L = _lib.lib()
    rc, h = _plan([(4, 8, F32), (4, 8, F32)], [(4, 16, F32)], 2,
                  [piece(src=0, peer=0, dc=0), piece(src=1, peer=1, dc=8)],
                  options=_lib.SrPlanOptions(0, 0, _lib.SR_OPT_GATHER_ONLY, 0))
    assert rc == _lib.SR_OK, _lib.last_error()
    info = _lib.SrPlanInfo()
    assert L.sr_plan_info_get(h, ctypes.byref(info)) == 0
    assert info.gather_tiles > 0 and info.pack_tiles == 0 and info.unpack_tiles == 0
    b = ctypes.c_uint64()
    assert L.sr_plan_peer_bytes(h, 1, ctypes.byref(b)) == 0 and b.value == 4 * 8 * 4
    null = (ctypes.c_void_p * 2)(None, None)
    assert L.sr_pack(h, null, null, None) == _lib.SR_EINVAL and "gather-only" in _lib.last_error()
    assert L.sr_unpack(h, null, null, None) == _lib.SR_EINVAL and "gather-only" in _lib.last_error()
    L.sr_plan_destroy(h)


def test_tile_counts():
    """Tiles per phase = sum over items of ceil(item bytes / tile_bytes); a
    strided item counts its source bytes, a ZERO item its destination bytes."""
    # dst [64, 3000] f32: column bands of 1000 and 1500 from two peers
    # (strided on the destination) and a band of 500 zero-filled columns.
    src = [(64, 1000, F32), (64, 2000, F32)]
    pcs = [piece(src=0, peer=0, rows=64, cols=1000, dc=0),
           piece(src=1, peer=1, rows=64, cols=1500, dc=1000),
           piece(kind=_lib.SR_PIECE_ZERO, peer=0, src=-1, rows=64, cols=500, dc=2500)]
    tile = 4096
    rc, h = _plan(src, [(64, 3000, F32)], 2, pcs, options=_lib.SrPlanOptions(tile, 0, 0, 0))
    assert rc == _lib.SR_OK, _lib.last_error()
    info = _lib.SrPlanInfo()
    assert _lib.lib().sr_plan_info_get(h, ctypes.byref(info)) == 0
    ceil = lambda n: -(-n // tile)  # noqa: E731
    copies = ceil(64 * 1000 * 4) + ceil(64 * 1500 * 4)
    zero = ceil(64 * 500 * 4)
    assert info.pack_tiles == copies
    assert info.unpack_tiles == copies + zero
    assert info.gather_tiles == copies + zero
    _lib.lib().sr_plan_destroy(h)


def test_tile_counts_recast():
    """A RECAST item that writes the f32 and the bf16 copy moves 2.5x its
    source bytes and is cut into tiles of half the tile size; a bf16-only
    RECAST item (2 + 4 bytes per element moved, less than a copy's 8) keeps
    the full tile."""
    tile = 4096
    # [64, 1000] f32 master -> f32 copy + bf16 copy; [64, 700] f32 -> bf16 only
    src = [(64, 1000, F32), (64, 700, F32)]
    dst = [(64, 1000, F32), (64, 1000, _lib.SR_DT_BF16), (64, 700, _lib.SR_DT_BF16)]
    pcs = [piece(kind=_lib.SR_PIECE_RECAST, src=0, peer=0, dst=0, dst2=1, rows=64, cols=1000),
           piece(kind=_lib.SR_PIECE_RECAST, src=1, peer=0, dst=-1, dst2=2, rows=64, cols=700)]
    rc, h = _plan(src, dst, 1, pcs, options=_lib.SrPlanOptions(tile, 0, 0, 0))
    assert rc == _lib.SR_OK, _lib.last_error()
    info = _lib.SrPlanInfo()
    assert _lib.lib().sr_plan_info_get(h, ctypes.byref(info)) == 0
    ceil = lambda n, t: -(-n // t)  # noqa: E731
    assert info.pack_tiles == ceil(64 * 1000 * 4, tile) + ceil(64 * 700 * 4, tile)
    want = ceil(64 * 1000 * 4, tile // 2) + ceil(64 * 700 * 4, tile)
    assert info.unpack_tiles == want
    assert info.gather_tiles == want
    _lib.lib().sr_plan_destroy(h)


def test_python_errors_are_assertion_errors():
    with pytest.raises(AssertionError):
        _lib.check(_lib.SR_EBOUNDS, "x")
    with pytest.raises(_lib.ReshardError):
        _lib.check(_lib.SR_EHIP, "x")


def test_missing_library_fails_loudly(tmp_path):
    """Without the built library every entry point raises: there is no CPU
    or torch fallback.  Run in a child interpreter so this process keeps its
    loaded library."""
    import os
    import subprocess
    import sys
    code = ("import torch\n"
            "from suika_amd import execute_param_transfer\n"
            "try:\n"
            "    execute_param_transfer([], {}, torch.device('cuda', 0), [('param', 'normal')], rank=0)\n"
            "except RuntimeError as e:\n"
            "    assert 'missing' in str(e) and 'no fallback' in str(e), e\n"
            "    print('raised')\n")
    env = dict(os.environ, SUIKA_RESHARD_LIB=str(tmp_path / "absent.so"))
    root = Path(__file__).resolve().parents[1]
    out = subprocess.run([sys.executable, "-c", code], cwd=root, env=env, capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0 and "raised" in out.stdout, out.stderr[-2000:]


def test_c_caller(tmp_path):
    """The headers and library serve a plain C11 program (the FFI view a
    cgo / JNI / N-API binding has), not only ctypes: schedule, plan, layout."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler on this host")
    root = Path(__file__).resolve().parents[1]
    exe = tmp_path / "abi_host_calls"
    cmd = [gcc, "-std=c11", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
           f"-I{root / 'include'}", "-I/opt/rocm/include", str(root / "tests" / "c" / "abi_host_calls.c"),
           f"-L{_lib.LIB_PATH.parent}", "-lsuika_reshard", f"-Wl,-rpath,{_lib.LIB_PATH.parent}",
           "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stdout + out.stderr
    lines = out.stdout.splitlines()
    assert lines == [
        f"abi {_lib.ABI_VERSION}",
        "peer_bytes 128 128",          # 4 x 8 f32 per peer
        "piece1_offset 0",             # first (only) piece of peer 1
        "pieces 2 peers 2 pack_bytes_read 256",
        f"hole {_lib.SR_EOVERLAP} null",
        "message mentions coverage",
        "schedule 0 ops 2",
        "op 0 -> 0 piece 0/2",
        "op 1 -> 0 piece 1/2",
        "lower 0 src 2 dst 1 pieces 2 peers 2",
        "piece peer 0 src 0 cols 8 dst_col 0",   # column halves of the row-parallel merge
        "piece peer 1 src 1 cols 8 dst_col 8",
        "planned 0 peer1_bytes 128",
    ], out.stdout


def test_overlapping_objects_rejected_before_launch():
    """Objects one launch writes must be disjoint from each other and from
    what it reads.  The check runs on the host before any HIP call, so fake
    addresses suffice here."""
    L = _lib.lib()
    vp = ctypes.c_void_p
    # two [4, 8] f32 destinations, each filled from its own source
    rc, h = _plan([(4, 8, F32), (4, 8, F32)], [(4, 8, F32), (4, 8, F32)], 2,
                  [piece(src=0, peer=0, dst=0), piece(src=1, peer=1, dst=1)])
    assert rc == _lib.SR_OK, _lib.last_error()
    base = 1 << 40
    src = (vp * 2)(base, base + 4096)
    # destinations overlap each other (128-byte objects 64 bytes apart)
    dst = (vp * 2)(base + 8192, base + 8192 + 64)
    assert L.sr_gather(h, src, dst, None) == _lib.SR_EOVERLAP
    assert "dst_ptrs[0] and dst_ptrs[1]" in _lib.last_error()
    # a destination overlaps a source (in place)
    dst = (vp * 2)(base + 64, base + 8192)
    assert L.sr_gather(h, src, dst, None) == _lib.SR_EOVERLAP
    assert "src_ptrs[0] is read" in _lib.last_error()
    # pack: two peer buffers overlapping
    bufs = (vp * 2)(base + 8192, base + 8192 + 32)
    assert L.sr_pack(h, src, bufs, None) == _lib.SR_EOVERLAP
    assert "peer_bufs[0] and peer_bufs[1]" in _lib.last_error()
    L.sr_plan_destroy(h)


def test_host_extension_loads():
    """The host extension (per-tensor work of the drop-in operator) is built
    in-tree (or is the one SUIKA_HOST_LIB names, as in the sanitizer run)
    and exposes its two entry points."""
    import os
    mod = _lib.host()
    assert callable(mod.collect_sources) and callable(mod.alloc_dst)
    want = Path(os.environ.get("SUIKA_HOST_LIB", str(_lib.HOST_PATH)))
    assert Path(mod.__file__).resolve() == want.resolve()


def test_missing_host_extension_raises(tmp_path):
    """No fallback: without the host extension the planner raises."""
    import os
    import subprocess
    import sys
    code = ("from suika_amd import _lib\n"
            "try:\n"
            "    _lib.host()\n"
            "except RuntimeError as e:\n"
            "    assert 'missing' in str(e) and 'no fallback' in str(e), e\n"
            "    print('raised')\n")
    env = dict(os.environ, SUIKA_HOST_LIB=str(tmp_path / "absent.so"))
    root = Path(__file__).resolve().parents[1]
    out = subprocess.run([sys.executable, "-c", code], cwd=root, env=env, capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0 and "raised" in out.stdout, out.stderr[-2000:]


def test_host_arena_views_checks_rows():
    """arena_views builds typed views of one byte buffer and rejects rows
    outside it or misaligned for their dtype."""
    import numpy as np
    import torch
    mod = _lib.host()
    buf = torch.arange(64, dtype=torch.uint8)
    rows = np.array([[0, 2, 2, 4] + [0] * 6, [32, 1, 8] + [0] * 7], dtype=np.int64)
    out = mod.arena_views(buf, ["a", "b"], ["f32", "u8"], rows, [torch.float32, torch.uint8])
    assert out["a"]["f32"].shape == (2, 4) and out["a"]["f32"].dtype == torch.float32
    assert out["a"]["f32"].untyped_storage().data_ptr() == buf.untyped_storage().data_ptr()
    assert out["b"]["u8"].tolist() == list(range(32, 40))
    with pytest.raises(ValueError, match="outside the buffer or misaligned"):
        mod.arena_views(buf, ["a"], ["f"], np.array([[60, 1, 2] + [0] * 7], dtype=np.int64), [torch.float32])
    with pytest.raises(ValueError, match="outside the buffer or misaligned"):
        mod.arena_views(buf, ["a"], ["f"], np.array([[2, 1, 2] + [0] * 7], dtype=np.int64), [torch.float32])


@pytest.mark.parametrize("seed", range(100))
def test_plan_create_rejects_corrupted_tables_without_crashing(seed):
    """Real lowerings with random fields of their sr_piece / sr_tensor tables
    replaced by extreme or off-by-one values: sr_plan_create returns a status
    in bounded time and never crashes or reads outside its tables."""
    import random
    import time

    import numpy as np
    import torch
    from suika_amd.plan import ReshardPlan, SlotSpec
    from tests.test_fuzz import random_case
    rng = random.Random(seed)
    w = random_case(seed)
    ops = w.ops()
    dt = w.dtypes
    specs = {(op.src_rank, op.param_name, f): SlotSpec(tuple(op.src_meta.actual_shape()), dt[f])
             for op in ops for f in w.src_fields}
    plan = ReshardPlan(ops, specs, list(w.src_fields), recast=w.recast_map)
    pieces, src, dst = plan._piece_arr.copy(), plan._src_arr.copy(), plan._dst_arr.copy()
    n_peers = len(plan.peers)
    plan.close()
    L = _lib.lib()
    extremes = [0, 1, 2, 7, (1 << 31) - 1, (1 << 62), (1 << 64) - 1]
    for trial in range(20):
        p2, s2, d2 = pieces.copy(), src.copy(), dst.copy()
        for _ in range(rng.randint(1, 3)):
            table = rng.choice([p2, p2, s2, d2]) if len(s2) else p2
            if not len(table):
                continue
            i = rng.randrange(len(table))
            field = rng.choice(table.dtype.names)
            if np.issubdtype(table.dtype[field], np.signedinteger):
                table[field][i] = rng.choice([-1, 0, 1, 3, 1 << 30, int(table[field][i]) + 1])
            else:
                table[field][i] = rng.choice(extremes + [(int(table[field][i]) + 1) % (1 << 64)])
        h = ctypes.c_void_p()
        t0 = time.perf_counter()
        rc = L.sr_plan_create(_lib.as_tensors(s2), len(s2), _lib.as_tensors(d2), len(d2), n_peers,
                              _lib.as_pieces(p2), len(p2), None, ctypes.byref(h))
        assert time.perf_counter() - t0 < 5.0
        assert rc <= 0
        if rc == 0:
            L.sr_plan_destroy(h)
        else:
            assert not h.value


def test_gather_noalloc_rejects_plans_beyond_the_scratch():
    """A plan whose gather tables exceed SR_SCRATCH_BYTES is refused with
    SR_ENOMEM before any device call (so this runs without a GPU); a larger
    tile size brings the same transfer within the limit."""
    assert _lib.SCRATCH_BYTES == 64 << 20
    L = _lib.lib()
    rows, cols = 1 << 20, 4096            # 16 GiB of f32: 4 Mi tiles of 4 KiB = 96 MiB of tiles
    small = _lib.SrPlanOptions(4096, 0, 0, 0)
    rc, h = _plan([(rows, cols, F32)], [(rows, cols, F32)], 1, [piece(rows=rows, cols=cols)], small)
    assert rc == 0, _lib.last_error()
    null = (ctypes.c_void_p * 1)(None)
    assert L.sr_gather_noalloc(h, null, null, None) == _lib.SR_ENOMEM
    msg = _lib.last_error()
    assert "scratch holds 67108864" in msg and "tile_bytes" in msg, msg
    L.sr_plan_destroy(h)
    # 64 KiB tiles: 256 Ki tiles = 6 MiB; past the size check, the null
    # pointers are the next thing refused -- still before any device call
    rc, h = _plan([(rows, cols, F32)], [(rows, cols, F32)], 1, [piece(rows=rows, cols=cols)],
                  _lib.SrPlanOptions(65536, 0, 0, 0))
    assert rc == 0, _lib.last_error()
    assert L.sr_gather_noalloc(h, null, null, None) == _lib.SR_EINVAL
    assert "src_ptrs[0] is null" in _lib.last_error()
    L.sr_plan_destroy(h)
    assert L.sr_gather_noalloc(None, null, null, None) == _lib.SR_EINVAL

"""The same-GPU hand-off on the host: the C ABI's argument checks (no device
call is made for a rejected argument) and the packing layout."""
import ctypes

import pytest

from suika_amd import _lib
from suika_amd.handoff import ALIGN, pack_layout


def test_handoff_abi_rejects_bad_arguments_before_any_device_call():
    L = _lib.lib()
    ptr, h = ctypes.c_void_p(), _lib.SrIpcHandle()
    assert ctypes.sizeof(h) == 64
    assert L.sr_handoff_alloc(0, ctypes.byref(ptr), ctypes.byref(h)) == _lib.SR_EINVAL
    assert L.sr_handoff_alloc(_lib.HANDOFF_MAX_BYTES + 1, ctypes.byref(ptr), ctypes.byref(h)) == _lib.SR_EINVAL
    assert "outside 1..2146435072" in _lib.last_error()
    assert L.sr_handoff_alloc(64, None, ctypes.byref(h)) == _lib.SR_EINVAL
    assert L.sr_handoff_open(None, ctypes.byref(ptr)) == _lib.SR_EINVAL
    assert L.sr_handoff_open(ctypes.byref(h), None) == _lib.SR_EINVAL
    assert L.sr_handoff_close(None) == _lib.SR_EINVAL
    assert L.sr_handoff_free(None) == _lib.SR_EINVAL
    assert _lib.HANDOFF_MAX_BYTES == (2 << 30) - (1 << 20) and _lib.HANDOFF_MAX_BYTES < 2 << 30


def test_pack_layout_aligned_chunks_within_limits():
    sizes_in = [100, 1000, 3000, 5000, 70000, 10, 1]
    where, sizes = pack_layout(sizes_in, chunk_bytes=8192)
    ends = {}
    for n, (c, off) in zip(sizes_in, where):
        assert off % ALIGN == 0
        assert off + n <= sizes[c]
        ends.setdefault(c, []).append((off, off + n))
    for c, spans in ends.items():
        spans.sort()
        assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:])), "tensors of a chunk overlap"
        assert sizes[c] == spans[-1][1], "a chunk ends where its last tensor does"
        assert sizes[c] <= 8192 or len(spans) == 1, "only a lone tensor exceeds the chunk size"
    assert [c for c, _ in where] == [0, 0, 0, 1, 2, 3, 3]
    assert where[4] == (2, 0) and sizes[2] == 70000     # larger than a chunk: alone


def test_pack_layout_refuses_tensors_beyond_the_limit():
    with pytest.raises(AssertionError, match="does not fit one hand-off allocation"):
        pack_layout([_lib.HANDOFF_MAX_BYTES + 1])
    with pytest.raises(AssertionError):
        pack_layout([0])
    where, sizes = pack_layout([_lib.HANDOFF_MAX_BYTES, 1])
    assert sizes == [_lib.HANDOFF_MAX_BYTES, 1] and where == [(0, 0), (1, 0)]


def test_destination_bytes_sum_the_new_ranks_shards():
    """The bytes a new rank reserves beside the old state: every name of its
    layout once, its shard's elements times each field's item size from the
    old ranks' records, each tensor rounded up to 256 bytes."""
    from suika_amd import schedule_param_transfer
    from suika_amd.handoff import _destination_bytes
    from suika_amd.workloads import CONFIGS
    w = CONFIGS["gpt125m_tp2_tp4"]
    spl, tpl = w.layouts()
    ops = schedule_param_transfer(spl, tpl)
    fields = {"param": "torch.bfloat16", "exp_avg": "torch.float32", "exp_avg_sq": "torch.float32"}
    records = [{"rank": r, "tensors": {n: {f: (0, 0, tuple(m.actual_shape()), dt) for f, dt in fields.items()}
                                       for n, m in metas.items()}}
               for r, metas in spl.layout.items()]
    per_elem = {"torch.bfloat16": 2, "torch.float32": 4}
    for rank, metas in tpl.layout.items():
        want = 0
        for n, m in metas.items():
            numel = 1
            for d in m.actual_shape():
                numel *= int(d)
            want += sum((numel * per_elem[dt] + ALIGN - 1) // ALIGN * ALIGN for dt in fields.values())
        assert _destination_bytes(ops, rank, records) == want, rank
    # a rank with no ops of its own needs nothing
    assert _destination_bytes([op for op in ops if op.dst_rank != 0], 0, records) == 0

"""pad_decode_launch_noalloc: the allocation-free entry point (static device scratch).

Called through the C ABI (ctypes) with raw device pointers.  Its output must
equal pad_decode_launch()'s on the same inputs (same kernel, same plan, so
the bits agree) and match the fp32 oracle at the parity tolerance - on two
calls in a row, the second with a smaller input, so that the static scratch
(partials and arrival counters left by the first call) is reused.  A shape
whose plan needs more scratch than the static array holds is refused
without a launch.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from paged_attention_decode_amd import _native, heuristics
from tests.helpers import assert_parity, make_cache, shuffled_table

pytestmark = pytest.mark.gpu

NOALLOC_WORKSPACE_BYTES = 48 * 1024 * 1024 - 256 * 1024  # PAD_NOALLOC_WORKSPACE_BYTES
NOALLOC_COUNTERS = 65536  # PAD_NOALLOC_COUNTERS


def _case(lens, hq, hkv, d, ps, seed):
    bt, n = shuffled_table(lens, ps, spare_pages=2, extra_cols=1, seed=seed)
    k, v = make_cache(n, ps, hkv, d, seed=seed)
    q = torch.randn(len(lens), hq, d, generator=torch.Generator().manual_seed(seed))
    sl = torch.tensor(lens, dtype=torch.int32)
    dev = [q.half().cuda(), k.half().cuda(), v.half().cuda(), bt.cuda(), sl.cuda()]
    return dev, (q, k, v, bt, sl)


def _with_workspace(lib, dev, out, splits, stream):
    """The existing entry point, with caller-owned scratch."""
    dm = _native.dims_for(*dev, out)
    wsb, nc = ctypes.c_size_t(), ctypes.c_int64()
    assert lib.pad_decode_workspace_bytes(ctypes.byref(dm), splits, 0, ctypes.byref(wsb)) == 0
    assert lib.pad_decode_counters_needed(ctypes.byref(dm), splits, 0, ctypes.byref(nc)) == 0
    ws = torch.empty(max(wsb.value, 1), dtype=torch.uint8, device="cuda")
    cnt = torch.zeros(max(nc.value, 1), dtype=torch.int32, device="cuda")
    q, k, v, bt, sl = dev
    st = lib.pad_decode_launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                               out.data_ptr(), ws.data_ptr(), wsb.value, cnt.data_ptr(), cnt.numel(),
                               ctypes.byref(dm), 1.0 / q.shape[2] ** 0.5, splits, stream)
    assert st == 0, lib.pad_status_string(st)
    return ws, cnt


def _noalloc(lib, dev, out, splits, stream):
    q, k, v, bt, sl = dev
    dm = _native.dims_for(*dev, out)
    return lib.pad_decode_launch_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                                         out.data_ptr(), ctypes.byref(dm), 1.0 / q.shape[2] ** 0.5, splits, stream)


# (large first call, smaller second call, split count): the heuristic on a
# batch that splits every sequence; an explicit count whose units merge in
# two levels (per-group counters); the in-kernel planner on ragged lengths.
CASES = [
    (([4096] * 16, 12, 2, 128, 16), ([900, 33, 2048], 12, 2, 128, 16), 0),
    (([20000, 4000], 8, 1, 128, 16), ([3000], 8, 1, 128, 16), 64),
    (([5000, 1, 777, 3000, 64, 8000], 12, 2, 128, 32), ([100, 2500], 12, 2, 128, 32), 0),
]


@pytest.mark.parametrize("first,second,splits", CASES)
def test_noalloc_matches_launch_on_two_calls(first, second, splits):
    from oracle.reference import decode_fp16_protocol

    lib = _native.capi()
    stream = torch.cuda.Stream()
    for i, shape in enumerate((first, second)):
        dev, cpu = _case(*shape, seed=400 + 10 * i + splits)
        print(f"noalloc call {i}: lens={shape[0][:4]}... heads={shape[1]}/{shape[2]} d={shape[3]} ps={shape[4]} "
              f"splits={splits}", flush=True)
        ref = torch.empty_like(dev[0])
        keep = _with_workspace(lib, dev, ref, splits, stream.cuda_stream)
        out = torch.full_like(dev[0], float("nan"))
        st = _noalloc(lib, dev, out, splits, stream.cuda_stream)
        assert st == 0, lib.pad_status_string(st)
        stream.synchronize()
        del keep
        assert torch.equal(out, ref), f"call {i}: the allocation-free entry point differs from pad_decode_launch"
        assert_parity(out, decode_fp16_protocol(*cpu))


def test_noalloc_refuses_plans_beyond_its_static_scratch():
    lib = _native.capi()
    # 256 sequences of 64/8 heads at head_dim 256: a 4-item-per-unit grid
    # needs ~68 MB of partials, more than the static array holds.
    cus = ctypes.c_int()
    assert lib.pad_device_num_cus(ctypes.byref(cus)) == 0
    m = heuristics.plan(256, 64, 8, 256, 16, 64, 0, cus.value)
    assert m.workspace_bytes > NOALLOC_WORKSPACE_BYTES
    q = torch.zeros(256, 64, 256, dtype=torch.float16, device="cuda")
    k = torch.zeros(8, 16, 8, 256, dtype=torch.float16, device="cuda")
    bt = torch.zeros(256, 64, dtype=torch.int32, device="cuda")
    sl = torch.full((256,), 1024, dtype=torch.int32, device="cuda")
    out = torch.full_like(q, 3.0)
    assert _noalloc(lib, [q, k, k, bt, sl], out, 0, None) == 11
    assert b"static" in lib.pad_status_string(11)
    torch.cuda.synchronize()
    assert bool((out == 3.0).all()), "a refused call must not launch"
    # Explicit split counts past the counter budget are refused the same way.
    m2 = heuristics.plan(256, 64, 8, 128, 16, 64, 300, cus.value)
    assert m2.counters > NOALLOC_COUNTERS or m2.workspace_bytes > NOALLOC_WORKSPACE_BYTES
    q2 = torch.zeros(256, 64, 128, dtype=torch.float16, device="cuda")
    k2 = torch.zeros(8, 16, 8, 128, dtype=torch.float16, device="cuda")
    assert _noalloc(lib, [q2, k2, k2, bt, sl], torch.empty_like(q2), 300, None) == 11

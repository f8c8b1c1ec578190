"""The C ABI of libpa_decode.so (include/pa_decode.h).

CPU tests: the library loads, exports every function the header declares,
and its host-only functions (plan, workspace size, status strings) behave;
the plan agrees with the Python mirror in heuristics.py.  GPU tests call
pad_decode_launch / pad_decode_launch_ex through ctypes with raw device
pointers, a caller-owned workspace and stream, and check parity.
"""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from paged_attention_decode_amd import _native, heuristics
from tests.helpers import assert_parity, make_cache, shuffled_table

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "pa_decode.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(pad_\w+)\s*\(", text, flags=re.M)))


def _dims(batch=4, hq=12, hkv=2, d=128, ps=16, max_pages=256, num_pages=1024):
    dm = _native.PadDims()
    dm.batch, dm.num_q_heads, dm.num_kv_heads, dm.head_dim = batch, hq, hkv, d
    dm.page_size, dm.max_pages, dm.num_pages = ps, max_pages, num_pages
    for i, s in enumerate((hq * d, d, 1)):
        dm.q_stride[i] = s
        dm.out_stride[i] = s
    for i, s in enumerate((ps * hkv * d, hkv * d, d, 1)):
        dm.k_stride[i] = s
        dm.v_stride[i] = s
    dm.bt_stride[0], dm.bt_stride[1] = max_pages, 1
    dm.sl_stride = 1
    return dm


def test_header_declares_the_expected_entry_points():
    assert _declared_functions() == sorted(_native.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _native.capi()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.pad_decode_abi_version() == 6


def test_status_strings():
    lib = _native.capi()
    assert lib.pad_status_string(0) == b"ok"
    for code in range(1, 13):
        assert lib.pad_status_string(code) not in (b"ok", b"unknown status")
    assert lib.pad_status_string(999) == b"unknown status"


@pytest.mark.parametrize("batch,hq,hkv,d,ps,max_pages,splits,cus", [
    (1, 12, 2, 128, 16, 256, 0, 256),
    (16, 12, 2, 128, 16, 256, 0, 256),
    (64, 12, 2, 128, 16, 256, 0, 256),
    (32, 12, 2, 128, 32, 256, 0, 256),
    (1, 32, 8, 128, 16, 8192, 0, 256),
    (256, 64, 8, 128, 16, 2048, 0, 256),
    (1, 12, 2, 128, 16, 64, 0, 256),
    (3, 12, 2, 128, 16, 250, 8, 256),
    (1, 12, 2, 128, 16, 1, 8, 256),
    (2, 32, 2, 256, 16, 40, 0, 80),
    (5, 16, 1, 96, 1, 100, 0, 0),
    (128, 12, 2, 128, 16, 256, 0, 256),
    (512, 12, 2, 128, 16, 256, 0, 256),
    (64, 8, 4, 64, 16, 32, 0, 256),
    (64, 8, 4, 64, 16, 64, 0, 256),
    (8, 16, 1, 256, 16, 512, 0, 256),
    (16, 32, 2, 256, 16, 256, 0, 256),
    (64, 24, 2, 256, 16, 128, 0, 256),
    (1, 11, 1, 256, 16, 512, 0, 256),
    (4, 16, 1, 128, 16, 256, 0, 256),
])
def test_plan_matches_python_mirror(batch, hq, hkv, d, ps, max_pages, splits, cus):
    lib = _native.capi()
    p = _native.PadPlan()
    assert lib.pad_decode_plan(ctypes.byref(_dims(batch, hq, hkv, d, ps, max_pages)), splits, cus, ctypes.byref(p)) == 0
    m = heuristics.plan(batch, hq, hkv, d, ps, max_pages, splits, cus)
    assert (p.num_splits, p.pages_per_split, p.waves_per_group, bool(p.single_pass), p.workspace_bytes,
            p.counters) == (m.num_splits, m.pages_per_split, m.waves_per_group, m.single_pass, m.workspace_bytes,
                            m.counters)
    ws = ctypes.c_size_t()
    assert lib.pad_decode_workspace_bytes(ctypes.byref(_dims(batch, hq, hkv, d, ps, max_pages)), splits, cus,
                                          ctypes.byref(ws)) == 0
    assert ws.value == m.workspace_bytes
    nc = ctypes.c_int64()
    assert lib.pad_decode_counters_needed(ctypes.byref(_dims(batch, hq, hkv, d, ps, max_pages)), splits, cus,
                                          ctypes.byref(nc)) == 0
    assert nc.value == m.counters


def test_plan_mirror_on_random_shapes():
    # 600 seeded shapes across every regime the heuristic has (latency-bound,
    # bandwidth-bound, oversubscribed, explicit splits, narrow rows, head_dim
    # 256, odd page sizes, CU counts other than 256), dense and CSR.
    import random

    lib = _native.capi()
    rng = random.Random(2024)
    for _ in range(600):
        hkv = rng.choice([1, 2, 4, 8])
        hq = hkv * rng.choice([1, 2, 4, 6, 8, 16])
        d = rng.choice([32, 64, 96, 128, 256])
        ps = rng.choice([1, 2, 3, 8, 12, 16, 24, 32, 64])
        batch = rng.choice([1, 2, 3, 8, 16, 33, 64, 100, 256, 300])
        max_pages = rng.choice([1, 5, 64, 256, 1000, 8192])
        splits = rng.choice([0, 0, 0, 1, 4, 64])
        cus = rng.choice([256, 256, 80, 0])
        csr = rng.random() < 0.3
        p = _native.PadPlan()
        fn = lib.pad_decode_plan_csr if csr else lib.pad_decode_plan
        assert fn(ctypes.byref(_dims(batch, hq, hkv, d, ps, max_pages)), splits, cus, ctypes.byref(p)) == 0
        m = heuristics.plan(batch, hq, hkv, d, ps, max_pages, splits, cus, csr=csr)
        got = (p.num_splits, p.pages_per_split, p.waves_per_group, bool(p.single_pass), p.workspace_bytes, p.counters)
        assert got == (m.num_splits, m.pages_per_split, m.waves_per_group, m.single_pass, m.workspace_bytes,
                       m.counters), (batch, hq, hkv, d, ps, max_pages, splits, cus, csr)


@pytest.mark.parametrize("batch,hq,hkv,d,ps,nnz,splits", [
    (1, 12, 2, 128, 16, 256, 0),
    (16, 12, 2, 128, 16, 16 * 256, 0),
    (64, 12, 2, 128, 16, 64 * 256, 0),
    (32, 12, 2, 128, 32, 4000, 0),
    (4, 12, 2, 128, 16, 1000, 0),
    (3, 8, 1, 64, 8, 10, 0),
    (5, 12, 2, 128, 16, 300, 3),
    (256, 64, 8, 128, 16, 256 * 1000, 0),
    (2, 32, 8, 128, 16, 16384, 0),
])
def test_plan_csr_matches_python_mirror(batch, hq, hkv, d, ps, nnz, splits):
    lib = _native.capi()
    p = _native.PadPlan()
    assert lib.pad_decode_plan_csr(ctypes.byref(_dims(batch, hq, hkv, d, ps, nnz)), splits, 256, ctypes.byref(p)) == 0
    m = heuristics.plan(batch, hq, hkv, d, ps, nnz, splits, 256, csr=True)
    assert (p.num_splits, p.pages_per_split, p.waves_per_group, bool(p.single_pass), p.workspace_bytes,
            p.counters) == (m.num_splits, m.pages_per_split, m.waves_per_group, m.single_pass, m.workspace_bytes,
                            m.counters)


def test_plan_csr_uses_pages_per_sequence():
    # 16 sequences of 256 pages as a CSR index of 4096 entries plan like the
    # dense table of 256 columns (the whole index is not one sequence).
    dense = heuristics.plan(16, 12, 2, 128, 16, 256)
    csr = heuristics.plan(16, 12, 2, 128, 16, 16 * 256, csr=True)
    assert (csr.num_splits, csr.pages_per_split, csr.waves_per_group) == (
        dense.num_splits, dense.pages_per_split, dense.waves_per_group)
    # Small batches plan like their dense twins too (latency-bound shapes:
    # short splits, up to 8 waves).
    for batch, width in ((2, 64), (4, 256), (1, 100)):
        d2 = heuristics.plan(batch, 12, 2, 128, 16, width)
        c2 = heuristics.plan(batch, 12, 2, 128, 16, batch * width, csr=True)
        assert (c2.num_splits, c2.pages_per_split, c2.waves_per_group) == (
            d2.num_splits, d2.pages_per_split, d2.waves_per_group), (batch, width)
    assert heuristics.plan(4, 12, 2, 128, 16, 4 * 256, csr=True).waves_per_group == 8


def test_plan_csr_scratch_never_exceeds_dense():
    # pad_decode_workspace_bytes() / pad_decode_counters_needed() on the
    # dense reading of the dims must size every CSR launch.
    for batch in (1, 2, 3, 4, 8, 16, 33, 64, 128, 256, 300):
        for hkv in (1, 2, 8):
            for nnz in (1, 7, 64, 256, 1000, 4096, 20000, 200000):
                for ps in (1, 16, 32):
                    for splits in (0, 4):
                        c = heuristics.plan(batch, 8 * hkv, hkv, 128, ps, nnz, splits, 256, csr=True)
                        dn = heuristics.plan(batch, 8 * hkv, hkv, 128, ps, nnz, splits, 256)
                        assert c.workspace_bytes <= dn.workspace_bytes and c.counters <= dn.counters, (
                            batch, hkv, nnz, ps, splits)


def test_launch_rejects_zero_num_pages_on_the_host():
    # num_pages bounds the page ids on the device; 0 would silently read
    # page 0 for every page, so the launch refuses it before any device call.
    lib = _native.capi()
    dm = _dims(batch=2, max_pages=4, num_pages=0)
    fake = ctypes.c_void_p(256)
    assert lib.pad_decode_launch(fake, fake, fake, fake, fake, fake, None, 0, None, 0, ctypes.byref(dm), 0.1, 1,
                                 None) == 2
    assert lib.pad_decode_launch_csr(fake, fake, fake, fake, fake, fake, fake, None, 0, None, 0, ctypes.byref(dm),
                                     0.1, 1, 0, None) == 2


def test_launch_kv8_checks_format_and_scales_on_the_host():
    # Format, head_dim and scale problems of the fp8 entry are answered
    # before any device call.
    lib = _native.capi()
    fake = ctypes.c_void_p(256)
    dm = _dims(batch=2, max_pages=4)
    args = (fake, fake, fake, fake, fake, fake, None, 0, None, 0, ctypes.byref(dm), 0.1)
    assert lib.pad_decode_launch_kv8(*args, 0, 1.0, 1.0, 1, None) == 12  # PAD_KV_FP16
    assert lib.pad_decode_launch_kv8(*args, 3, 1.0, 1.0, 1, None) == 12
    assert lib.pad_decode_launch_kv8(*args, -1, 1.0, 1.0, 1, None) == 12
    for ks, vs in ((0.0, 1.0), (1.0, -2.0), (float("nan"), 1.0), (1.0, float("inf")), (1e31, 1.0)):
        assert lib.pad_decode_launch_kv8(*args, 1, ks, vs, 1, None) == 12, (ks, vs)
    dm96 = _dims(batch=2, max_pages=4, d=96)
    assert lib.pad_decode_launch_kv8(fake, fake, fake, fake, fake, fake, None, 0, None, 0, ctypes.byref(dm96), 0.1,
                                     2, 1.0, 1.0, 1, None) == 3


@pytest.mark.parametrize("d", [32, 64, 96, 128, 256])
def test_planned_waves_fit_lds(d):
    # Every group size and split shape: the planned workgroup fits a CU's
    # 160 KB of LDS, and the widest rows still get 4+ waves.
    for gqa in range(1, 17):
        for batch, max_pages in ((1, 512), (8, 512), (64, 128), (256, 64)):
            for engine in (0, 1):
                m = heuristics.plan(batch, gqa, 1, d, 16, max_pages, 0, 256, engine)
                assert heuristics.group_lds_bytes(m.waves_per_group, gqa, d, engine) <= 160 * 1024
    # head_dim 256 stops at 4 waves (one per SIMD, no register spills).
    assert heuristics.plan(8, 16, 1, 256, 16, 512).waves_per_group == 4
    for gqa in range(1, 17):
        assert heuristics.plan(1, gqa, 1, 256, 16, 4096).waves_per_group <= 4


def test_heuristic_properties():
    # Batch 1 (latency-bound): 8-wave workgroups on at most half the CUs,
    # each split at least 16 blocks (2 per wave).  Bandwidth-bound batches:
    # one 4-wave workgroup per CU, no more.
    p1 = heuristics.plan(1, 12, 2, 128, 16, 256)
    assert p1.waves_per_group == 8 and p1.pages_per_split * 16 >= 16 * 16
    assert 32 <= p1.num_splits * 2 * p1.waves_per_group and p1.num_splits * 2 <= 128
    for b in (16, 32, 64):
        p = heuristics.plan(b, 12, 2, 128, 16, 256)
        assert p.waves_per_group == 4 and p.num_splits * b * 2 == 256
    p64 = heuristics.plan(64, 12, 2, 128, 16, 256)
    assert p64.num_splits <= 8
    # More than one unit per two CUs: a grid of 4 items per unit for the
    # in-kernel planner (one item per unit if every sequence is full), and at
    # least 8 workgroups per CU (8 items per unit at one unit per CU, 5 at
    # 410 units); past the planner's batch limit, one workgroup per unit.
    p_big = heuristics.plan(256, 64, 8, 128, 16, 2048)
    assert p_big.num_splits == heuristics.OVERSUBSCRIBE_SPLITS == 4 and not p_big.single_pass
    assert p_big.workspace_bytes == heuristics.workspace_bytes(256, 8, 8, 128, 4)
    p128 = heuristics.plan(128, 12, 2, 128, 16, 256)
    assert p128.num_splits == 8 and p128.waves_per_group == 4
    p_share = heuristics.plan(256, 8, 1, 128, 16, 2048)  # C5 over 8 GPUs by kv heads: 256 units
    assert p_share.num_splits == 8 and p_share.workspace_bytes == heuristics.workspace_bytes(256, 1, 8, 128, 8)
    assert heuristics.plan(205, 12, 2, 128, 16, 256).num_splits == 5  # 410 units: 2050 workgroups
    assert heuristics.plan(256, 8, 2, 128, 16, 2048).num_splits == 4  # 512 units
    # From more than one unit per two CUs (where one split per unit would leave a ragged batch's
    # long units to one workgroup each); at most one unit per two CUs keeps the power-of-two rule.
    assert heuristics.plan(96, 12, 2, 128, 16, 256).num_splits == 11  # 192 units: 2112 workgroups
    assert heuristics.plan(65, 12, 2, 128, 16, 256).num_splits == 16  # 130 units
    assert heuristics.plan(64, 12, 2, 128, 16, 256).num_splits == 2  # 128 units: C2 batch 64
    # The largest split count that fits the workgroup budget replaces the power of two where it is
    # 1.5 times as large or more: batch 20 (40 units) 6 splits, 17 -> 7, 5 (latency-bound, half the
    # CUs) -> 12; batch 12 (24 units: 10 against 8) and 7 (9 against 8) keep the power of two.
    for b, s in ((20, 6), (17, 7), (5, 12), (12, 8), (7, 8), (24, 4), (32, 4)):
        assert heuristics.plan(b, 12, 2, 128, 16, 256).num_splits == s, b
    p_over = heuristics.plan(512, 12, 2, 128, 16, 256)
    assert p_over.num_splits == 1 and p_over.single_pass


@pytest.mark.parametrize("field,value,code", [
    ("head_dim", 48, 3),
    ("head_dim", 512, 3),
    ("num_q_heads", 13, 4),
    ("num_q_heads", 34, 4),
    ("num_kv_heads", 0, 2),
    ("page_size", 0, 2),
    ("batch", -1, 2),
])
def test_plan_rejects_bad_shapes(field, value, code):
    lib = _native.capi()
    dm = _dims()
    setattr(dm, field, value)
    p = _native.PadPlan()
    assert lib.pad_decode_plan(ctypes.byref(dm), 0, 256, ctypes.byref(p)) == code


def test_plan_rejects_bad_strides_and_splits():
    lib = _native.capi()
    p = _native.PadPlan()
    dm = _dims()
    dm.k_stride[3] = 2
    assert lib.pad_decode_plan(ctypes.byref(dm), 0, 256, ctypes.byref(p)) == 5
    assert lib.pad_decode_plan(ctypes.byref(_dims()), -1, 256, ctypes.byref(p)) == 8
    assert lib.pad_decode_plan(ctypes.byref(_dims()), 1025, 256, ctypes.byref(p)) == 8
    assert lib.pad_decode_plan(None, 0, 256, ctypes.byref(p)) == 1


# --------------------------------------------------------------------- GPU ---

def _launch(lib, q, k, v, bt, sl, out, ws, dm, scale, splits, engine=None, stream=None, events=None, counters=None):
    wsp = ws.data_ptr() if ws is not None else None
    wsb = ws.numel() if ws is not None else 0
    cp = counters.data_ptr() if counters is not None else None
    cn = counters.numel() if counters is not None else 0
    if engine is None:
        return lib.pad_decode_launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                                     out.data_ptr(), wsp, wsb, cp, cn, ctypes.byref(dm), scale, splits, stream)
    return lib.pad_decode_launch_ex(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                                    out.data_ptr(), wsp, wsb, cp, cn, ctypes.byref(dm), scale, splits, engine, events,
                                    stream)


@pytest.mark.gpu
@pytest.mark.parametrize("splits", [0, 1, 6, 64])
def test_launch_through_c_abi(splits):
    from oracle.reference import decode_fp16_protocol

    lib = _native.capi()
    lens = [1, 77, 400, 1000]
    bt, n = shuffled_table(lens, 16, spare_pages=3, extra_cols=1, seed=3)
    k, v = make_cache(n, 16, 2, 128, seed=3)
    q = torch.randn(4, 12, 128, generator=torch.Generator().manual_seed(3))
    sl = torch.tensor(lens, dtype=torch.int32)
    expected = decode_fp16_protocol(q, k, v, bt, sl)
    qd, kd, vd = q.half().cuda(), k.half().cuda(), v.half().cuda()
    btd, sld = bt.cuda(), sl.cuda()
    out = torch.empty_like(qd)
    dm = _native.dims_for(qd, kd, vd, btd, sld, out)
    wsb = ctypes.c_size_t()
    nc = ctypes.c_int64()
    assert lib.pad_decode_workspace_bytes(ctypes.byref(dm), splits, 0, ctypes.byref(wsb)) == 0
    assert lib.pad_decode_counters_needed(ctypes.byref(dm), splits, 0, ctypes.byref(nc)) == 0
    # 8 (sequence, kv head) counters, plus one per split slot where a unit
    # may get more than 48 items (two-level merge).
    cus = ctypes.c_int()
    assert lib.pad_device_num_cus(ctypes.byref(cus)) == 0
    m = heuristics.plan(4, 12, 2, 128, 16, bt.shape[1], splits, cus.value)
    assert nc.value == m.counters and nc.value in (0, 8, 8 + 8 * m.num_splits)
    # The workspace keeps no state: fill it with garbage before every launch.
    ws = torch.empty(max(wsb.value, 1), dtype=torch.uint8, device="cuda")
    counters = torch.full((max(nc.value, 1),), 12345, dtype=torch.int32, device="cuda")
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    assert lib.pad_decode_counters_init(counters.data_ptr(), counters.numel(), stream.cuda_stream) == 0
    for _ in range(3):  # the counters come back to zero after every launch
        out.fill_(float("nan"))
        ws.fill_(0x7F)
        torch.cuda.synchronize()
        st = _launch(lib, qd, kd, vd, btd, sld, out, ws, dm, 1.0 / 128 ** 0.5, splits, stream=stream.cuda_stream,
                     counters=counters)
        assert st == 0, lib.pad_status_string(st)
        stream.synchronize()
        assert_parity(out, expected)
        assert torch.all(counters == 0), counters


@pytest.mark.gpu
def test_launch_ex_events_and_engines():
    from oracle.reference import decode_fp16_protocol

    lib = _native.capi()
    lens = [300, 2000]
    bt, n = shuffled_table(lens, 16, spare_pages=2, extra_cols=0, seed=4)
    k, v = make_cache(n, 16, 2, 128, seed=4)
    q = torch.randn(2, 12, 128, generator=torch.Generator().manual_seed(4))
    sl = torch.tensor(lens, dtype=torch.int32)
    expected = decode_fp16_protocol(q, k, v, bt, sl)
    qd, kd, vd, btd, sld = q.half().cuda(), k.half().cuda(), v.half().cuda(), bt.cuda(), sl.cuda()
    for engine in (0, 1):
        out = torch.empty_like(qd)
        dm = _native.dims_for(qd, kd, vd, btd, sld, out)
        ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
        counters = torch.zeros(64, dtype=torch.int32, device="cuda")
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        arr = (ctypes.c_void_p * 3)(*[e.cuda_event for e in evs])
        for e in evs:  # events must exist on the device before the library records them
            e.record()
        torch.cuda.synchronize()
        st = _launch(lib, qd, kd, vd, btd, sld, out, ws, dm, 1.0 / 128 ** 0.5, 4, engine=engine,
                     stream=torch.cuda.current_stream().cuda_stream, events=arr, counters=counters)
        assert st == 0, lib.pad_status_string(st)
        torch.cuda.synchronize()
        assert evs[0].elapsed_time(evs[1]) > 0.0
        assert evs[0].elapsed_time(evs[2]) >= 0.0
        assert_parity(out, expected)


@pytest.mark.gpu
def test_launch_rejects_bad_arguments_without_launching():
    lib = _native.capi()
    q = torch.zeros(1, 12, 128, dtype=torch.float16, device="cuda")
    k = torch.zeros(4, 16, 2, 128, dtype=torch.float16, device="cuda")
    bt = torch.zeros(1, 4, dtype=torch.int32, device="cuda")
    sl = torch.full((1,), 40, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    dm = _native.dims_for(q, k, k, bt, sl, out)
    # Workspace or counters missing for a split launch.
    assert _launch(lib, q, k, k, bt, sl, out, None, dm, 0.1, 4) == 7
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    assert _launch(lib, q, k, k, bt, sl, out, ws, dm, 0.1, 4) == 7
    assert _launch(lib, q, k, k, bt, sl, out, ws, dm, 0.1, 4, counters=torch.zeros(1, dtype=torch.int32,
                                                                                      device="cuda")) == 7
    # Misaligned output row.
    flat = torch.empty(12 * 128 + 8, dtype=torch.float16, device="cuda")
    bad_out = flat[1:1 + 12 * 128].view(1, 12, 128)
    assert lib.pad_decode_launch(q.data_ptr(), k.data_ptr(), k.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                                 bad_out.data_ptr(), None, 0, None, 0, ctypes.byref(dm), 0.1, 1, None) == 6
    # Null pointer.
    assert lib.pad_decode_launch(None, k.data_ptr(), k.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                                 out.data_ptr(), None, 0, None, 0, ctypes.byref(dm), 0.1, 1, None) == 1
    # VALU engine does not cover a group of 16.
    q16 = torch.zeros(1, 32, 128, dtype=torch.float16, device="cuda")
    dm16 = _native.dims_for(q16, k, k, bt, sl, torch.empty_like(q16))
    assert lib.pad_decode_launch_ex(q16.data_ptr(), k.data_ptr(), k.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                                    q16.data_ptr(), None, 0, None, 0, ctypes.byref(dm16), 0.1, 1, 1, None, None) == 4
    torch.cuda.synchronize()


@pytest.mark.gpu
@pytest.mark.parametrize("splits", [0, 3])
def test_launch_csr_through_c_abi(splits):
    """pad_decode_launch_csr with a caller-owned workspace, counters and stream."""
    from oracle.csr import paged_kv_indices
    from oracle.reference import decode_fp16_protocol

    lib = _native.capi()
    lens = [0, 5, 77, 400, 1000]
    bt, n = shuffled_table(lens, 16, spare_pages=3, extra_cols=1, seed=5)
    k, v = make_cache(n, 16, 2, 128, seed=5)
    q = torch.randn(len(lens), 12, 128, generator=torch.Generator().manual_seed(5))
    sl = torch.tensor(lens, dtype=torch.int32)
    expected = decode_fp16_protocol(q, k, v, bt, sl)
    indptr, indices, last = (x.cuda() for x in paged_kv_indices(bt, sl, 16))
    qd, kd, vd = q.half().cuda(), k.half().cuda(), v.half().cuda()
    out = torch.empty_like(qd)
    dm = _native.dims_for(qd, kd, vd, indices.view(1, -1), last, out)
    dm.bt_stride[0], dm.bt_stride[1] = 0, 1
    wsb = ctypes.c_size_t()
    nc = ctypes.c_int64()
    assert lib.pad_decode_workspace_bytes(ctypes.byref(dm), splits, 0, ctypes.byref(wsb)) == 0
    assert lib.pad_decode_counters_needed(ctypes.byref(dm), splits, 0, ctypes.byref(nc)) == 0
    ws = torch.empty(max(wsb.value, 1), dtype=torch.uint8, device="cuda")
    counters = torch.zeros(max(nc.value, 1), dtype=torch.int32, device="cuda")
    stream = torch.cuda.Stream()
    for _ in range(2):
        out.fill_(float("nan"))
        ws.fill_(0x7F)
        torch.cuda.synchronize()
        st = lib.pad_decode_launch_csr(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), indices.data_ptr(),
                                       indptr.data_ptr(), last.data_ptr(), out.data_ptr(), ws.data_ptr(), wsb.value,
                                       counters.data_ptr(), counters.numel(), ctypes.byref(dm), 1.0 / 128 ** 0.5,
                                       splits, 0, stream.cuda_stream)
        assert st == 0, lib.pad_status_string(st)
        stream.synchronize()
        assert_parity(out, expected)
        assert torch.all(counters == 0), counters
    # Missing CSR arrays are rejected before any launch.
    assert lib.pad_decode_launch_csr(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), indices.data_ptr(), None,
                                     last.data_ptr(), out.data_ptr(), ws.data_ptr(), wsb.value, counters.data_ptr(),
                                     counters.numel(), ctypes.byref(dm), 0.1, splits, 0, None) == 1


def test_fp8_plan_keeps_the_scratch_of_the_fp16_plan():
    # pad_decode_launch_kv8 plans with one byte per K/V element: the same
    # splits, workspace and counters as pad_decode_plan (which sizes its
    # scratch), except where the fp16 plan is an oversubscribed grid: fp8
    # takes the 4-item grid from one unit per CU up only, so never more
    # scratch; 8-wave workgroups only where the fp16 plan has 4 waves for
    # 256-byte rows.
    import random

    rng = random.Random(5)
    for _ in range(300):
        batch, hkv = rng.choice([1, 2, 8, 16, 32, 64, 128, 300]), rng.choice([1, 2, 4, 8])
        gqa, d = rng.choice([1, 2, 4, 6, 8, 16]), rng.choice([64, 128, 256])
        ps = rng.choice([1, 4, 12, 16, 32, 64])
        max_pages = rng.randint(1, 4096) // ps + 1
        a = heuristics.plan(batch, hkv * gqa, hkv, d, ps, max_pages)
        b = heuristics.plan(batch, hkv * gqa, hkv, d, ps, max_pages, kv_bytes=1)
        units = batch * hkv
        lat = units * -(-max_pages * ps // 16) <= 16 * 256
        fewer = heuristics.oversubscribed(batch, hkv, max_pages, lat, 256)  # the fp16 grid
        if fewer:
            assert b.num_splits <= a.num_splits and b.workspace_bytes <= a.workspace_bytes
            assert b.counters <= a.counters
        else:
            assert (a.num_splits, a.pages_per_split, a.single_pass, a.workspace_bytes, a.counters) == (
                b.num_splits, b.pages_per_split, b.single_pass, b.workspace_bytes, b.counters)
        assert b.waves_per_group >= a.waves_per_group
        if d != 128:
            assert b.waves_per_group == a.waves_per_group


def test_call_descriptor_layout_matches_the_header(tmp_path):
    # The ctypes mirror of pad_decode_call (and pad_decode_dims, pad_decode_plan_t)
    # has the C compiler's field offsets and size for the header as written.
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not found")
    structs = {"pad_decode_call": _native.PadCall, "pad_decode_dims": _native.PadDims,
               "pad_decode_plan_t": _native.PadPlan}
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "pa_decode.h"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'  printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'  printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run([gcc, "-std=c99", f"-I{os.path.dirname(HEADER)}", str(src), "-o", str(exe)], check=True)
    got = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    for line in filter(None, got):
        cname, field, value = line.split()
        py = structs[cname]
        want = ctypes.sizeof(py) if field == "sizeof" else getattr(py, field).offset
        assert int(value) == want, (cname, field, int(value), want)


def test_launch_call_checks_on_the_host():
    # The descriptor entry answers argument problems before any device call.
    lib = _native.capi()
    fake = 256
    dm = _dims(batch=2, max_pages=4)
    c = _native.PadCall(q=fake, k_cache=fake, v_cache=fake, block_table=fake, seq_lens=fake, out=fake, scale=0.1,
                        num_splits=1, engine=0, kv_format=0, k_scale=1.0, v_scale=1.0)
    assert lib.pad_decode_launch_call(None, ctypes.byref(dm), None) == 1
    half_csr = _native.PadCall.from_buffer_copy(c)
    half_csr.indptr = fake  # CSR needs indptr and last_page_len together
    assert lib.pad_decode_launch_call(ctypes.byref(half_csr), ctypes.byref(dm), None) == 1
    wl_valu = _native.PadCall.from_buffer_copy(c)
    wl_valu.worklist, wl_valu.worklist_bytes, wl_valu.engine = fake, 1 << 20, 1
    assert lib.pad_decode_launch_call(ctypes.byref(wl_valu), ctypes.byref(dm), None) == 2
    for fmt, ks, engine, code in ((6, 1.0, 0, 12), (-1, 1.0, 0, 12), (1, 0.0, 0, 12), (1, 1.0, 1, 12),
                                  (4, 0.0, 0, 12), (2, float("inf"), 0, 12), (3, 1.0, 1, 12)):
        bad = _native.PadCall.from_buffer_copy(c)
        bad.kv_format, bad.k_scale, bad.engine = fmt, ks, engine
        assert lib.pad_decode_launch_call(ctypes.byref(bad), ctypes.byref(dm), None) == code, (fmt, ks, engine)
    dm96 = _dims(batch=2, max_pages=4, d=96)
    fp8 = _native.PadCall.from_buffer_copy(c)
    fp8.kv_format = 1
    assert lib.pad_decode_launch_call(ctypes.byref(fp8), ctypes.byref(dm96), None) == 3
    # Planning a work list: NULL descriptor, VALU engine, bad format.
    wl = ctypes.create_string_buffer(1 << 16)
    assert lib.pad_decode_plan_worklist_call(None, ctypes.byref(dm), wl, len(wl), None) == 1
    valu = _native.PadCall.from_buffer_copy(c)
    valu.engine = 1
    assert lib.pad_decode_plan_worklist_call(ctypes.byref(valu), ctypes.byref(dm), wl, len(wl), None) == 2
    badf = _native.PadCall.from_buffer_copy(c)
    badf.kv_format = 7
    assert lib.pad_decode_plan_worklist_call(ctypes.byref(badf), ctypes.byref(dm), wl, len(wl), None) == 12

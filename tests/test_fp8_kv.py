"""GPU tests of the decode over fp8 K/V caches (pad_decode_launch_kv8).

The caches hold float8_e4m3fn or float8_e5m2 codes of K / k_scale and
V / v_scale; q and the output are fp16.  No counterpart in the reference,
whose caches are fp16 only (src/kernel_cuda_v4.py:37-48).

* Parity: against the fp32 oracle on the dequantised caches
  (oracle/reference.py decode_fp8_protocol), atol = rtol = 2e-3 and the
  reference's own 1e-2 / 1e-3, over both formats, head_dim 64/128/256, page
  sizes of the uniform, sub-page and generic block modes, split counts and
  scales other than 1.
* Bit-exact: with unit scales the fp8 kernel must return exactly what the
  fp16 kernel returns on the same codes widened to fp16 by PyTorch (same
  plan, same split count), on random data and on caches that hold every
  finite code of the format: every fp8 value is an fp16 value, and the
  kernel's in-register conversion must produce it.
* NaN codes in unused pages and in the unused slots of a last page leave the
  output untouched; error statuses for a bad format, head_dim and scale.
"""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

from oracle.reference import decode_fp8_protocol
from paged_attention_decode_amd import _native, heuristics
from tests.helpers import assert_parity, make_cache, shuffled_table

pytestmark = pytest.mark.gpu

FMTS = {"e4m3fn": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
# Largest finite magnitude of each format.
FMAX = {"e4m3fn": 448.0, "e5m2": 57344.0}


def _quant(x, fmt, scale):
    """x / scale as fp8 codes (x / scale stays inside the format's range)."""
    y = x / scale
    assert float(y.abs().max()) < FMAX[fmt]
    return y.to(FMTS[fmt])


def _case(lens, ps, hkv, gqa, d, seed, spare=2, extra=1):
    bt, n = shuffled_table(lens, ps, spare_pages=spare, extra_cols=extra, seed=seed)
    k, v = make_cache(n, ps, hkv, d, seed=seed)
    q = torch.randn(len(lens), hkv * gqa, d, generator=torch.Generator().manual_seed(seed))
    return q, k, v, bt, torch.tensor(lens, dtype=torch.int32)


def _fp8(q, k8, v8, bt, sl, ks, vs, splits):
    import paged_attention_decode_amd as pad

    out = pad.paged_attention_decode_fp8(q.half().cuda(), k8.cuda(), v8.cuda(), bt.cuda(), sl.cuda(),
                                         k_scale=ks, v_scale=vs, num_splits=splits)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and out.shape == q.shape
    return out.cpu()


@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("ps", [16, 1, 4, 12, 64])
def test_fp8_matches_oracle(fmt, d, ps):
    lens = [1, ps + 3, 150, 777]
    q, k, v, bt, sl = _case(lens, ps, 2, 6, d, seed=ps + d)
    # Scales that are not powers of two, with the codes spanning the range.
    ks, vs = float(k.abs().max()) / 300.0, float(v.abs().max()) / 111.0
    k8, v8 = _quant(k, fmt, ks), _quant(v, fmt, vs)
    expected = decode_fp8_protocol(q, k8, v8, bt, sl, ks, vs)
    for splits in (None, 1, 5):
        assert_parity(_fp8(q, k8, v8, bt, sl, ks, vs, splits), expected)


@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("hkv,gqa", [(1, 1), (4, 2), (2, 8), (1, 16)])
def test_fp8_group_sizes(fmt, hkv, gqa):
    lens = [33, 2000, 5]
    q, k, v, bt, sl = _case(lens, 16, hkv, gqa, 128, seed=hkv * 31 + gqa)
    ks, vs = 0.02, 0.5
    k8, v8 = _quant(k, fmt, ks), _quant(v, fmt, vs)
    expected = decode_fp8_protocol(q, k8, v8, bt, sl, ks, vs)
    for splits in (None, 64):
        assert_parity(_fp8(q, k8, v8, bt, sl, ks, vs, splits), expected)


@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("d", [64, 128, 256])
def test_unit_scales_equal_the_fp16_kernel_bitwise(fmt, d):
    import paged_attention_decode_amd as pad

    lens = [7, 300, 1500, 64]
    q, k, v, bt, sl = _case(lens, 16, 2, 4, d, seed=d + 1)
    k8, v8 = k.to(FMTS[fmt]), v.to(FMTS[fmt])
    qd, btd, sld = q.half().cuda(), bt.cuda(), sl.cuda()
    for splits in (None, 1, 8):
        a = pad.paged_attention_decode_fp8(qd, k8.cuda(), v8.cuda(), btd, sld, num_splits=splits)
        b = pad.paged_attention_decode(qd, k8.half().cuda(), v8.half().cuda(), btd, sld, num_splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(a, b), (splits, (a.float() - b.float()).abs().max().item())


@pytest.mark.parametrize("fmt", list(FMTS))
def test_every_finite_code_converts_exactly(fmt):
    # K and V cycle through every finite code (subnormals, extremes, both
    # zeros) in every head_dim position; unit scales, so the fp8 kernel must
    # match the fp16 kernel on PyTorch's widening of the same codes.
    import paged_attention_decode_amd as pad

    dt = FMTS[fmt]
    codes = torch.arange(256, dtype=torch.uint8)
    finite = codes[torch.isfinite(codes.view(dt).float())]
    ps, hkv, d, n_pages = 16, 1, 128, 8
    n = n_pages * ps * hkv * d
    idx = torch.arange(n)
    kc = finite[(idx * 7) % finite.numel()].view(n_pages, ps, hkv, d)
    vc = finite[(idx * 11 + 3) % finite.numel()].view(n_pages, ps, hkv, d)
    k8, v8 = kc.view(dt), vc.view(dt)
    # Small q keeps the scores of the largest e5m2 codes finite in fp16 terms.
    q = torch.randn(2, 4, d, generator=torch.Generator().manual_seed(0)) * (1e-4 if fmt == "e5m2" else 1e-2)
    bt = torch.arange(n_pages, dtype=torch.int32).view(2, n_pages // 2)
    sl = torch.tensor([n_pages // 2 * ps, n_pages // 2 * ps - 5], dtype=torch.int32)
    qd, btd, sld = q.half().cuda(), bt.cuda(), sl.cuda()
    for splits in (None, 1, 4):
        a = pad.paged_attention_decode_fp8(qd, k8.cuda(), v8.cuda(), btd, sld, num_splits=splits)
        b = pad.paged_attention_decode(qd, k8.half().cuda(), v8.half().cuda(), btd, sld, num_splits=splits)
        torch.cuda.synchronize()
        assert torch.isfinite(b).all()
        assert torch.equal(a, b), (splits, (a.float() - b.float()).abs().max().item())


@pytest.mark.parametrize("fmt", list(FMTS))
def test_nan_codes_in_unused_slots(fmt):
    # Unused pages and the unused tail of each last page hold NaN codes (and
    # infinities for e5m2): a kernel that reads them into the result gives NaN.
    lens = [37, 5]
    q, k, v, bt, sl = _case(lens, 16, 2, 6, 128, seed=9, spare=3, extra=2)
    ks, vs = 0.05, 0.05
    k8, v8 = _quant(k, fmt, ks), _quant(v, fmt, vs)
    expected = decode_fp8_protocol(q, k8, v8, bt, sl, ks, vs)
    ku, vu = k8.view(torch.uint8).clone(), v8.view(torch.uint8).clone()
    bad = [0x7F, 0xFF] if fmt == "e4m3fn" else [0x7F, 0xFE, 0x7C, 0xFC]
    used = {int(bt[0, j]) for j in range(3)} | {int(bt[1, 0])}
    for p in range(ku.shape[0]):
        if p not in used:
            ku[p] = bad[p % len(bad)]
            vu[p] = bad[(p + 1) % len(bad)]
    for last in (int(bt[0, 2]), int(bt[1, 0])):
        ku[last, 5:] = bad[0]
        vu[last, 5:] = bad[-1]
    k8p, v8p = ku.view(FMTS[fmt]), vu.view(FMTS[fmt])
    for s in (None, 1, 2):
        out = _fp8(q, k8p, v8p, bt, sl, ks, vs, s)
        assert torch.isfinite(out).all()
        assert_parity(out, expected)


def test_nan_code_in_a_used_slot_propagates():
    # A NaN code inside the sequence is a NaN key: its query rows become NaN,
    # as the fp16 kernel and the oracle give for a NaN in an fp16 cache.
    lens = [40]
    q, k, v, bt, sl = _case(lens, 16, 1, 2, 64, seed=5, spare=0, extra=0)
    k8 = _quant(k, "e4m3fn", 0.02)
    ku = k8.view(torch.uint8).clone()
    ku[int(bt[0, 1]), 3, 0, 10] = 0x7F
    out = _fp8(q, ku.view(torch.float8_e4m3fn), _quant(v, "e4m3fn", 0.02), bt, sl, 0.02, 0.02, None)
    assert torch.isnan(out).all()


def test_kv8_through_the_c_abi():
    lib = _native.capi()
    lens = [1, 77, 400, 1000]
    q, k, v, bt, sl = _case(lens, 16, 2, 6, 128, seed=3)
    ks, vs = float(k.abs().max()) / 400.0, float(v.abs().max()) / 50.0
    k8, v8 = _quant(k, "e4m3fn", ks), _quant(v, "e4m3fn", vs)
    expected = decode_fp8_protocol(q, k8, v8, bt, sl, ks, vs)
    qd, kd, vd, btd, sld = q.half().cuda(), k8.cuda(), v8.cuda(), bt.cuda(), sl.cuda()
    out = torch.empty_like(qd)
    dm = _native.dims_for(qd, kd, vd, btd, sld, out)
    for splits in (0, 1, 6):
        wsb, nc = ctypes.c_size_t(), ctypes.c_int64()
        assert lib.pad_decode_workspace_bytes(ctypes.byref(dm), splits, 0, ctypes.byref(wsb)) == 0
        assert lib.pad_decode_counters_needed(ctypes.byref(dm), splits, 0, ctypes.byref(nc)) == 0
        ws = torch.empty(max(wsb.value, 1), dtype=torch.uint8, device="cuda")
        counters = torch.zeros(max(nc.value, 1), dtype=torch.int32, device="cuda")
        stream = torch.cuda.current_stream().cuda_stream
        out.fill_(float("nan"))
        st = lib.pad_decode_launch_kv8(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), btd.data_ptr(), sld.data_ptr(),
                                       out.data_ptr(), ws.data_ptr(), ws.numel(), counters.data_ptr(),
                                       counters.numel(), ctypes.byref(dm), 1.0 / math.sqrt(128), 1, ks, vs, splits,
                                       stream)
        assert st == 0, lib.pad_status_string(st)
        torch.cuda.synchronize()
        assert_parity(out, expected)
        assert torch.all(counters == 0)


def test_fp8_rejects_bad_arguments():
    import paged_attention_decode_amd as pad

    q, k, v, bt, sl = _case([20], 16, 2, 2, 96, seed=1)
    k8 = k.to(torch.float8_e4m3fn).cuda()
    with pytest.raises(AssertionError, match="head_dim"):
        pad.paged_attention_decode_fp8(q.half().cuda(), k8, k8, bt.cuda(), sl.cuda())
    q, k, v, bt, sl = _case([20], 16, 2, 2, 64, seed=1)
    qd, btd, sld = q.half().cuda(), bt.cuda(), sl.cuda()
    k8, v5 = k.to(torch.float8_e4m3fn).cuda(), v.to(torch.float8_e5m2).cuda()
    with pytest.raises(AssertionError, match="float8"):
        pad.paged_attention_decode_fp8(qd, k8, v5, btd, sld)
    for bad in (0.0, -1.0, float("inf"), float("nan")):
        with pytest.raises(AssertionError, match="k_scale"):
            pad.paged_attention_decode_fp8(qd, k8, k8, btd, sld, k_scale=bad)
    # The binding and the C ABI refuse them as well.
    from paged_attention_decode_amd._native import ext

    with pytest.raises(RuntimeError, match="fp8"):
        ext().forward_kv8(qd, k8, k8, btd, sld, 0.125, -1.0, 1.0, 0)
    with pytest.raises(RuntimeError, match="float8"):
        ext().forward_kv8(qd, k8.half(), k8.half(), btd, sld, 0.125, 1.0, 1.0, 0)
    lib = _native.capi()
    out = torch.empty_like(qd)
    dm = _native.dims_for(qd, k8, k8, btd, sld, out)
    args = (qd.data_ptr(), k8.data_ptr(), k8.data_ptr(), btd.data_ptr(), sld.data_ptr(), out.data_ptr(), None, 0,
            None, 0, ctypes.byref(dm), 0.125)
    assert lib.pad_decode_launch_kv8(*args, 0, 1.0, 1.0, 1, None) == 12  # fp16 is pad_decode_launch's
    assert lib.pad_decode_launch_kv8(*args, 3, 1.0, 1.0, 1, None) == 12
    assert lib.pad_decode_launch_kv8(*args, 1, 0.0, 1.0, 1, None) == 12
    assert lib.pad_decode_launch_kv8(*args, 2, 1.0, float("nan"), 1, None) == 12
    torch.cuda.synchronize()


def test_fp8_graph_capture_replays():
    # The fp8 entry under HIP graph capture: scratch exists before capture,
    # every replay with new q written in place equals an eager call.
    import paged_attention_decode_amd as pad

    lens = [4096, 300, 2500, 1]
    q, k, v, bt, sl = _case(lens, 16, 2, 6, 128, seed=93)
    ks, vs = float(k.abs().max()) / 300.0, float(v.abs().max()) / 111.0
    k8, v8 = _quant(k, "e4m3fn", ks), _quant(v, "e4m3fn", vs)
    dev = [k8.cuda(), v8.cuda(), bt.cuda(), sl.cuda()]
    qs = [torch.randn(len(lens), 12, 128, generator=torch.Generator().manual_seed(94 + i)).half().cuda()
          for i in range(3)]
    q_static = qs[0].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            pad.paged_attention_decode_fp8(q_static, *dev, k_scale=ks, v_scale=vs)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out_static = pad.paged_attention_decode_fp8(q_static, *dev, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    for rep in range(2):
        for qn in qs:
            q_static.copy_(qn)
            graph.replay()
            torch.cuda.synchronize()
            eager = pad.paged_attention_decode_fp8(qn, *dev, k_scale=ks, v_scale=vs)
            torch.cuda.synchronize()
            assert torch.equal(out_static, eager), f"replay {rep} differs from the eager call"
    assert_parity(out_static.cpu(), decode_fp8_protocol(qs[-1].float().cpu(), k8, v8, bt, sl, ks, vs))


def _csr_of(bt, sl, ps):
    from oracle.csr import paged_kv_indices as ref_indices

    return [t.cuda() for t in ref_indices(bt, sl, ps)]


@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("ps", [16, 4, 12])
def test_fp8_csr_matches_oracle_and_fp16_csr(fmt, ps):
    # The CSR entry over fp8 caches: oracle parity with scales, and at unit
    # scales the fp16 CSR call on the widened codes, bit for bit.
    import paged_attention_decode_amd as pad

    lens = [1, ps + 3, 150, 777, 0, 2000]
    q, k, v, bt, sl = _case(lens, ps, 2, 6, 128, seed=ps + 7)
    indptr, indices, last = _csr_of(bt, sl, ps)
    ks, vs = float(k.abs().max()) / 300.0, float(v.abs().max()) / 111.0
    k8, v8 = _quant(k, fmt, ks), _quant(v, fmt, vs)
    expected = decode_fp8_protocol(q, k8, v8, bt, sl, ks, vs)
    qd = q.half().cuda()
    for splits in (None, 1, 5):
        out = pad.paged_attention_decode_csr(qd, k8.cuda(), v8.cuda(), indptr, indices, last, num_splits=splits,
                                             k_scale=ks, v_scale=vs)
        torch.cuda.synchronize()
        assert_parity(out.cpu(), expected)
    k1, v1 = k.to(FMTS[fmt]), v.to(FMTS[fmt])
    for splits in (None, 3):
        a = pad.paged_attention_decode_csr(qd, k1.cuda(), v1.cuda(), indptr, indices, last, num_splits=splits)
        b = pad.paged_attention_decode_csr(qd, k1.half().cuda(), v1.half().cuda(), indptr, indices, last,
                                           num_splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(a, b), splits


@pytest.mark.parametrize("fmt", list(FMTS))
def test_fp8_wrapper_plan_once_run_many(fmt):
    # BatchDecodeWrapper over fp8 caches: plan with kv_data_type, run with
    # k_scale / v_scale; the same output as the one-shot fp8 calls (dense and
    # CSR), for two steps of new q, and oracle parity.
    import paged_attention_decode_amd as pad

    lens = [4096, 300, 2500, 1, 777, 0, 1500, 64]
    q, k, v, bt, sl = _case(lens, 16, 2, 6, 128, seed=41)
    ks, vs = float(k.abs().max()) / 300.0, float(v.abs().max()) / 111.0
    k8, v8 = _quant(k, fmt, ks), _quant(v, fmt, vs)
    kd, vd, btd, sld = k8.cuda(), v8.cuda(), bt.cuda(), sl.cuda()
    indptr, indices, last = _csr_of(bt, sl, 16)
    dense = pad.BatchDecodeWrapper()
    dense.plan_block_table(btd, sld, 12, 2, 128, 16, kv_data_type=FMTS[fmt])
    csr = pad.BatchDecodeWrapper()
    csr.plan(indptr, indices, last, 12, 2, 128, 16, kv_data_type=fmt)
    for step in range(2):
        qd = (q if step == 0 else torch.randn(q.shape, generator=torch.Generator().manual_seed(42))).half().cuda()
        a = dense.run(qd, (kd, vd), k_scale=ks, v_scale=vs)
        b = pad.paged_attention_decode_fp8(qd, kd, vd, btd, sld, k_scale=ks, v_scale=vs)
        c = csr.run(qd, (kd, vd), k_scale=ks, v_scale=vs)
        d = pad.paged_attention_decode_csr(qd, kd, vd, indptr, indices, last, k_scale=ks, v_scale=vs)
        torch.cuda.synchronize()
        assert torch.equal(a, b) and torch.equal(c, d), step
        assert_parity(a.cpu(), decode_fp8_protocol(qd.float().cpu(), k8, v8, bt, sl, ks, vs))
    # A wrapper planned for fp16 caches refuses fp8 ones.
    w16 = pad.BatchDecodeWrapper()
    w16.plan_block_table(btd, sld, 12, 2, 128, 16)
    with pytest.raises(AssertionError, match="kv_data_type"):
        w16.run(q.half().cuda(), (kd, vd), k_scale=ks, v_scale=vs)


def test_fp8_launch_with_an_fp16_work_list_plans_in_the_kernel():
    # A work list made for fp16 caches carries another plan key (the fp8
    # launch runs 8-wave workgroups here), so the fp8 launch ignores it and
    # plans in the kernel: the result is the one-shot fp8 call's.
    import paged_attention_decode_amd as pad
    from paged_attention_decode_amd._native import ext

    lens = [4096] * 16  # bandwidth-bound: fp16 plans 4-wave, fp8 8-wave workgroups
    q, k, v, bt, sl = _case(lens, 16, 2, 6, 128, seed=43, spare=0, extra=0)
    assert heuristics.plan(16, 12, 2, 128, 16, 256).waves_per_group == 4
    assert heuristics.plan(16, 12, 2, 128, 16, 256, kv_bytes=1).waves_per_group == 8
    k8, v8 = k.to(torch.float8_e4m3fn).cuda(), v.to(torch.float8_e4m3fn).cuda()
    qd, btd, sld = q.half().cuda(), bt.cuda(), sl.cuda()
    wl16 = ext().plan_worklist(btd, sld, 12, 2, 128, 16, 0, 0)
    wl8 = ext().plan_worklist(btd, sld, 12, 2, 128, 16, 0, 1)
    assert not torch.equal(wl16[:32], wl8[:32])  # different plan keys in the headers
    scale = 1.0 / math.sqrt(128)
    a = ext().forward_worklist(qd, k8, v8, btd, sld, wl16, scale, 0, 1.0, 1.0)
    b = ext().forward_worklist(qd, k8, v8, btd, sld, wl8, scale, 0, 1.0, 1.0)
    c = pad.paged_attention_decode_fp8(qd, k8, v8, btd, sld)
    torch.cuda.synchronize()
    assert torch.equal(a, c) and torch.equal(b, c)


def test_launch_call_descriptor_through_the_c_abi():
    # pad_decode_launch_call() runs what the dedicated entry points run: the
    # fp16 dense call equals pad_decode_launch bit for bit, and an fp8 CSR
    # call with a planned work list equals the binding's one-shot CSR call.
    import paged_attention_decode_amd as pad

    lib = _native.capi()
    lens = [1, 77, 400, 1000, 2500]
    q, k, v, bt, sl = _case(lens, 16, 2, 6, 128, seed=44)
    qd, kd, vd, btd, sld = q.half().cuda(), k.half().cuda(), v.half().cuda(), bt.cuda(), sl.cuda()
    scale = 1.0 / math.sqrt(128)
    stream = torch.cuda.current_stream().cuda_stream
    ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    counters = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    ref = torch.empty_like(qd)
    dm = _native.dims_for(qd, kd, vd, btd, sld, ref)
    assert lib.pad_decode_launch(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), btd.data_ptr(), sld.data_ptr(),
                                 ref.data_ptr(), ws.data_ptr(), ws.numel(), counters.data_ptr(), counters.numel(),
                                 ctypes.byref(dm), scale, 0, stream) == 0
    out = torch.empty_like(qd)
    c = _native.PadCall(q=qd.data_ptr(), k_cache=kd.data_ptr(), v_cache=vd.data_ptr(), block_table=btd.data_ptr(),
                        seq_lens=sld.data_ptr(), out=out.data_ptr(), workspace=ws.data_ptr(),
                        workspace_bytes=ws.numel(), counters=counters.data_ptr(), num_counters=counters.numel(),
                        scale=scale, num_splits=0, engine=0, kv_format=0, k_scale=1.0, v_scale=1.0)
    assert lib.pad_decode_launch_call(ctypes.byref(c), ctypes.byref(dm), stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    # fp8 codes with a CSR index and a work list planned through the descriptor.
    ks, vs = float(k.abs().max()) / 300.0, float(v.abs().max()) / 111.0
    k8, v8 = _quant(k, "e5m2", ks).cuda(), _quant(v, "e5m2", vs).cuda()
    indptr, indices, last = _csr_of(bt, sl, 16)
    out8 = torch.empty_like(qd)
    d8 = _native.dims_for(qd, k8, v8, indices.view(1, -1), last, out8)
    d8.max_pages, d8.bt_stride[0], d8.bt_stride[1] = indices.numel(), 0, 1
    wlb = ctypes.c_size_t()
    assert lib.pad_decode_worklist_bytes(ctypes.byref(d8), 0, 0, 1, ctypes.byref(wlb)) == 0
    wl = torch.empty(wlb.value, dtype=torch.uint8, device="cuda")
    c8 = _native.PadCall(q=qd.data_ptr(), k_cache=k8.data_ptr(), v_cache=v8.data_ptr(), block_table=indices.data_ptr(),
                         indptr=indptr.data_ptr(), last_page_len=last.data_ptr(), out=out8.data_ptr(),
                         workspace=ws.data_ptr(), workspace_bytes=ws.numel(), counters=counters.data_ptr(),
                         num_counters=counters.numel(), worklist=wl.data_ptr(), worklist_bytes=wl.numel(),
                         scale=scale, num_splits=0, engine=0, kv_format=2, k_scale=ks, v_scale=vs)
    assert lib.pad_decode_plan_worklist_call(ctypes.byref(c8), ctypes.byref(d8), wl.data_ptr(), wl.numel(),
                                             stream) == 0
    assert lib.pad_decode_launch_call(ctypes.byref(c8), ctypes.byref(d8), stream) == 0
    want = pad.paged_attention_decode_csr(qd, k8, v8, indptr, indices, last, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    assert torch.equal(out8, want)
    assert_parity(out8.cpu(), decode_fp8_protocol(q, k8.cpu(), v8.cpu(), bt, sl, ks, vs))
    assert torch.all(counters == 0)


FUZZ = int(__import__("os").environ.get("PAD_KERNEL_FUZZ_ITERS", "20"))


@pytest.mark.parametrize("seed", range(FUZZ))
def test_fp8_fuzz_matrix(seed):
    # Both formats, fp16 or bf16 q, over head_dim 64/128/256, group sizes to
    # 16, every block mode, ragged batches with empty rows, random scales,
    # the heuristic plan, a fixed split and 60 splits (two-level merge),
    # dense and CSR; oracle parity on the dequantised caches.
    import random

    import paged_attention_decode_amd as pad
    from tests.helpers import random_case

    rng = random.Random(9000 + seed)
    fmt = rng.choice(list(FMTS))
    q_dtype = rng.choice((torch.float16, torch.bfloat16))
    q, k, v, bt, sl = random_case(9100 + seed, kv_heads=(1, 2, 4), gqa=(1, 3, 8, 16), head_dims=(64, 128, 256),
                                  page_sizes=(1, 2, 3, 4, 8, 12, 16, 24, 32), min_len=0, max_len=400)
    ps = k.shape[1]
    ks = float(k.abs().max()) / rng.uniform(100.0, 400.0)
    vs = float(v.abs().max()) / rng.uniform(20.0, 400.0)
    k8, v8 = _quant(k, fmt, ks), _quant(v, fmt, vs)
    expected = decode_fp8_protocol(q, k8, v8, bt, sl, ks, vs, q_dtype=q_dtype)
    check = assert_parity if q_dtype == torch.float16 else _close_bf16
    qd, kd, vd = q.to(q_dtype).cuda(), k8.cuda(), v8.cuda()
    indptr, indices, last = _csr_of(bt, sl, ps)
    for s in (None, 4, 60):
        a = pad.paged_attention_decode_fp8(qd, kd, vd, bt.cuda(), sl.cuda(), k_scale=ks, v_scale=vs, num_splits=s)
        b = pad.paged_attention_decode_csr(qd, kd, vd, indptr, indices, last, num_splits=s, k_scale=ks,
                                           v_scale=vs)
        torch.cuda.synchronize()
        check(a.cpu(), expected)
        check(b.cpu(), expected)


# fp8 caches with bfloat16 q and output (PAD_KV_FP8_*_BF16): the codes widen
# to bf16 exactly, the rest is the bfloat16 path (bf16 MFMAs, P and output
# rounded to bf16), so the tolerance is the bf16 one, atol = rtol = 1e-2.
BF16_TOL = 1e-2


def _close_bf16(actual, expected):
    a, e = actual.float().cpu(), expected.float().cpu()
    assert torch.isfinite(a).all()
    err = (a - e).abs()
    assert bool((err <= BF16_TOL + BF16_TOL * e.abs()).all()), err.max().item()


@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("ps", [16, 4, 12])
def test_fp8_caches_with_bf16_q_match_oracle(fmt, d, ps):
    import paged_attention_decode_amd as pad

    lens = [1, ps + 3, 150, 777, 0]
    q, k, v, bt, sl = _case(lens, ps, 2, 6, d, seed=ps + d + 500)
    ks, vs = float(k.abs().max()) / 300.0, float(v.abs().max()) / 111.0
    k8, v8 = _quant(k, fmt, ks), _quant(v, fmt, vs)
    expected = decode_fp8_protocol(q, k8, v8, bt, sl, ks, vs, q_dtype=torch.bfloat16)
    qd = q.bfloat16().cuda()
    for splits in (None, 1, 5):
        out = pad.paged_attention_decode_fp8(qd, k8.cuda(), v8.cuda(), bt.cuda(), sl.cuda(), k_scale=ks,
                                             v_scale=vs, num_splits=splits)
        torch.cuda.synchronize()
        assert out.dtype == torch.bfloat16
        _close_bf16(out, expected)


@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("d", [64, 128, 256])
def test_fp8_caches_with_bf16_q_equal_the_bf16_kernel_bitwise(fmt, d):
    # Unit scales: the same arithmetic as the bfloat16 kernel on PyTorch's
    # widening of the codes to bf16, bit for bit, on random data and on every
    # finite code.
    import paged_attention_decode_amd as pad

    q, k, v, bt, sl = _case([7, 300, 1500, 64], 16, 2, 4, d, seed=d + 3)
    dt = FMTS[fmt]
    codes = torch.arange(256, dtype=torch.uint8)
    finite = codes[torch.isfinite(codes.view(dt).float())]
    idx = torch.arange(k.numel())
    every = finite[(idx * 7) % finite.numel()].view(k.shape).view(dt)
    q = q * (1e-4 if fmt == "e5m2" else 1e-2)
    qd, btd, sld = q.bfloat16().cuda(), bt.cuda(), sl.cuda()
    for k8, v8 in ((k.to(dt), v.to(dt)), (every, v.to(dt))):
        for splits in (None, 1, 8):
            a = pad.paged_attention_decode_fp8(qd, k8.cuda(), v8.cuda(), btd, sld, num_splits=splits)
            b = pad.paged_attention_decode_ex(qd, k8.bfloat16().cuda(), v8.bfloat16().cuda(), btd, sld,
                                              num_splits=splits)
            torch.cuda.synchronize()
            assert torch.equal(a, b), (splits, (a.float() - b.float()).abs().max().item())


def test_fp8_caches_with_bf16_q_through_csr_and_wrapper():
    import paged_attention_decode_amd as pad

    lens = [4096, 300, 2500, 1, 777, 0, 1500, 64]
    q, k, v, bt, sl = _case(lens, 16, 2, 6, 128, seed=45)
    ks, vs = float(k.abs().max()) / 300.0, float(v.abs().max()) / 111.0
    k8, v8 = _quant(k, "e4m3fn", ks), _quant(v, "e4m3fn", vs)
    kd, vd, btd, sld = k8.cuda(), v8.cuda(), bt.cuda(), sl.cuda()
    indptr, indices, last = _csr_of(bt, sl, 16)
    qd = q.bfloat16().cuda()
    w = pad.BatchDecodeWrapper()
    w.plan(indptr, indices, last, 12, 2, 128, 16, q_data_type=torch.bfloat16, kv_data_type="e4m3fn")
    a = w.run(qd, (kd, vd), k_scale=ks, v_scale=vs)
    b = pad.paged_attention_decode_csr(qd, kd, vd, indptr, indices, last, k_scale=ks, v_scale=vs)
    c = pad.paged_attention_decode_fp8(qd, kd, vd, btd, sld, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and a.dtype == torch.bfloat16
    expected = decode_fp8_protocol(q, k8, v8, bt, sl, ks, vs, q_dtype=torch.bfloat16)
    _close_bf16(a, expected)
    _close_bf16(c, expected)


@pytest.mark.parametrize("q_dtype", [torch.float16, torch.bfloat16])
def test_fp8_strided_caches(q_dtype):
    # fp8 caches as views of a wider buffer (an extra kv head, a padded row
    # of 136 elements: strides in bytes, multiples of 8), q a slice of a
    # wider tensor.
    import paged_attention_decode_amd as pad

    lens = [40, 90]
    q, k, v, bt, sl = _case(lens, 16, 2, 6, 128, seed=61, spare=1, extra=0)
    ks, vs = float(k.abs().max()) / 300.0, float(v.abs().max()) / 111.0
    k8, v8 = _quant(k, "e4m3fn", ks), _quant(v, "e4m3fn", vs)
    expected = decode_fp8_protocol(q, k8, v8, bt, sl, ks, vs, q_dtype=q_dtype)
    n = k.shape[0]
    kw = torch.zeros(n, 16, 3, 136, dtype=torch.uint8, device="cuda")
    vw = torch.zeros(n, 16, 3, 136, dtype=torch.uint8, device="cuda")
    kw[:, :, :2, :128] = k8.view(torch.uint8).cuda()
    vw[:, :, :2, :128] = v8.view(torch.uint8).cuda()
    kv8 = kw.view(torch.float8_e4m3fn)[:, :, :2, :128]
    vv8 = vw.view(torch.float8_e4m3fn)[:, :, :2, :128]
    qw = torch.zeros(2, 12, 256, dtype=q_dtype, device="cuda")
    qw[:, :, 64:192] = q.to(q_dtype).cuda()
    out = pad.paged_attention_decode_fp8(qw[:, :, 64:192], kv8, vv8, bt.cuda(), sl.cuda(), k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    if q_dtype == torch.float16:
        assert_parity(out.cpu(), expected)
    else:
        _close_bf16(out, expected)


@pytest.mark.parametrize("q_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("splits", [1, 5, 60])
def test_fp8_wrapper_with_explicit_splits(q_dtype, splits):
    # Work lists planned with an explicit split count (two-level merge at 60)
    # equal the one-shot calls with the same count, dense and CSR.
    import paged_attention_decode_amd as pad

    lens = [4096, 300, 2500, 1, 777, 0]
    q, k, v, bt, sl = _case(lens, 12, 2, 6, 128, seed=47)
    ks, vs = float(k.abs().max()) / 300.0, float(v.abs().max()) / 111.0
    k8, v8 = _quant(k, "e5m2", ks).cuda(), _quant(v, "e5m2", vs).cuda()
    btd, sld, qd = bt.cuda(), sl.cuda(), q.to(q_dtype).cuda()
    indptr, indices, last = _csr_of(bt, sl, 12)
    wd, wc = pad.BatchDecodeWrapper(), pad.BatchDecodeWrapper()
    wd.plan_block_table(btd, sld, 12, 2, 128, 12, num_splits=splits, kv_data_type="e5m2", q_data_type=q_dtype)
    wc.plan(indptr, indices, last, 12, 2, 128, 12, num_splits=splits, kv_data_type="e5m2", q_data_type=q_dtype)
    a = wd.run(qd, (k8, v8), k_scale=ks, v_scale=vs)
    b = pad.paged_attention_decode_fp8(qd, k8, v8, btd, sld, k_scale=ks, v_scale=vs, num_splits=splits)
    c = wc.run(qd, (k8, v8), k_scale=ks, v_scale=vs)
    d = pad.paged_attention_decode_csr(qd, k8, v8, indptr, indices, last, num_splits=splits, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(c, d)

"""Plan once, run many: the work-list path (BatchDecodeWrapper, pad_decode_plan_worklist).

GPU: a decode run from a work list must return exactly (bit for bit) what the
same call returns when the kernel plans its items itself, for every way the
launcher picks items: the in-kernel planner on ragged batches (up to 64 and
past 64 sequences), the oversubscribed grid (one item per unit, or two
static splits per unit on the first workgroups, for full rows; chunks over
the whole grid for ragged ones), the static split (full batches, an
explicit num_splits), empty sequences, block modes
other than whole-page blocks, and the CSR index.  One list serves several
runs with different q/K/V; a list planned for another split count is
detected and ignored; a list planned from other sequence lengths leaves the
scratch counters as every launch must (later launches stay correct).  The
FlashInfer-style ``plan(indptr, indices, last_page_len, ...)`` /
``run(q, (k_cache, v_cache))`` surface is checked against the fp32 oracle
on the cases of the reference's tests/test_flashinfer_adapter.py:34-136.

The lists themselves are checked for structure: every (sequence, kv head)
unit's pages are covered by its items exactly once and in order, an empty
unit has the one item that writes its zero rows, the item slots of a unit
are its own contiguous range, and each wave's first page id is the table's.

CPU: the work-list size is a header plus one record per workgroup; the
structure check rejects planted mistakes in a hand-built list.
"""

from __future__ import annotations

import ctypes
import random

import pytest
import torch

from oracle.reference import decode_fp16_protocol
from paged_attention_decode_amd import _native
from tests.helpers import assert_parity, make_cache, shuffled_table

WL_HEADER_BYTES = 128
WL_RECORD_BYTES = 128


# ---------------------------------------------------------------- CPU
@pytest.mark.parametrize("batch,hkv,num_splits", [(1, 2, 16), (32, 2, 4), (3, 8, 0), (0, 2, 0)])
def test_worklist_bytes_is_header_plus_one_record_per_workgroup(batch, hkv, num_splits):
    lib = _native.capi()
    d = _native.PadDims()
    d.batch, d.num_q_heads, d.num_kv_heads, d.head_dim = batch, 6 * hkv, hkv, 128
    d.page_size, d.max_pages, d.num_pages = 16, 256, 1 << 20
    d.q_stride[2] = d.k_stride[3] = d.v_stride[3] = d.out_stride[2] = 1
    for csr in (0, 1):
        plan = _native.PadPlan()
        fn = lib.pad_decode_plan_csr if csr else lib.pad_decode_plan
        assert fn(ctypes.byref(d), num_splits, 256, ctypes.byref(plan)) == 0
        nbytes = ctypes.c_size_t()
        assert lib.pad_decode_worklist_bytes(ctypes.byref(d), num_splits, 256, csr, ctypes.byref(nbytes)) == 0
        assert nbytes.value == WL_HEADER_BYTES + WL_RECORD_BYTES * plan.num_splits * hkv * batch


# ---------------------------------------------------------------- GPU
def _extra_cols(kind):
    return 0 if kind.endswith("_exact") else 1


def _dense_case(lens, hkv, group, d, ps, seed, extra_cols=1):
    bt, num_pages = shuffled_table(lens, ps, spare_pages=3, extra_cols=extra_cols, seed=seed)
    k, v = make_cache(num_pages, ps, hkv, d, seed, dtype=torch.float16)
    g = torch.Generator().manual_seed(seed + 1)
    q = torch.randn(len(lens), hkv * group, d, generator=g).half()
    return q.cuda(), k.cuda(), v.cuda(), bt.cuda(), torch.tensor(lens, dtype=torch.int32).cuda()


def _lens(kind, seed):
    rng = random.Random(seed)
    if kind == "ragged32":  # the planner, 32 sequences (C3-like lengths)
        lens = [rng.randint(1, 8192) for _ in range(32)]
        lens[0] = 1
        return lens, 32
    if kind == "ragged100":  # the planner with 4 sequences per lane
        return [rng.randint(0, 3000) for _ in range(100)], 16
    if kind == "oversub":  # at least as many units as CUs: one item per unit when full
        return [rng.randint(1, 700) for _ in range(200)], 16
    if kind == "oversub_full":
        return [640] * 200, 16
    if kind == "oversub_exact":  # every row exactly full (no spare column): one item per unit
        return [640] * 200, 16
    if kind == "mid":  # 65-127 units: the oversubscribed grid, chunks over all of it
        return [rng.randint(1, 4096) for _ in range(48)], 16
    if kind == "mid_exact":  # the same grid, rows exactly full: two static splits per unit
        return [2048] * 48, 16
    if kind == "mid3_exact":  # 80 units, rows exactly full: three static splits per unit
        return [2048] * 40, 16
    if kind == "full16":  # every sequence at capacity: the static split
        return [4096] * 16, 16
    if kind == "empty":
        lens = [rng.randint(0, 900) for _ in range(12)]
        lens[3] = lens[7] = 0
        return lens, 16
    if kind == "allempty":  # no sequence has a page (the CSR index has no entries)
        return [0] * 5, 16
    raise ValueError(kind)


GPU_CASES = [
    # (lens kind, hkv, group, head_dim, page_size, num_splits)
    ("ragged32", 2, 6, 128, 32, None),
    ("ragged32", 2, 6, 128, 32, 4),
    ("ragged100", 4, 4, 128, 16, None),
    ("oversub", 2, 6, 128, 16, None),
    ("oversub_full", 2, 6, 128, 16, None),
    # head_dim 96 and 32 with an even kv-head count: kv heads paired on an
    # XCD (grid_pos), so a workgroup's index differs from its unit's
    ("oversub_full", 2, 6, 96, 16, None),
    ("oversub_full", 2, 4, 32, 16, None),
    ("oversub", 2, 6, 96, 16, None),
    ("oversub_exact", 2, 6, 128, 16, None),
    ("mid", 2, 6, 128, 16, None),
    ("mid_exact", 2, 6, 128, 16, None),
    ("mid_exact", 2, 6, 96, 16, None),  # head pairing off on this grid
    ("mid3_exact", 2, 6, 128, 16, None),
    ("full16", 2, 6, 128, 16, None),
    ("empty", 2, 6, 128, 16, None),
    ("empty", 2, 6, 64, 8, None),  # sub-page blocks
    ("empty", 1, 8, 128, 12, None),  # generic page size
    ("allempty", 2, 6, 128, 16, None),
    ("ragged100", 4, 4, 256, 16, None),
]


@pytest.mark.gpu
@pytest.mark.parametrize("kind,hkv,group,d,ps,num_splits", GPU_CASES)
def test_planned_run_equals_in_kernel_plan(kind, hkv, group, d, ps, num_splits):
    import paged_attention_decode_amd as pad

    lens, seed = _lens(kind, 11)[0], 11
    q, k, v, bt, sl = _dense_case(lens, hkv, group, d, ps, seed, _extra_cols(kind))
    w = pad.BatchDecodeWrapper()
    w.plan_block_table(bt, sl, q.shape[1], hkv, d, ps, num_splits=num_splits)
    out = w.run(q, (k, v))
    ref = pad.paged_attention_decode(q, k, v, bt, sl, num_splits=num_splits)
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"max diff {(out.float() - ref.float()).abs().max().item()}"
    # The same list serves another layer's q / K / V.
    q2 = torch.randn_like(q.float()).half()
    k2, v2 = torch.randn_like(k.float()).half(), torch.randn_like(v.float()).half()
    out2 = w.run(q2, (k2, v2))
    ref2 = pad.paged_attention_decode(q2, k2, v2, bt, sl, num_splits=num_splits)
    torch.cuda.synchronize()
    assert torch.equal(out2, ref2)


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["ragged32", "empty", "oversub", "allempty"])
def test_planned_csr_run_equals_in_kernel_plan(kind):
    import paged_attention_decode_amd as pad

    lens, _ = _lens(kind, 23)
    ps = 16
    q, k, v, bt, sl = _dense_case(lens, 2, 6, 128, ps, 23)
    indptr, indices, last = pad.paged_kv_indices(bt, sl, ps)
    w = pad.BatchDecodeWrapper()
    w.plan(indptr, indices, last, 12, 2, 128, ps)
    out = w.run(q, (k, v))
    ref = pad.paged_attention_decode_csr(q, k, v, indptr, indices, last)
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"max diff {(out.float() - ref.float()).abs().max().item()}"


# The reference's FlashInfer adapter cases (tests/test_flashinfer_adapter.py):
# primary shape :34-58, page-boundary remainder :61-75, exact multiple
# :78-94, GQA ratios :97-109, ragged batch :112-136.
ADAPTER_CASES = [
    ([200, 333, 64], 2, 6, 16),
    ([17, 33], 2, 4, 16),
    ([64, 128], 2, 4, 16),
    ([100, 250], 4, 1, 16),
    ([100, 250], 2, 8, 16),
    ([5, 300, 1, 48, 129], 2, 6, 16),
]


@pytest.mark.gpu
@pytest.mark.parametrize("lens,hkv,group,ps", ADAPTER_CASES)
def test_plan_run_matches_oracle_on_adapter_cases(lens, hkv, group, ps):
    import paged_attention_decode_amd as pad

    seed = 31 + len(lens)
    bt, num_pages = shuffled_table(lens, ps, spare_pages=2, extra_cols=1, seed=seed)
    k, v = make_cache(num_pages, ps, hkv, 128, seed)
    q = torch.randn(len(lens), hkv * group, 128, generator=torch.Generator().manual_seed(seed + 1))
    sl = torch.tensor(lens, dtype=torch.int32)
    qh, kh, vh = q.half(), k.half(), v.half()
    indptr, indices, last = pad.paged_kv_indices(bt.cuda(), sl.cuda(), ps)
    w = pad.BatchDecodeWrapper()
    w.plan(indptr, indices, last, hkv * group, hkv, 128, ps)
    out = w.run(qh.cuda(), (kh.cuda(), vh.cuda()))
    assert_parity(out, decode_fp16_protocol(qh.float(), kh.float(), vh.float(), bt, sl))


def _capi_args(q, k, v, bt, sl, out):
    return _native.dims_for(q, k, v, bt, sl, out)


@pytest.mark.gpu
def test_list_for_another_split_count_is_ignored():
    # Planned with 2 splits, launched with 8: the header's key does not match,
    # so the kernel plans in-kernel and the result is the 8-split launch's.
    lib = _native.capi()
    lens = [4096] * 4
    q, k, v, bt, sl = _dense_case(lens, 2, 6, 128, 16, 41)
    out = torch.empty_like(q)
    ref = torch.empty_like(q)
    d = _capi_args(q, k, v, bt, sl, out)
    stream = torch.cuda.current_stream().cuda_stream
    nbytes = ctypes.c_size_t()
    assert lib.pad_decode_worklist_bytes(ctypes.byref(d), 8, 0, 0, ctypes.byref(nbytes)) == 0
    wl = torch.empty(nbytes.value, dtype=torch.uint8, device="cuda")
    assert lib.pad_decode_plan_worklist(bt.data_ptr(), sl.data_ptr(), ctypes.byref(d), 2, wl.data_ptr(),
                                        wl.numel(), stream) == 0
    ws_bytes, n_cnt = ctypes.c_size_t(), ctypes.c_int64()
    assert lib.pad_decode_workspace_bytes(ctypes.byref(d), 8, 0, ctypes.byref(ws_bytes)) == 0
    assert lib.pad_decode_counters_needed(ctypes.byref(d), 8, 0, ctypes.byref(n_cnt)) == 0
    ws = torch.empty(max(ws_bytes.value, 256), dtype=torch.uint8, device="cuda")
    cnt = torch.zeros(max(n_cnt.value, 1), dtype=torch.int32, device="cuda")
    scale = ctypes.c_float(128 ** -0.5)
    st = lib.pad_decode_launch_worklist(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                                        out.data_ptr(), ws.data_ptr(), ws.numel(), cnt.data_ptr(), cnt.numel(),
                                        ctypes.byref(d), scale, 8, wl.data_ptr(), wl.numel(), stream)
    assert st == 0
    st = lib.pad_decode_launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                               ref.data_ptr(), ws.data_ptr(), ws.numel(), cnt.data_ptr(), cnt.numel(),
                               ctypes.byref(d), scale, 8, stream)
    assert st == 0
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert int(cnt.abs().sum()) == 0
    # Status codes: a list too small for the launch's plan, and none at all.
    st = lib.pad_decode_launch_worklist(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                                        out.data_ptr(), ws.data_ptr(), ws.numel(), cnt.data_ptr(), cnt.numel(),
                                        ctypes.byref(d), scale, 8, wl.data_ptr(), 256, stream)
    assert st == 7  # PAD_ERR_WORKSPACE
    st = lib.pad_decode_launch_worklist(q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(),
                                        out.data_ptr(), ws.data_ptr(), ws.numel(), cnt.data_ptr(), cnt.numel(),
                                        ctypes.byref(d), scale, 8, None, 0, stream)
    assert st == 1  # PAD_ERR_NULL_POINTER


@pytest.mark.gpu
def test_list_from_other_lengths_keeps_scratch_consistent():
    # A list planned from one set of lengths and run with another (same
    # shapes) gives rows of the planned items; its merges still complete, so
    # the counters return to zero and the next launches are correct.
    import paged_attention_decode_amd as pad

    rng = random.Random(5)
    lens_a = [rng.randint(1, 4000) for _ in range(24)]
    lens_b = [rng.randint(1, 4000) for _ in range(24)]
    bt, num_pages = shuffled_table([4096] * 24, 16, spare_pages=2, extra_cols=0, seed=5)
    k, v = make_cache(num_pages, 16, 2, 128, 5, dtype=torch.float16)
    q = torch.randn(24, 12, 128, generator=torch.Generator().manual_seed(6)).half()
    qc, kc, vc, btc = q.cuda(), k.cuda(), v.cuda(), bt.cuda()
    sla = torch.tensor(lens_a, dtype=torch.int32).cuda()
    slb = torch.tensor(lens_b, dtype=torch.int32).cuda()
    w = pad.BatchDecodeWrapper()
    w.plan_block_table(btc, sla, 12, 2, 128, 16)
    stale = pad.ops.ext().forward_worklist(qc, kc, vc, btc, slb, w._plan[2], 128 ** -0.5, 0)
    torch.cuda.synchronize()
    assert torch.isfinite(stale.float()).all()
    out = pad.paged_attention_decode(qc, kc, vc, btc, slb)
    assert_parity(out, decode_fp16_protocol(q.float(), k.float(), v.float(), bt, torch.tensor(lens_b)))
    out_a = w.run(qc, (kc, vc))
    assert torch.equal(out_a, pad.paged_attention_decode(qc, kc, vc, btc, sla))


# ---------------------------------------------------------------- plan structure
WL_INTS = WL_RECORD_BYTES // 4


def _check_plan_structure(wl, lens, ps, hkv, bt_rows, nw, max_pages):
    """The items a work list holds cover every (sequence, kv head) unit's pages exactly once.

    wl: the list as int32 on the host; lens: sequence lengths; bt_rows[b]: the
    page ids of sequence b in order (its row of the dense table, or its CSR
    slice); nw: waves per workgroup."""
    assert wl[0] == 0x574C4150
    G = int(wl[2])
    recs = wl[WL_INTS:WL_INTS + WL_INTS * G].view(G, WL_INTS)
    units = {}
    for g in range(G):
        r = recs[g].tolist()
        b, kvh, p0, p1, L, nsplit, slot0, col_max, valid = r[:9]
        if not valid:
            continue
        assert 0 <= b < len(lens) and 0 <= kvh < hkv and L == lens[b]
        pages = min(-(-L // ps), max_pages)
        units.setdefault((b, kvh), []).append((p0, p1, g, nsplit, slot0))
        if pages == 0:
            assert nsplit == 0
            continue
        assert 0 <= p0 < p1 <= pages and slot0 <= g < slot0 + nsplit and col_max >= p1 - 1
        if ps % 16 == 0:  # whole-page blocks: each wave's first page id is in the record
            for w in range(nw):
                col = min(p0 + (w * 16) // ps, col_max)
                assert r[16 + w] == int(bt_rows[b][col]), (g, w)
    slots = []
    for b, L in enumerate(lens):
        pages = min(-(-L // ps), max_pages)
        for kvh in range(hkv):
            items = sorted(units.get((b, kvh), []))
            if pages == 0:
                assert len(items) == 1, (b, kvh)  # one workgroup writes the zero rows
                continue
            assert len(items) == items[0][3], (b, kvh)  # nsplit items
            assert items[0][0] == 0 and items[-1][1] == pages, (b, kvh)
            for (_, e, *_), (s, *_) in zip(items, items[1:]):
                assert e == s, (b, kvh)  # contiguous, no overlap
            slot0 = items[0][4]
            assert all(it[4] == slot0 for it in items)
            assert sorted(it[2] for it in items) == list(range(slot0, slot0 + len(items)))
            slots.append((slot0, slot0 + len(items)))
    slots.sort()
    for (_, e), (s, _) in zip(slots, slots[1:]):
        assert e <= s  # units' slot ranges are disjoint


@pytest.mark.gpu
@pytest.mark.parametrize("kind,ps,csr,d", [("ragged32", 32, False, 128), ("ragged100", 16, False, 128),
                                           ("oversub", 16, False, 128), ("full16", 16, False, 128),
                                           ("empty", 16, False, 128), ("allempty", 16, False, 128),
                                           ("ragged32", 32, True, 128), ("empty", 8, True, 128),
                                           ("oversub_full", 16, False, 96), ("oversub_full", 16, False, 32),
                                           ("oversub", 16, False, 96), ("ragged32", 32, False, 96),
                                           ("oversub_exact", 16, False, 128), ("mid", 16, False, 128),
                                           ("mid_exact", 16, False, 128), ("mid_exact", 16, False, 96),
                                           ("mid3_exact", 16, False, 128)])
def test_work_list_covers_every_page_once(kind, ps, csr, d):
    import paged_attention_decode_amd as pad
    from paged_attention_decode_amd._native import ext

    lens, seed = _lens(kind, 31)
    hkv, group = 2, 6
    q, k, v, bt, sl = _dense_case(lens, hkv, group, d, ps, seed, _extra_cols(kind))
    if csr:
        indptr, indices, last = pad.paged_kv_indices(bt, sl, ps)
        plan = lambda: ext().plan_worklist_csr(indptr, indices, last, hkv * group, hkv, d, ps, 0)  # noqa: E731
        ip = indptr.cpu().tolist()
        rows = [indices.cpu()[ip[b]:ip[b + 1]].tolist() for b in range(len(lens))]
        max_pages = 1 << 30
        nw = pad.plan(len(lens), hkv * group, hkv, d, ps, max(indices.numel(), 1), csr=True)["waves_per_group"]
    else:
        plan = lambda: ext().plan_worklist(bt, sl, hkv * group, hkv, d, ps, 0)  # noqa: E731
        rows = bt.cpu().tolist()
        max_pages = bt.shape[1]
        nw = pad.plan(len(lens), hkv * group, hkv, d, ps, max_pages)["waves_per_group"]
    wl = plan()
    # Planning the same inputs again (into fresh memory) gives the same list
    # word for word, including the records of slots without an item.
    junk = torch.full((wl.numel(),), 0x5A, dtype=torch.uint8, device="cuda")
    del junk
    wl2 = plan()
    torch.cuda.synchronize()
    assert torch.equal(wl, wl2)
    _check_plan_structure(wl.cpu().view(torch.int32), lens, ps, hkv, rows, nw, max_pages)


def _synthetic_list():
    # Two sequences of 5 and 0 pages (page size 16), one kv head, 4 slots:
    # sequence 0 in items [0, 3) and [3, 5) (slots 0, 1), sequence 1's zero
    # rows in slot 2, slot 3 without an item.
    wl = torch.zeros(WL_INTS * 5, dtype=torch.int32)
    wl[0], wl[2] = 0x574C4150, 4
    rows = [[10, 11, 12, 13, 14, 15], [20, 21, 22, 23, 24, 25]]

    def rec(g, vals, pids):
        base = WL_INTS * (1 + g)
        wl[base:base + len(vals)] = torch.tensor(vals, dtype=torch.int32)
        wl[base + 16:base + 16 + len(pids)] = torch.tensor(pids, dtype=torch.int32)

    # b, kvh, p_begin, p_end, L, nsplit, slot0, col_max, valid, row
    rec(0, [0, 0, 0, 3, 70, 2, 0, 5, 1, 0], [10, 11])
    rec(1, [0, 0, 3, 5, 70, 2, 0, 5, 1, 0], [13, 14])
    rec(2, [1, 0, 0, 0, 0, 0, 2, -1, 1, 0], [])
    return wl, rows


def test_plan_structure_check_catches_planted_mistakes():
    lens, ps, hkv, nw, max_pages = [70, 0], 16, 1, 2, 6
    wl, rows = _synthetic_list()
    _check_plan_structure(wl, lens, ps, hkv, rows, nw, max_pages)
    base = WL_INTS
    mistakes = [
        (base * 2 + 2, 2),   # second item starts inside the first: overlap
        (base * 2 + 3, 4),   # a page left uncovered at the end
        (base * 1 + 16, 12),  # wrong first page id of wave 0
        (base * 2 + 6, 1),   # inconsistent slot0 inside a unit
        (base * 3 + 8, 0),   # the empty sequence's zero rows have no item
    ]
    for idx, val in mistakes:
        bad = wl.clone()
        bad[idx] = val
        with pytest.raises(AssertionError):
            _check_plan_structure(bad, lens, ps, hkv, rows, nw, max_pages)

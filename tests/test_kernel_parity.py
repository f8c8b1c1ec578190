"""GPU parity of the HIP decode path against the CPU oracle.

Mirrors the reference's tests/test_kernel_cuda_v4.py (primary shape :36-59,
split invariance :62-76, num_splits=1 anchor :79-111, oversplit :114-127,
partial page :130-141, GQA ratios :144-155, ragged :158-178, fuzz :181-190)
for both phase-1 engines, with the fp16-rounding protocol of
tests/kernel_test_utils.py:47-51 (the oracle sees the same fp16 inputs).

Tolerance: atol = rtol = 2e-3 against the fp32 oracle (the contract), and the
reference's own rtol 1e-2 / atol 1e-3 (assert_parity checks both).
"""

from __future__ import annotations

import os

import random

import pytest
import torch

from oracle.reference import decode_fp16_protocol
from tests.helpers import (
    assert_parity,
    cdiv,
    contiguous_table,
    make_cache,
    random_case,
    shuffled_table,
)

pytestmark = pytest.mark.gpu

FUZZ = int(os.environ.get("PAD_KERNEL_FUZZ_ITERS", "20"))
ENGINES = [0, 1]


def _run(q, k, v, bt, sl, engine=0, **kw):
    import paged_attention_decode_amd as pad

    dev = "cuda"
    return pad.paged_attention_decode_ex(q.half().to(dev), k.half().to(dev), v.half().to(dev), bt.to(dev),
                                         sl.to(dev), engine=engine, **kw)


def _check(q, k, v, bt, sl, engine=0, num_splits=None, scale=None):
    expected = decode_fp16_protocol(q, k, v, bt, sl, scale)
    actual = _run(q, k, v, bt, sl, engine=engine, num_splits=num_splits, scale=scale)
    assert actual.dtype == torch.float16 and actual.shape == q.shape
    assert_parity(actual, expected)
    return actual


def _engine_ok(engine, group, d):
    return engine == 0 or (d in (64, 128) and group <= 8)


@pytest.mark.parametrize("engine", ENGINES)
@pytest.mark.parametrize("num_splits", [None, 1, 8])
def test_primary_target_shape(engine, num_splits):
    lens = [1, 17, 256, 4000]
    bt, total = contiguous_table(lens, 16, extra_cols=0)
    k, v = make_cache(total + 3, 16, 2, 128, seed=0)
    q = torch.randn(4, 12, 128, generator=torch.Generator().manual_seed(0))
    _check(q, k, v, bt, torch.tensor(lens, dtype=torch.int32), engine, num_splits)


@pytest.mark.parametrize("engine", ENGINES)
@pytest.mark.parametrize("num_splits", [1, 2, 4, 8, 16, 64, 125, 200])
def test_split_invariance(engine, num_splits):
    seq, ps = 2000, 16
    n = cdiv(seq, ps)
    k, v = make_cache(n, ps, 2, 128, seed=600 + num_splits)
    q = torch.randn(1, 12, 128, generator=torch.Generator().manual_seed(num_splits))
    _check(q, k, v, torch.arange(n, dtype=torch.int32)[None], torch.tensor([seq], dtype=torch.int32), engine,
           num_splits)


@pytest.mark.parametrize("engine", ENGINES)
def test_split_counts_agree_tightly(engine):
    # num_splits=1 (single pass, phase 1 normalises) is the unsplit anchor
    # (analysis/split_k_derivation.md:88-99); every split count must agree
    # with it far inside the oracle tolerance.
    lens = [1, 17, 4000]
    bt, total = contiguous_table(lens, 16)
    k, v = make_cache(total + 3, 16, 2, 128, seed=42)
    q = torch.randn(3, 12, 128, generator=torch.Generator().manual_seed(42))
    sl = torch.tensor(lens, dtype=torch.int32)
    base = _run(q, k, v, bt, sl, engine, num_splits=1).float()
    for s in (2, 3, 7, 16, 64, 250):
        other = _run(q, k, v, bt, sl, engine, num_splits=s).float()
        torch.testing.assert_close(other, base, rtol=2e-3, atol=1e-3)


@pytest.mark.parametrize("group,d", [(1, 64), (2, 128), (1, 256)])
def test_many_splits_few_rows(group, d):
    # More than 16 splits of 1-2 rows: merges of several 16-split batches
    # (17, 40 splits; the last batch ragged) and of two levels (150 splits).
    lens = [3000, 1111]
    bt, total = contiguous_table(lens, 16)
    k, v = make_cache(total + 2, 16, 4, d, seed=900 + d)
    q = torch.randn(2, 4 * group, d, generator=torch.Generator().manual_seed(900 + group))
    sl = torch.tensor(lens, dtype=torch.int32)
    base = _run(q, k, v, bt, sl, 0, num_splits=1).float()
    for s in (17, 40, 150):
        out = _check(q, k, v, bt, sl, 0, s)
        torch.testing.assert_close(out.float(), base, rtol=2e-3, atol=1e-3)


@pytest.mark.parametrize("group,d", [(1, 64), (4, 64), (4, 128), (1, 128), (2, 256)])
def test_folds_of_many_entries(group, d):
    # The merging workgroup folds a unit's entries in one batch of 4, 8 or
    # 16, or in batches of 16 in turn beyond 16 (here 17 to 47 splits, the
    # last batch ragged), and the group results of two-level merges (stride
    # 16; 300 splits give 19 groups, two batches), with plans of 1 to 8
    # waves per workgroup and 16 to 128 (row, 4 columns) elements per unit.
    # Against the oracle and against one split.
    lens = [16 * 600, 16 * 13 + 5, 16 * 29, 16 * 5 + 1, 16 * 48]
    hkv = 2
    bt, total = contiguous_table(lens, 16)
    k, v = make_cache(total + 1, 16, hkv, d, seed=1200 + d + group)
    q = torch.randn(len(lens), hkv * group, d, generator=torch.Generator().manual_seed(1201 + d + group))
    sl = torch.tensor(lens, dtype=torch.int32)
    base = _run(q, k, v, bt, sl, 0, num_splits=1).float()
    for s in (5, 17, 20, 33, 48, 75, 300, 600):
        out = _check(q, k, v, bt, sl, 0, s)
        torch.testing.assert_close(out.float(), base, rtol=2e-3, atol=1e-3)


@pytest.mark.parametrize("batch,full,d", [(48, True, 128), (48, False, 128), (48, True, 96), (48, False, 96),
                                          (48, True, 64), (40, True, 128), (40, False, 128), (40, True, 96)])
def test_oversubscribed_grid_below_one_unit_per_two_cus(batch, full, d):
    # 96 or 80 units (48 or 40 sequences x 2 kv heads) on 256 CUs: the
    # heuristic grid holds several items per unit.  Rows at full capacity
    # run the static splits, two or three per unit, on its first workgroups
    # (head pairing off at head_dim 96); ragged rows run equal page chunks
    # over the whole grid.
    from paged_attention_decode_amd.heuristics import plan

    rng = random.Random(77 + d + batch)
    lens = [2048] * batch if full else [rng.randint(1, 4096) for _ in range(batch)]
    bt, total = shuffled_table(lens, 16, spare_pages=2, extra_cols=0, seed=78 + d + batch)
    assert (bt.shape[1] == 128) == full
    k, v = make_cache(total, 16, 2, d, seed=79 + d + batch)
    q = torch.randn(batch, 12, d, generator=torch.Generator().manual_seed(80 + d + batch))
    assert plan(batch, 12, 2, d, 16, bt.shape[1]).num_splits > 3
    out = _check(q, k, v, bt, torch.tensor(lens, dtype=torch.int32), 0, None)
    for _ in range(2):  # counters back to zero, same bits
        assert torch.equal(_run(q, k, v, bt, torch.tensor(lens, dtype=torch.int32), 0), out)


@pytest.mark.parametrize("num_splits", [60, 100, 200])
def test_two_level_merge(num_splits):
    # More than 48 splits of one sequence merge in two levels: groups of 16
    # consecutive splits first (the last group ragged), then the groups.
    lens = [5000, 3000, 1]
    bt, total = contiguous_table(lens, 16)
    k, v = make_cache(total + 2, 16, 2, 128, seed=77)
    q = torch.randn(3, 8, 128, generator=torch.Generator().manual_seed(77))
    sl = torch.tensor(lens, dtype=torch.int32)
    base = _run(q, k, v, bt, sl, 0, num_splits=1).float()
    for _ in range(2):  # the group counters come back to zero
        out = _check(q, k, v, bt, sl, 0, num_splits)
        torch.testing.assert_close(out.float(), base, rtol=2e-3, atol=1e-3)


def test_two_level_merge_rows_across_waves():
    # head_dim 96 has 24 four-column elements per row, so with one wave a
    # row's elements span two loop passes: the group merger must not publish
    # a row's (m, l) before every pass has read the original.  (Regression:
    # the last 8 elements of row 2 came out wrong before.)
    lens = [153, 250, 200]
    bt, total = contiguous_table(lens, 1)
    k, v = make_cache(total + 2, 1, 1, 96, seed=1042)
    q = torch.randn(3, 3, 96, generator=torch.Generator().manual_seed(1043))
    _check(q, k, v, bt, torch.tensor(lens, dtype=torch.int32), 0, 60)


def test_two_level_merge_planned_long_row():
    # A long single-kv-head row next to a short one: the in-kernel planner
    # hands the long unit ~255 items, which merge in two levels.
    lens = [131072 - 5, 16]
    bt, total = contiguous_table(lens, 16)
    k, v = make_cache(total + 1, 16, 1, 128, seed=78)
    q = torch.randn(2, 8, 128, generator=torch.Generator().manual_seed(78))
    _check(q, k, v, bt, torch.tensor(lens, dtype=torch.int32), 0, None)


@pytest.mark.parametrize("engine", ENGINES)
def test_oversplit_more_splits_than_tokens(engine):
    k, v = make_cache(1, 16, 2, 128, seed=700)
    q = torch.randn(1, 12, 128, generator=torch.Generator().manual_seed(700))
    _check(q, k, v, torch.zeros(1, 1, dtype=torch.int32), torch.tensor([5], dtype=torch.int32), engine, 8)


@pytest.mark.parametrize("engine", ENGINES)
def test_partial_last_page(engine):
    seq, ps = 100, 16
    n = cdiv(seq, ps)
    k, v = make_cache(n, ps, 2, 128, seed=1)
    q = torch.randn(1, 12, 128, generator=torch.Generator().manual_seed(1))
    _check(q, k, v, torch.arange(n, dtype=torch.int32)[None], torch.tensor([seq], dtype=torch.int32), engine)


@pytest.mark.parametrize("engine", ENGINES)
@pytest.mark.parametrize("group", [1, 2, 4, 6, 8, 16])
def test_gqa_ratios(engine, group):
    if not _engine_ok(engine, group, 128):
        pytest.skip("VALU engine covers groups <= 8")
    seq, ps = 200, 16
    n = cdiv(seq, ps)
    k, v = make_cache(n, ps, 2, 128, seed=100 + group)
    q = torch.randn(1, 2 * group, 128, generator=torch.Generator().manual_seed(group))
    _check(q, k, v, torch.arange(n, dtype=torch.int32)[None], torch.tensor([seq], dtype=torch.int32), engine)


@pytest.mark.parametrize("engine", ENGINES)
def test_ragged_batch_and_row_isolation(engine):
    lens = [3, 17, 100, 512]
    bt, total = contiguous_table(lens, 16)
    k, v = make_cache(total + 3, 16, 2, 128, seed=43)
    q = torch.randn(4, 12, 128, generator=torch.Generator().manual_seed(43))
    sl = torch.tensor(lens, dtype=torch.int32)
    batched = _check(q, k, v, bt, sl, engine)
    for b in range(4):
        solo = _run(q[b:b + 1], k, v, bt[b:b + 1], sl[b:b + 1], engine)
        torch.testing.assert_close(solo.float(), batched[b:b + 1].float(), rtol=2e-3, atol=1e-3)


@pytest.mark.parametrize("engine", ENGINES)
def test_zero_length_rows_give_zeros(engine):
    lens = [0, 20, 0, 33]
    bt, n = shuffled_table(lens, 16, spare_pages=2, extra_cols=1, seed=5)
    k, v = make_cache(n, 16, 2, 128, seed=5)
    q = torch.randn(4, 8, 128, generator=torch.Generator().manual_seed(5))
    for s in (None, 1, 4):
        out = _check(q, k, v, bt, torch.tensor(lens, dtype=torch.int32), engine, s)
        assert torch.all(out[0] == 0) and torch.all(out[2] == 0)


@pytest.mark.parametrize("engine", ENGINES)
def test_block_table_without_columns_gives_zeros(engine):
    # A [batch, 0] table (every sequence empty) is valid input: the oracle
    # returns zeros, and the kernel must not read a page id for it.
    k, v = make_cache(2, 16, 2, 128, seed=6)
    q = torch.randn(3, 8, 128, generator=torch.Generator().manual_seed(6))
    bt = torch.zeros(3, 0, dtype=torch.int32)
    sl = torch.zeros(3, dtype=torch.int32)
    for s in (None, 1, 4):
        out = _check(q, k, v, bt, sl, engine, s)
        assert torch.all(out == 0)


@pytest.mark.parametrize("engine", ENGINES)
def test_poisoned_holes_and_nan_slots(engine):
    # Unused columns/pages and the unused tail slots of the last page hold
    # NaN: a kernel that reads or weights any of them produces NaN.
    lens = [37, 5]
    bt, n = shuffled_table(lens, 16, spare_pages=3, extra_cols=2, seed=9)
    k, v = make_cache(n, 16, 2, 128, seed=9)
    used = {int(bt[0, j]) for j in range(3)} | {int(bt[1, 0])}
    for p in range(n):
        if p not in used:
            k[p] = float("nan")
            v[p] = float("nan")
    last0, last1 = int(bt[0, 2]), int(bt[1, 0])
    k[last0, 5:] = float("nan")
    v[last0, 5:] = float("nan")
    k[last1, 5:] = float("nan")
    v[last1, 5:] = float("nan")
    q = torch.randn(2, 12, 128, generator=torch.Generator().manual_seed(9))
    sl = torch.tensor(lens, dtype=torch.int32)
    k_clean, v_clean = torch.nan_to_num(k), torch.nan_to_num(v)
    expected = decode_fp16_protocol(q, k_clean, v_clean, bt, sl)
    for s in (None, 1, 2):
        assert_parity(_run(q, k, v, bt, sl, engine, num_splits=s), expected)


@pytest.mark.parametrize("engine", ENGINES)
@pytest.mark.parametrize("ps", [1, 2, 4, 8, 12, 16, 32, 64])
def test_page_sizes(engine, ps):
    lens = [1, ps + 3, 150, 77]
    bt, n = shuffled_table(lens, ps, spare_pages=2, extra_cols=1, seed=ps)
    k, v = make_cache(n, ps, 2, 128, seed=ps)
    q = torch.randn(4, 12, 128, generator=torch.Generator().manual_seed(ps))
    for s in (None, 3):
        _check(q, k, v, bt, torch.tensor(lens, dtype=torch.int32), engine, s)


@pytest.mark.parametrize("engine", ENGINES)
@pytest.mark.parametrize("d", [32, 64, 96, 128, 256])
def test_head_dims(engine, d):
    if not _engine_ok(engine, 4, d):
        pytest.skip("VALU engine covers head_dim 64/128")
    lens = [9, 130, 300]
    bt, n = shuffled_table(lens, 16, spare_pages=2, extra_cols=1, seed=d)
    k, v = make_cache(n, 16, 2, d, seed=d)
    q = torch.randn(3, 8, d, generator=torch.Generator().manual_seed(d))
    for s in (None, 1, 5):
        _check(q, k, v, bt, torch.tensor(lens, dtype=torch.int32), engine, s)


@pytest.mark.parametrize("ps", [1, 4, 12, 32])
def test_head_dim_256_block_modes(ps):
    # head_dim 256 reads each token row as two 256-byte halves and stages q in
    # LDS: cover every block mode (sub-page, generic, uniform) and a full
    # 16-row group.
    lens = [5, ps * 7 + 3, 333]
    bt, n = shuffled_table(lens, ps, spare_pages=2, extra_cols=1, seed=256 + ps)
    k, v = make_cache(n, ps, 1, 256, seed=256 + ps)
    q = torch.randn(3, 16, 256, generator=torch.Generator().manual_seed(ps))
    for s in (None, 1, 4):
        _check(q, k, v, bt, torch.tensor(lens, dtype=torch.int32), 0, s)


@pytest.mark.parametrize("engine", ENGINES)
def test_scaled_keys_stress_softmax_range(engine):
    lens = [300, 64]
    bt, n = shuffled_table(lens, 16, spare_pages=1, extra_cols=0, seed=21)
    k, v = make_cache(n, 16, 2, 128, seed=21)
    g = torch.Generator().manual_seed(21)
    for _ in range(6):
        p, s = int(torch.randint(0, n, (1,), generator=g)), int(torch.randint(0, 16, (1,), generator=g))
        k[p, s] *= 8.0
    q = torch.randn(2, 12, 128, generator=g)
    for s in (None, 1, 8):
        _check(q, k, v, bt, torch.tensor(lens, dtype=torch.int32), engine, s)


@pytest.mark.parametrize("engine", ENGINES)
def test_explicit_scale_and_int64_indices(engine):
    lens = [50, 200]
    bt, n = shuffled_table(lens, 16, spare_pages=2, extra_cols=0, seed=31)
    k, v = make_cache(n, 16, 2, 128, seed=31)
    q = torch.randn(2, 12, 128, generator=torch.Generator().manual_seed(31))
    _check(q, k, v, bt.long(), torch.tensor(lens, dtype=torch.int64), engine, None, scale=0.05)


@pytest.mark.parametrize("engine", ENGINES)
def test_strided_inputs(engine):
    # q as a slice of a wider tensor; caches as views of a bigger buffer with
    # padded strides (the reference passes all strides, cuda/kernel_v4_split_k.cu:248-254).
    import paged_attention_decode_amd as pad

    lens = [40, 90]
    bt, n = shuffled_table(lens, 16, spare_pages=1, extra_cols=0, seed=41)
    k, v = make_cache(n, 16, 2, 128, seed=41)
    q = torch.randn(2, 12, 128, generator=torch.Generator().manual_seed(41))
    expected = decode_fp16_protocol(q, k, v, bt, torch.tensor(lens, dtype=torch.int32))
    qw = torch.zeros(2, 12, 256, dtype=torch.float16, device="cuda")
    qw[:, :, 64:192] = q.half().cuda()
    kw = torch.zeros(n, 16, 3, 136, dtype=torch.float16, device="cuda")
    vw = torch.zeros(n, 16, 3, 136, dtype=torch.float16, device="cuda")
    kw[:, :, :2, :128] = k.half().cuda()
    vw[:, :, :2, :128] = v.half().cuda()
    out = pad.paged_attention_decode_ex(qw[:, :, 64:192], kw[:, :, :2, :128], vw[:, :, :2, :128], bt.cuda(),
                                        torch.tensor(lens, dtype=torch.int32).cuda(), engine=engine)
    assert_parity(out, expected)


def test_runs_on_current_stream():
    import paged_attention_decode_amd as pad

    lens = [500, 1000]
    bt, n = shuffled_table(lens, 16, spare_pages=1, extra_cols=0, seed=51)
    k, v = make_cache(n, 16, 2, 128, seed=51)
    q = torch.randn(2, 12, 128, generator=torch.Generator().manual_seed(51))
    expected = decode_fp16_protocol(q, k, v, bt, torch.tensor(lens, dtype=torch.int32))
    args = [q.half().cuda(), k.half().cuda(), v.half().cuda(), bt.cuda(), torch.tensor(lens, dtype=torch.int32).cuda()]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        outs = [pad.paged_attention_decode(*args) for _ in range(3)]
    s.synchronize()
    for o in outs:
        assert_parity(o, expected)


def test_concurrent_streams_keep_their_own_scratch():
    # Two streams decode different batches at the same time; the binding
    # keeps split scratch (partials and arrival counters) per stream, so the
    # interleaved launches must not disturb each other.
    import paged_attention_decode_amd as pad

    cases = []
    for lens, seed in (([4096, 4096, 3000], 81), ([2500, 17, 4096, 900, 1], 82)):
        bt, n = shuffled_table(lens, 16, spare_pages=1, extra_cols=0, seed=seed)
        k, v = make_cache(n, 16, 2, 128, seed=seed)
        q = torch.randn(len(lens), 12, 128, generator=torch.Generator().manual_seed(seed))
        sl = torch.tensor(lens, dtype=torch.int32)
        cases.append(([q.half().cuda(), k.half().cuda(), v.half().cuda(), bt.cuda(), sl.cuda()],
                      decode_fp16_protocol(q, k, v, bt, sl)))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[], []]
    for _ in range(20):
        for i, st in enumerate(streams):
            with torch.cuda.stream(st):
                outs[i].append(pad.paged_attention_decode(*cases[i][0]))
    for st in streams:
        st.synchronize()
    for i in range(2):
        assert_parity(outs[i][0], cases[i][1])
        for o in outs[i][1:]:
            assert torch.equal(o, outs[i][0])


@pytest.mark.parametrize("case", ["ragged", "two_level"])
def test_graph_capture_replays(case):
    # Serving engines capture the decode in a HIP graph and replay it with
    # new inputs written in place.  The launch allocates nothing once its
    # stream's scratch exists, the split merge leaves its arrival (and group)
    # counters at zero, and the workspace carries no state, so every replay
    # must equal an eager call on the same inputs - with eager decodes (other
    # scratch) run between the replays.  "two_level": a long single-kv-head
    # row whose ~250 planned items merge in two levels.
    import paged_attention_decode_amd as pad

    lens, hq, hkv = ([4096, 300, 2500, 1], 12, 2) if case == "ragged" else ([60000, 16], 8, 1)
    bt, n = shuffled_table(lens, 16, spare_pages=1, extra_cols=1, seed=91)
    k, v = make_cache(n, 16, hkv, 128, seed=91)
    dev = [k.half().cuda(), v.half().cuda(), bt.cuda(), torch.tensor(lens, dtype=torch.int32).cuda()]
    qs = [torch.randn(len(lens), hq, 128, generator=torch.Generator().manual_seed(92 + i)).half().cuda()
          for i in range(4)]
    q_static = qs[0].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):  # allocates this stream's scratch before capture
            pad.paged_attention_decode(q_static, *dev)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out_static = pad.paged_attention_decode(q_static, *dev)
    torch.cuda.synchronize()
    for rep in range(3):
        for q in qs:
            q_static.copy_(q)
            graph.replay()
            torch.cuda.synchronize()
            eager = pad.paged_attention_decode(q, *dev)
            torch.cuda.synchronize()
            assert torch.equal(out_static, eager), f"replay {rep} differs from the eager call"
    assert_parity(out_static, decode_fp16_protocol(qs[-1].float().cpu(), k, v, bt,
                                                   torch.tensor(lens, dtype=torch.int32)))


# The refused capture ends with nothing recorded; torch warns that its graph is empty.
@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_graph_replay_survives_scratch_growth_and_capture_refuses_growth():
    # A graph captured with the stream's small scratch keeps that address.
    # A later, larger eager call on the same stream grows the scratch; the
    # replaced buffer must stay alive (not go back to the caching allocator),
    # so replays still write their partials and counters somewhere private.
    # Growing during capture itself is refused with a clear error.
    import paged_attention_decode_amd as pad

    def case(lens, seed):
        bt, n = shuffled_table(lens, 16, spare_pages=1, extra_cols=0, seed=seed)
        k, v = make_cache(n, 16, 2, 128, seed=seed)
        q = torch.randn(len(lens), 12, 128, generator=torch.Generator().manual_seed(seed))
        sl = torch.tensor(lens, dtype=torch.int32)
        return [q.half().cuda(), k.half().cuda(), v.half().cuda(), bt.cuda(), sl.cuda()], (q, k, v, bt, sl)

    small, small_cpu = case([700, 1500], 301)
    big, big_cpu = case([4096] * 48, 302)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pad.paged_attention_decode(*small)  # sizes this stream's scratch for the small shape only
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out_static = pad.paged_attention_decode(*small)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        big_out = pad.paged_attention_decode(*big)  # grows the scratch of stream s
        # Allocations that could reuse the replaced scratch, written with a pattern.
        fillers = [torch.full((1 << 18,), 7.0, device="cuda") for _ in range(16)]
    torch.cuda.synchronize()
    expected_small = decode_fp16_protocol(*small_cpu)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert_parity(out_static, expected_small)
        assert all(bool((f == 7.0).all()) for f in fillers), "a replay wrote into memory it no longer owns"
    assert_parity(big_out, decode_fp16_protocol(*big_cpu))
    # Capturing a call whose scratch would have to grow raises.
    fresh = torch.cuda.Stream()
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="graph capture"):
        with torch.cuda.graph(g2, stream=fresh):
            pad.paged_attention_decode(*small)
    torch.cuda.synchronize()


def test_mixed_call_shapes_share_scratch():
    # Calls of different shapes reuse the binding's per-stream scratch: a call
    # with few long sequences (many partials) followed by calls with many
    # sequences (many arrival counters) must each stay correct.
    import paged_attention_decode_amd as pad

    cases = []
    # ... and so do oversubscribed grids (at least one (sequence, kv head)
    # unit per CU): a full batch (one item per unit) and a ragged one.
    ragged = [random.Random(75).randint(0, 1200) for _ in range(150)]
    for lens, seed in (([4000, 3000], 71), ([300] * 100, 72), ([1500] * 7, 73), ([64] * 300, 74),
                       ([1200] * 150, 75), (ragged, 76)):
        bt, n = shuffled_table(lens, 16, spare_pages=1, extra_cols=0, seed=seed)
        k, v = make_cache(n, 16, 2, 128, seed=seed)
        q = torch.randn(len(lens), 12, 128, generator=torch.Generator().manual_seed(seed))
        sl = torch.tensor(lens, dtype=torch.int32)
        dev = [q.half().cuda(), k.half().cuda(), v.half().cuda(), bt.cuda(), sl.cuda()]
        cases.append((dev, decode_fp16_protocol(q, k, v, bt, sl)))
    for _ in range(2):
        for dev, expected in cases + cases[::-1]:
            for s in (None, 5):
                assert_parity(pad.paged_attention_decode(*dev, num_splits=s), expected)


@pytest.mark.parametrize("engine", ENGINES)
@pytest.mark.parametrize("num_splits", [None, 7, 64])
def test_repeated_calls_are_bit_identical(engine, num_splits):
    # The fused split merge runs in the last workgroup to arrive, in a fixed
    # split order, so every call must give the same bits; a lost or doubled
    # arrival count (or a counter left non-zero) would break this.
    import paged_attention_decode_amd as pad

    lens = [4096, 33, 2500, 1, 777, 4000]
    bt, n = shuffled_table(lens, 16, spare_pages=2, extra_cols=1, seed=61)
    k, v = make_cache(n, 16, 2, 128, seed=61)
    q = torch.randn(len(lens), 12, 128, generator=torch.Generator().manual_seed(61))
    args = [q.half().cuda(), k.half().cuda(), v.half().cuda(), bt.cuda(), torch.tensor(lens, dtype=torch.int32).cuda()]
    first = pad.paged_attention_decode_ex(*args, num_splits=num_splits, engine=engine)
    outs = [pad.paged_attention_decode_ex(*args, num_splits=num_splits, engine=engine) for _ in range(60)]
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o, first)
    assert_parity(first, decode_fp16_protocol(q, k, v, bt, torch.tensor(lens, dtype=torch.int32)))


@pytest.mark.parametrize("engine", ENGINES)
@pytest.mark.parametrize("seed", range(FUZZ))
def test_fuzz_shape_matrix(engine, seed):
    q, k, v, bt, sl = random_case(seed, gqa=(1, 2, 4, 6, 8), head_dims=(32, 64, 128), page_sizes=(1, 8, 16, 32),
                                  min_len=0, max_len=300)
    if not _engine_ok(engine, q.shape[1] // k.shape[2], q.shape[2]):
        pytest.skip("shape outside the VALU engine")
    for s in (None, 4):
        _check(q, k, v, bt, sl, engine, s)


@pytest.mark.parametrize("seed", range(FUZZ))
def test_fuzz_wide_matrix(seed):
    # MFMA engine over every head_dim, group sizes up to 16 and every block
    # mode (sub-page 1/2/4/8, uniform 16/32, generic 3/12/24), with the
    # heuristic plan, a fixed split and 60 splits (two-level merge once a
    # row has more than 48 pages).
    q, k, v, bt, sl = random_case(1000 + seed, kv_heads=(1, 2, 4), gqa=(1, 3, 8, 16),
                                  head_dims=(32, 64, 96, 128, 256),
                                  page_sizes=(1, 2, 3, 4, 8, 12, 16, 24, 32), min_len=0, max_len=400)
    for s in (None, 4, 60):
        _check(q, k, v, bt, sl, 0, s)


@pytest.mark.parametrize("seed", range(max(FUZZ // 4, 1)))
def test_fuzz_large_batches(seed):
    # Batches of 40-300 ragged rows (empty ones included) with the heuristic
    # plan: the in-kernel planner for up to 256 rows (an oversubscribed grid
    # once there are at least as many (row, kv head) units as CUs), the static
    # split beyond.
    rng = random.Random(7000 + seed)
    batch = rng.randint(40, 300)
    hkv = rng.choice((2, 4, 8))
    group = rng.choice((1, 4, 8))
    d = rng.choice((64, 128))
    ps = rng.choice((1, 12, 16))
    lens = [rng.randint(0, 600) for _ in range(batch)]
    bt, n = shuffled_table(lens, ps, spare_pages=2, extra_cols=rng.randint(0, 3), seed=7100 + seed)
    k, v = make_cache(n, ps, hkv, d, seed=7200 + seed)
    q = torch.randn(batch, hkv * group, d, generator=torch.Generator().manual_seed(7300 + seed))
    _check(q, k, v, bt, torch.tensor(lens, dtype=torch.int32), 0, None)

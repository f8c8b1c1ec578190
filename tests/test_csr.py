"""CSR page-index input and the in-kernel work planner.

CPU: the oracle's dense -> CSR conversion (a restatement of
src/flashinfer_adapter.py:40-65) against hand-computed answers and round
trips, and the product's vectorised ``paged_kv_indices`` against it.

GPU: ``paged_attention_decode_csr`` against the fp32 oracle on the cases of
the reference's tests/test_flashinfer_adapter.py (primary shape :34-58, page
boundary remainder :61-75 and exact multiple :78-94, GQA ratios :97-109,
ragged batch :112-136), plus CSR-only layouts (pages shared between
sequences, indices out of table order), and ragged batches that exercise
the planner (sequences shorter than the table, empty sequences, batches
past the planner's 256-sequence limit).
"""

from __future__ import annotations

import random

import pytest
import torch

from oracle.csr import csr_to_dense, paged_kv_indices as ref_indices
from oracle.reference import decode_fp16_protocol
from tests.helpers import assert_parity, cdiv, contiguous_table, make_cache, random_case, shuffled_table


# ---------------------------------------------------------------- CPU pins
def test_known_answer_remainder_multiple_and_empty():
    # page_size 4: lengths 5 (remainder), 4 (exact multiple), 1, 0 (empty).
    bt = torch.tensor([[7, 3, 9], [2, 8, 1], [5, 6, 0], [4, 4, 4]], dtype=torch.int32)
    sl = torch.tensor([5, 4, 1, 0], dtype=torch.int32)
    indptr, indices, last = ref_indices(bt, sl, 4)
    assert indptr.tolist() == [0, 2, 3, 4, 4]
    assert indices.tolist() == [7, 3, 2, 5]
    # exact multiple -> page_size, not 0; empty -> 0 - (-1) * 4 = 4
    assert last.tolist() == [1, 4, 1, 4]


def _ragged(seed, batch=6, ps=8, max_len=90):
    rng = random.Random(seed)
    lens = [rng.randint(0, max_len) for _ in range(batch)]
    lens[0] = 0
    lens[1] = ps * 3  # exact multiple
    bt, _ = shuffled_table(lens, ps, spare_pages=3, extra_cols=2, seed=seed)
    return bt, torch.tensor(lens, dtype=torch.int32), ps


@pytest.mark.parametrize("seed", range(5))
def test_round_trip_and_length_identity(seed):
    bt, sl, ps = _ragged(seed)
    indptr, indices, last = ref_indices(bt, sl, ps)
    assert int(indptr[-1]) == indices.numel()
    for b in range(sl.numel()):
        pages = int(indptr[b + 1] - indptr[b])
        assert pages == cdiv(int(sl[b]), ps)
        if pages:
            assert (pages - 1) * ps + int(last[b]) == int(sl[b])
            assert 1 <= int(last[b]) <= ps
    bt2, sl2 = csr_to_dense(indptr, indices, last, ps)
    assert sl2.tolist() == sl.tolist()
    for b in range(sl.numel()):
        n = cdiv(int(sl[b]), ps)
        assert bt2[b, :n].tolist() == bt[b, :n].tolist()


@pytest.mark.parametrize("seed", range(5))
def test_product_conversion_matches_oracle(seed):
    from paged_attention_decode_amd import paged_kv_indices

    bt, sl, ps = _ragged(seed)
    got = paged_kv_indices(bt, sl, ps)
    want = ref_indices(bt, sl, ps)
    for g, w in zip(got, want):
        assert g.dtype == torch.int32
        assert g.tolist() == w.tolist()


# ---------------------------------------------------------------- GPU parity
def _run_csr(q, k, v, indptr, indices, last, **kw):
    import paged_attention_decode_amd as pad

    dev = "cuda"
    return pad.paged_attention_decode_csr(q.half().to(dev), k.half().to(dev), v.half().to(dev), indptr.to(dev),
                                          indices.to(dev), last.to(dev), **kw)


def _check_csr(q, k, v, bt, sl, ps, num_splits=None, scale=None):
    indptr, indices, last = ref_indices(bt, sl, ps)
    expected = decode_fp16_protocol(q, k, v, bt, sl, scale)
    actual = _run_csr(q, k, v, indptr, indices, last, num_splits=num_splits, scale=scale)
    assert actual.dtype == torch.float16 and actual.shape == q.shape
    assert_parity(actual, expected)
    return actual


def _primary_case(lens, ps=16, hkv=2, group=6, d=128, seed=0):
    bt, total = contiguous_table(lens, ps)
    k, v = make_cache(total + 3, ps, hkv, d, seed)
    g = torch.Generator().manual_seed(seed + 1)
    q = torch.randn(len(lens), hkv * group, d, generator=g)
    return q, k, v, bt, torch.tensor(lens, dtype=torch.int32)


@pytest.mark.gpu
@pytest.mark.parametrize("num_splits", [None, 1, 8])
def test_csr_primary_target_shape(num_splits):
    q, k, v, bt, sl = _primary_case([1, 17, 256, 4000])
    _check_csr(q, k, v, bt, sl, 16, num_splits=num_splits)


@pytest.mark.gpu
@pytest.mark.parametrize("seq_len", [100, 96])
def test_csr_page_boundaries(seq_len):
    q, k, v, bt, sl = _primary_case([seq_len], seed=seq_len)
    _check_csr(q, k, v, bt, sl, 16)


@pytest.mark.gpu
@pytest.mark.parametrize("group", [1, 4, 6, 8])
def test_csr_gqa_ratios(group):
    q, k, v, bt, sl = _primary_case([200], group=group, seed=100 + group)
    _check_csr(q, k, v, bt, sl, 16)


@pytest.mark.gpu
def test_csr_ragged_batch():
    q, k, v, bt, sl = _primary_case([3, 17, 100, 512], seed=43)
    _check_csr(q, k, v, bt, sl, 16)


@pytest.mark.gpu
@pytest.mark.parametrize("num_splits", [None, 100])
def test_csr_two_level_merge(num_splits):
    # A long single-kv-head row read through the CSR index: the planner (or
    # 100 explicit splits) gives it more than 48 items, merged in two levels.
    q, k, v, bt, sl = _primary_case([40000, 33, 1], hkv=1, group=8, seed=61)
    _check_csr(q, k, v, bt, sl, 16, num_splits=num_splits)


@pytest.mark.gpu
@pytest.mark.parametrize("ps", [1, 8, 16, 32])
def test_csr_shared_and_reordered_pages(ps):
    """CSR rows may share physical pages and list them in any order."""
    rng = random.Random(ps)
    lens = [rng.randint(1, 300) for _ in range(5)] + [0]
    hkv, group, d = 2, 4, 64
    num_pages = 40
    k, v = make_cache(num_pages, ps, hkv, d, seed=ps)
    indptr, indices, last = [0], [], []
    for n in lens:
        pages = cdiv(n, ps)
        indices += [rng.randrange(num_pages) for _ in range(pages)]
        indptr.append(indptr[-1] + pages)
        last.append(n - (pages - 1) * ps if pages else 0)
    indptr, indices, last = (torch.tensor(x, dtype=torch.int32) for x in (indptr, indices, last))
    bt, sl = csr_to_dense(indptr, indices, last, ps)
    assert sl.tolist() == lens
    g = torch.Generator().manual_seed(ps + 5)
    q = torch.randn(len(lens), hkv * group, d, generator=g)
    expected = decode_fp16_protocol(q, k, v, bt, sl)
    for splits in (None, 1, 4):
        assert_parity(_run_csr(q, k, v, indptr, indices, last, num_splits=splits), expected)


@pytest.mark.gpu
def test_csr_matches_dense_on_c3_like_batch():
    """Ragged C3-like batch (page 32, lengths 1..8192): CSR and dense agree."""
    import paged_attention_decode_amd as pad

    rng = random.Random(3)
    lens = [rng.randint(1, 8192) for _ in range(32)]
    lens[0] = 1
    ps, hkv, group, d = 32, 2, 6, 128
    bt, num_pages = shuffled_table(lens, ps, spare_pages=4, extra_cols=0, seed=3)
    k, v = make_cache(num_pages, ps, hkv, d, seed=3)
    q = torch.randn(len(lens), hkv * group, d, generator=torch.Generator().manual_seed(4))
    sl = torch.tensor(lens, dtype=torch.int32)
    rows = [0, 1, 7, 31]
    expected = decode_fp16_protocol(q[rows], k, v, bt[rows], sl[rows])
    dev = "cuda"
    dense = pad.paged_attention_decode(q.half().to(dev), k.half().to(dev), v.half().to(dev), bt.to(dev), sl.to(dev))
    indptr, indices, last = pad.paged_kv_indices(bt.to(dev), sl.to(dev), ps)
    csr = pad.paged_attention_decode_csr(q.half().to(dev), k.half().to(dev), v.half().to(dev), indptr, indices, last)
    assert_parity(dense[rows], expected)
    assert_parity(csr[rows], expected)
    torch.testing.assert_close(csr.float(), dense.float(), rtol=1e-3, atol=1e-3)


@pytest.mark.gpu
def test_csr_large_batch_single_pass():
    """Past the planner's batch limit the CSR path runs one workgroup per sequence."""
    rng = random.Random(9)
    lens = [rng.randint(0, 70) for _ in range(300)]
    ps, hkv, group, d = 16, 1, 2, 32
    bt, num_pages = shuffled_table(lens, ps, spare_pages=2, extra_cols=0, seed=9)
    k, v = make_cache(num_pages, ps, hkv, d, seed=9)
    q = torch.randn(len(lens), hkv * group, d, generator=torch.Generator().manual_seed(10))
    sl = torch.tensor(lens, dtype=torch.int32)
    _check_csr(q, k, v, bt, sl, ps)
    _check_csr(q, k, v, bt, sl, ps, num_splits=3)


# ------------------------------------------------------- in-kernel planner
def _dense(lens, ps=16, hkv=2, group=6, d=128, extra_cols=0, seed=0):
    bt, num_pages = shuffled_table(lens, ps, spare_pages=3, extra_cols=extra_cols, seed=seed)
    k, v = make_cache(num_pages, ps, hkv, d, seed)
    q = torch.randn(len(lens), hkv * group, d, generator=torch.Generator().manual_seed(seed + 1))
    return q, k, v, bt, torch.tensor(lens, dtype=torch.int32)


def _run_dense(q, k, v, bt, sl, **kw):
    import paged_attention_decode_amd as pad

    dev = "cuda"
    return pad.paged_attention_decode(q.half().to(dev), k.half().to(dev), v.half().to(dev), bt.to(dev), sl.to(dev),
                                      **kw)


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["short_of_capacity", "ragged", "mostly_empty", "all_empty", "one_long"])
def test_planner_layouts(case):
    """Heuristic launches re-plan the grid over the pages in use; results match the oracle."""
    if case == "short_of_capacity":  # table sized for 4096 tokens, sequences of 700
        lens, extra = [700] * 8, 212
    elif case == "ragged":
        rng = random.Random(11)
        lens, extra = [rng.randint(1, 3000) for _ in range(12)], 0
    elif case == "mostly_empty":
        lens, extra = [0, 0, 2500, 0, 1, 0], 0
    elif case == "all_empty":
        lens, extra = [0, 0, 0], 8
    else:  # one sequence much longer than the rest
        lens, extra = [8000, 3, 40, 17], 0
    q, k, v, bt, sl = _dense(lens, extra_cols=extra, seed=len(case))
    expected = decode_fp16_protocol(q, k, v, bt, sl)
    planned = _run_dense(q, k, v, bt, sl)
    assert_parity(planned, expected)
    single = _run_dense(q, k, v, bt, sl, num_splits=1)
    torch.testing.assert_close(planned.float(), single.float(), rtol=1e-3, atol=1e-3)
    if case == "all_empty":
        assert torch.all(planned == 0)


@pytest.mark.gpu
@pytest.mark.parametrize("batch", [64, 256, 257])
def test_planner_batch_limit(batch):
    """The planner handles up to 256 sequences; larger batches keep the static split."""
    rng = random.Random(batch)
    lens = [rng.randint(0, 200) for _ in range(batch)]
    q, k, v, bt, sl = _dense(lens, ps=16, hkv=1, group=4, d=64, extra_cols=1, seed=batch)
    rows = [0, 1, batch // 2, batch - 1]
    expected = decode_fp16_protocol(q[rows], k, v, bt[rows], sl[rows])
    out = _run_dense(q, k, v, bt, sl)
    assert_parity(out[rows], expected)


@pytest.mark.gpu
def test_planner_repeatable():
    """Planned launches are bit-identical call to call (the fused merge is race-free)."""
    rng = random.Random(21)
    lens = [rng.randint(1, 4000) for _ in range(10)]
    q, k, v, bt, sl = _dense(lens, seed=21)
    first = _run_dense(q, k, v, bt, sl)
    for _ in range(20):
        assert torch.equal(_run_dense(q, k, v, bt, sl), first)


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["uniform_full", "full_partial_last_page", "ragged", "ragged_csr"])
def test_oversubscribed_grid(case):
    """At least one (sequence, kv head) unit per CU: the launch sizes the grid for 4 items per unit.

    With every sequence at full capacity the kernel gives each unit one item
    (written straight to the output) and the other workgroups exit; with
    ragged lengths it plans equal page chunks over the whole grid.
    """
    import paged_attention_decode_amd as pad

    batch, ps, hkv, group, d, width = 64, 16, 4, 2, 64, 64
    assert pad.plan(batch, hkv * group, hkv, d, ps, width)["num_splits"] == 4
    rng = random.Random(len(case))
    if case == "uniform_full":
        lens = [width * ps] * batch
    elif case == "full_partial_last_page":  # every table row in use, last pages partly filled
        lens = [width * ps - rng.randint(0, ps - 1) for _ in range(batch)]
    else:
        lens = [rng.randint(0, width * ps) for _ in range(batch)]
        lens[3], lens[10], lens[11] = 0, width * ps, 1
    bt, num_pages = shuffled_table(lens, ps, spare_pages=3, extra_cols=width - max(cdiv(n, ps) for n in lens),
                                   seed=len(case))
    assert bt.shape[1] == width
    k, v = make_cache(num_pages, ps, hkv, d, seed=len(case))
    q = torch.randn(batch, hkv * group, d, generator=torch.Generator().manual_seed(3))
    sl = torch.tensor(lens, dtype=torch.int32)
    expected = decode_fp16_protocol(q, k, v, bt, sl)
    if case == "ragged_csr":
        _check_csr(q, k, v, bt, sl, ps)
        return
    out = _run_dense(q, k, v, bt, sl)
    assert_parity(out, expected)
    single = _run_dense(q, k, v, bt, sl, num_splits=1)
    torch.testing.assert_close(out.float(), single.float(), rtol=1e-3, atol=1e-3)
    for _ in range(5):
        assert torch.equal(_run_dense(q, k, v, bt, sl), out)


@pytest.mark.gpu
@pytest.mark.parametrize("ps", [1, 2, 4, 8, 3, 5, 12, 24, 48])
def test_subpage_blocks_ragged_planned(ps):
    """Page sizes that are not multiples of 16: a 16-token block spans several pages whose ids are read
    ahead into registers (16 / page_size pages for page sizes dividing 16; up to 6 pages at any
    offset for the others, 3 and up).

    Ragged lengths (partial last blocks and pages, an empty row, one row of a
    single token) on shuffled pages, through the planner, a static split and
    the CSR entry.
    """
    rng = random.Random(100 + ps)
    lens = [rng.randint(1, 3000) for _ in range(10)] + [0, 1, 16 * 40 + 3]
    q, k, v, bt, sl = _dense(lens, ps=ps, hkv=2, group=4, d=128, extra_cols=2, seed=100 + ps)
    expected = decode_fp16_protocol(q, k, v, bt, sl)
    assert_parity(_run_dense(q, k, v, bt, sl), expected)
    assert_parity(_run_dense(q, k, v, bt, sl, num_splits=5), expected)
    _check_csr(q, k, v, bt, sl, ps)


@pytest.mark.gpu
@pytest.mark.parametrize("d", [32, 96])
@pytest.mark.parametrize("case", ["static_full", "oversubscribed_full", "ragged", "explicit_splits"])
def test_head_pair_placement(d, case):
    """Rows that are not a multiple of 128 bytes (head_dim 32, 96): kv heads 2m and 2m+1 share a
    cache line per token slot, so the kernel places their workgroups 8 apart (same XCD); the
    placement is a bijection of the grid, so every path must still match the oracle."""
    ps, hkv, group = 16, 8, 2
    if case == "oversubscribed_full":
        lens = [512] * 32              # 256 (sequence, kv head) units: one per CU or more
    elif case == "ragged":
        rng = random.Random(d)
        lens = [rng.randint(1, 1500) for _ in range(8)]
    else:
        lens = [1024] * 8
    q, k, v, bt, sl = _dense(lens, ps=ps, hkv=hkv, group=group, d=d, seed=d + len(case))
    expected = decode_fp16_protocol(q, k, v, bt, sl)
    splits = 3 if case == "explicit_splits" else None
    out = _run_dense(q, k, v, bt, sl, num_splits=splits)
    assert_parity(out, expected)
    for _ in range(3):
        assert torch.equal(_run_dense(q, k, v, bt, sl, num_splits=splits), out)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(int(__import__("os").environ.get("PAD_KERNEL_FUZZ_ITERS", "20"))))
def test_csr_fuzz_wide(seed):
    # The CSR entry over random ragged batches (empty rows included), every
    # block mode and head_dim, heuristic and explicit split counts.
    q, k, v, bt, sl = random_case(5000 + seed, kv_heads=(1, 2, 4), gqa=(1, 2, 5, 8, 16),
                                  head_dims=(32, 64, 96, 128, 256),
                                  page_sizes=(1, 2, 3, 4, 8, 12, 16, 24, 32), max_batch=6, min_len=0, max_len=700)
    ps = k.shape[1]
    for s in (None, 7, 100):
        _check_csr(q, k, v, bt, sl, ps, num_splits=s)


@pytest.mark.gpu
@pytest.mark.parametrize("num_splits", [None, 1, 4])
def test_csr_index_without_pages_gives_zeros(num_splits):
    # Every sequence empty: indptr all zero and no entries in indices (its
    # data pointer may be NULL); the oracle gives zeros.
    k, v = make_cache(2, 16, 2, 128, seed=7)
    q = torch.randn(3, 12, 128, generator=torch.Generator().manual_seed(7))
    indptr = torch.zeros(4, dtype=torch.int32)
    indices = torch.zeros(0, dtype=torch.int32)
    last = torch.full((3,), 16, dtype=torch.int32)
    out = _run_csr(q, k, v, indptr, indices, last, num_splits=num_splits)
    assert out.shape == q.shape and torch.all(out == 0)

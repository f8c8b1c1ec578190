"""Pins for the CPU oracle (oracle/reference.py, oracle/brute.py).

Mirrors the reference's oracle tests - tests/test_reference.py:7-36 (SDPA
without paging), tests/test_reference_edge_cases.py:21-160 and
tests/test_reference_fuzz.py:23-30 - against this build's own restatement,
plus closed-form known answers and invariants chosen so that a dropped
term, a wrong index or a transposed operand fails at least one of them.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.brute import decode_f64
from oracle.reference import paged_attention_decode_reference as ref
from tests.helpers import cdiv, contiguous_table, make_cache, random_case, sdpa_check, shuffled_table

FUZZ = int(os.environ.get("PAD_ORACLE_FUZZ_ITERS", "50"))


def _vs_sdpa(q, k, v, bt, sl, tol=1e-4):
    out = ref(q, k, v, bt, sl)
    torch.testing.assert_close(out, sdpa_check(q, k, v, bt, sl), rtol=tol, atol=tol)
    return out


def test_matches_sdpa_without_paging():
    # tests/test_reference.py:7-36: contiguous pages, no ragged batch.
    g = torch.Generator().manual_seed(0)
    batch, seq, ps, hq, hkv, d = 2, 8, 4, 4, 2, 16
    q = torch.randn(batch, hq, d, generator=g)
    kt = torch.randn(batch, seq, hkv, d, generator=g)
    vt = torch.randn(batch, seq, hkv, d, generator=g)
    k = kt.reshape(batch * seq // ps, ps, hkv, d)
    v = vt.reshape(batch * seq // ps, ps, hkv, d)
    bt = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32)
    sl = torch.full((batch,), seq, dtype=torch.int32)
    got = ref(q, k, v, bt, sl)
    ke = kt.repeat_interleave(hq // hkv, dim=2).transpose(1, 2).contiguous()
    ve = vt.repeat_interleave(hq // hkv, dim=2).transpose(1, 2).contiguous()
    want = F.scaled_dot_product_attention(q.unsqueeze(2), ke, ve).squeeze(2)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def test_partial_last_page():
    seq, ps = 100, 16
    k, v = make_cache(cdiv(seq, ps), ps, 2, 32, seed=0)
    q = torch.randn(1, 12, 32, generator=torch.Generator().manual_seed(1))
    _vs_sdpa(q, k, v, torch.arange(cdiv(seq, ps), dtype=torch.int32)[None], torch.tensor([seq], dtype=torch.int32))



def test_seq_len_one_equals_first_value_row():
    # Closed form: one token -> softmax weight 1 -> out = V[token 0] for every head of the group.
    k, v = make_cache(3, 16, 2, 32, seed=1)
    q = torch.randn(1, 8, 32, generator=torch.Generator().manual_seed(2))
    bt = torch.tensor([[2, 0]], dtype=torch.int32)
    out = _vs_sdpa(q, k, v, bt, torch.tensor([1], dtype=torch.int32))
    for h in range(8):
        torch.testing.assert_close(out[0, h], v[2, 0, h // 4], rtol=0, atol=1e-6)


def test_exactly_one_full_page():
    k, v = make_cache(1, 16, 2, 32, seed=2)
    q = torch.randn(1, 12, 32, generator=torch.Generator().manual_seed(3))
    _vs_sdpa(q, k, v, torch.zeros(1, 1, dtype=torch.int32), torch.tensor([16], dtype=torch.int32))


def test_shuffled_table_with_poisoned_holes():
    # tests/test_reference_edge_cases.py:60-79: unused columns/pages hold other data.
    k, v = make_cache(10, 16, 2, 32, seed=3)
    q = torch.randn(1, 12, 32, generator=torch.Generator().manual_seed(4))
    bt = torch.tensor([[7, 2, 9, 5, 5, 5]], dtype=torch.int32)
    out = _vs_sdpa(q, k, v, bt, torch.tensor([48], dtype=torch.int32))
    # Changing anything outside the 3 referenced pages must not change the output.
    k2, v2 = k.clone(), v.clone()
    for p in (0, 1, 3, 4, 5, 6, 8):
        k2[p] = 1e3
        v2[p] = -1e3
    torch.testing.assert_close(ref(q, k2, v2, bt, torch.tensor([48], dtype=torch.int32)), out, rtol=0, atol=0)


@pytest.mark.parametrize("group", [1, 4, 6, 8])
def test_gqa_ratios(group):
    k, v = make_cache(3, 16, 2, 32, seed=100 + group)
    q = torch.randn(1, 2 * group, 32, generator=torch.Generator().manual_seed(group))
    _vs_sdpa(q, k, v, torch.arange(3, dtype=torch.int32)[None], torch.tensor([40], dtype=torch.int32))


def test_gqa_equals_mha_with_repeated_kv_heads():
    # Invariant: GQA with group r == MHA over KV heads repeated r times.
    group, hkv, d, ps = 3, 2, 32, 8
    k, v = make_cache(5, ps, hkv, d, seed=5)
    q = torch.randn(2, hkv * group, d, generator=torch.Generator().manual_seed(6))
    bt = torch.tensor([[4, 1, 3], [0, 2, 2]], dtype=torch.int32)
    sl = torch.tensor([19, 11], dtype=torch.int32)
    gqa_out = ref(q, k, v, bt, sl)
    mha_out = ref(q, k.repeat_interleave(group, dim=2), v.repeat_interleave(group, dim=2), bt, sl)
    torch.testing.assert_close(gqa_out, mha_out, rtol=1e-6, atol=1e-6)


def test_ragged_batch_rows_are_independent():
    # tests/test_reference_edge_cases.py:99-127.
    lens = [3, 8, 17, 64]
    bt, total = contiguous_table(lens, 8)
    k, v = make_cache(total, 8, 2, 32, seed=42)
    q = torch.randn(4, 12, 32, generator=torch.Generator().manual_seed(7))
    sl = torch.tensor(lens, dtype=torch.int32)
    batched = _vs_sdpa(q, k, v, bt, sl)
    for b in range(4):
        solo = ref(q[b:b + 1], k, v, bt[b:b + 1], sl[b:b + 1])
        torch.testing.assert_close(batched[b:b + 1], solo, rtol=1e-5, atol=1e-5)


def test_zero_length_row_gives_zeros():
    k, v = make_cache(4, 16, 2, 32, seed=7)
    q = torch.randn(2, 8, 32, generator=torch.Generator().manual_seed(8))
    bt = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32)
    out = _vs_sdpa(q, k, v, bt, torch.tensor([0, 20], dtype=torch.int32))
    assert torch.all(out[0] == 0.0)


def test_long_sequence():
    seq, ps = 32768, 16
    k, v = make_cache(seq // ps, ps, 2, 128, seed=9)
    q = torch.randn(1, 12, 128, generator=torch.Generator().manual_seed(9))
    _vs_sdpa(q, k, v, torch.arange(seq // ps, dtype=torch.int32)[None], torch.tensor([seq], dtype=torch.int32))


def test_zero_query_gives_mean_of_values():
    # Closed form: q = 0 -> uniform weights -> mean of V over the valid tokens.
    lens = [37]
    bt, n = shuffled_table(lens, 16, spare_pages=3, extra_cols=2, seed=11)
    k, v = make_cache(n, 16, 2, 64, seed=11)
    q = torch.zeros(1, 4, 64)
    out = ref(q, k, v, bt, torch.tensor(lens, dtype=torch.int32))
    toks = torch.cat([v[int(bt[0, j])] for j in range(3)])[:37]  # [37, Hkv, d]
    for h in range(4):
        torch.testing.assert_close(out[0, h], toks[:, h // 2].mean(0), rtol=1e-5, atol=1e-6)


def test_identical_keys_give_mean_of_values():
    k, v = make_cache(2, 16, 1, 32, seed=12)
    k[:] = k[0, 0]
    q = torch.randn(1, 2, 32, generator=torch.Generator().manual_seed(12))
    out = ref(q, k, v, torch.tensor([[1, 0]], dtype=torch.int32), torch.tensor([20], dtype=torch.int32))
    toks = torch.cat([v[1], v[0]])[:20, 0]
    torch.testing.assert_close(out[0, 0], toks.mean(0), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(out[0, 1], toks.mean(0), rtol=1e-5, atol=1e-6)


def test_one_dominant_key_selects_its_value():
    k, v = make_cache(2, 16, 1, 32, seed=13)
    q = torch.randn(1, 1, 32, generator=torch.Generator().manual_seed(13))
    k[0, 5, 0] = q[0, 0] * 50.0  # token 5 of logical page 0 dominates
    out = ref(q, k, v, torch.tensor([[0, 1]], dtype=torch.int32), torch.tensor([30], dtype=torch.int32))
    torch.testing.assert_close(out[0, 0], v[0, 5, 0], rtol=0, atol=1e-5)


def test_page_relabelling_invariance():
    # Permuting the physical pages (and the table with them) changes nothing.
    lens = [50, 7]
    bt, n = shuffled_table(lens, 8, spare_pages=2, extra_cols=1, seed=14)
    k, v = make_cache(n, 8, 2, 32, seed=14)
    q = torch.randn(2, 4, 32, generator=torch.Generator().manual_seed(14))
    sl = torch.tensor(lens, dtype=torch.int32)
    perm = torch.randperm(n, generator=torch.Generator().manual_seed(15))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(n)
    out1 = ref(q, k, v, bt, sl)
    out2 = ref(q, k[perm], v[perm], inv[bt.long()].to(torch.int32), sl)
    torch.testing.assert_close(out1, out2, rtol=0, atol=0)


def test_scale_argument_and_default():
    k, v = make_cache(2, 16, 2, 64, seed=16)
    q = torch.randn(1, 4, 64, generator=torch.Generator().manual_seed(16))
    bt = torch.tensor([[1, 0]], dtype=torch.int32)
    sl = torch.tensor([25], dtype=torch.int32)
    torch.testing.assert_close(ref(q, k, v, bt, sl), ref(q, k, v, bt, sl, scale=0.125), rtol=0, atol=0)
    torch.testing.assert_close(ref(q, k, v, bt, sl, scale=0.3), sdpa_check(q, k, v, bt, sl, scale=0.3),
                               rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("seed", range(FUZZ))
def test_fuzz_reference_vs_sdpa_and_f64(seed):
    # tests/test_reference_fuzz.py:23-30, plus the float64 brute force.
    q, k, v, bt, sl = random_case(seed, head_dims=(16, 32, 64, 128))
    out = _vs_sdpa(q, k, v, bt, sl)
    f64 = decode_f64(q.numpy(), k.numpy(), v.numpy(), bt.numpy(), sl.numpy())
    np.testing.assert_allclose(out.numpy(), f64, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("seed", range(8))
def test_brute_f64_vs_sdpa_f64(seed):
    # The float64 brute force against SDPA evaluated in float64.
    q, k, v, bt, sl = random_case(1000 + seed, max_len=300)
    want = sdpa_check(q.double(), k.double(), v.double(), bt, sl)
    got = decode_f64(q.numpy(), k.numpy(), v.numpy(), bt.numpy(), sl.numpy())
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-10, atol=1e-12)


def test_row_subset_oracle_matches_full_oracle():
    # decode_rows_fp16_protocol (the C5 subset oracle) relabels the selected
    # rows' pages onto a compact cache.  It must give exactly the rows of the
    # full oracle, here with two sequences sharing physical pages, unused
    # columns pointing at other pages, an empty row, a partial last page and
    # rows asked for out of order.
    from oracle.reference import decode_fp16_protocol, decode_rows_fp16_protocol

    lens = [37, 0, 64, 5, 50, 17]
    ps, hkv, group, d = 16, 2, 3, 32
    bt, num_pages = shuffled_table(lens, ps, spare_pages=3, extra_cols=2, seed=31)
    bt[4, :2] = bt[0, :2]  # sequences 0 and 4 share their first two pages
    k, v = make_cache(num_pages, ps, hkv, d, seed=31)
    q = torch.randn(len(lens), hkv * group, d, generator=torch.Generator().manual_seed(32))
    sl = torch.tensor(lens, dtype=torch.int32)
    full = decode_fp16_protocol(q, k, v, bt, sl)
    for rows in ([4, 0], [1], [5, 2, 3], [0, 1, 2, 3, 4, 5], [3, 3]):
        sub = decode_rows_fp16_protocol(q, k, v, bt, sl, rows)
        assert sub.shape == (len(rows), hkv * group, d)
        assert torch.equal(sub, full[rows]), rows
    # A planted mistake (the relabelled table shifted by one page) is caught.
    bt_bad = bt.clone()
    bt_bad[0, 0] = bt[0, 1]
    assert not torch.allclose(decode_rows_fp16_protocol(q, k, v, bt_bad, sl, [0]), full[[0]], atol=1e-3)

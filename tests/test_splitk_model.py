"""Pins for the float64 split-K model (oracle/splitk.py).

The model restates analysis/split_k_derivation.md of the reference.  Its
checks: split invariance against the unsplit float64 brute force for many
split counts in both split modes (token chunks as in
cuda/kernel_v4_split_k.cu:73-75, page-aligned chunks as in this build),
oversplit (more splits than tokens, tests/test_kernel_cuda_v4.py:114-127),
empty splits in any position of the fold, and planted mistakes: each
plausible bug in the merge (dropped rescale, dropped -inf guard, wrong
split index, l not rescaled) must fail one of these checks.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import splitk
from oracle.brute import decode_f64
from tests.helpers import random_case


def _case(seed, **kw):
    q, k, v, bt, sl = random_case(seed, **kw)
    return q.numpy(), k.numpy(), v.numpy(), bt.numpy(), sl.numpy()


@pytest.mark.parametrize("mode", ["tokens", "pages"])
@pytest.mark.parametrize("num_splits", [1, 2, 3, 4, 8, 16, 64])
def test_split_invariance(mode, num_splits):
    q, k, v, bt, sl = _case(7, min_len=1, max_len=150)
    want = decode_f64(q, k, v, bt, sl)
    got = splitk.decode_splitk_f64(q, k, v, bt, sl, num_splits, mode)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_oversplit_more_splits_than_tokens():
    q, k, v, bt, sl = _case(3, min_len=1, max_len=6)
    bounds = splitk.split_bounds(5, 8, "tokens")
    assert sum(1 for a, e in bounds if e <= a) >= 3  # empty chunks are exercised
    for mode in ("tokens", "pages"):
        np.testing.assert_allclose(splitk.decode_splitk_f64(q, k, v, bt, sl, 8, mode), decode_f64(q, k, v, bt, sl),
                                   rtol=1e-12, atol=1e-12)


def test_empty_split_first_in_fold():
    # The guard must make the fold independent of where empty splits sit.
    rng = np.random.default_rng(0)
    qh, keys, vals = rng.normal(size=16), rng.normal(size=(30, 16)), rng.normal(size=(30, 16))
    parts = [splitk.phase1(qh, keys, vals, 0.25, a, e) for a, e in [(0, 0), (0, 10), (10, 10), (10, 30), (30, 30)]]
    whole = splitk.phase2([splitk.phase1(qh, keys, vals, 0.25, 0, 30)])
    np.testing.assert_allclose(splitk.phase2(parts), whole, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(splitk.phase2(parts[::-1]), whole, rtol=1e-13, atol=1e-13)


def test_all_splits_empty_gives_zeros():
    z = (np.zeros(8), float("-inf"), 0.0)
    assert np.all(splitk.phase2([z, z, z]) == 0.0)


def test_page_mode_bounds_are_page_aligned():
    for n_tok, ps, mp, s in [(100, 16, 7, 3), (4096, 16, 256, 64), (5, 16, 1, 8), (33, 32, 4, 2)]:
        bounds = splitk.split_bounds(n_tok, s, "pages", ps, mp)
        assert bounds[0][0] == 0 and max(e for _, e in bounds) == n_tok
        for a, e in bounds:
            assert a % ps == 0 or a == n_tok
        covered = sorted(t for a, e in bounds for t in range(a, e))
        assert covered == list(range(n_tok))


# --- planted mistakes: each broken merge must be caught by the checks above ---

def _no_alpha(parts):
    d = parts[0][0].shape[0]
    m_run, l_run, acc = float("-inf"), 0.0, np.zeros(d)
    for o_s, m_s, l_s in parts:
        m_new = max(m_run, m_s)
        beta = 0.0 if m_s == float("-inf") else math.exp(m_s - m_new)
        l_run = l_run + l_s * beta  # missing * alpha
        acc = acc + o_s * beta
        m_run = m_new
    return acc / l_run


def _no_guard(parts):
    d = parts[0][0].shape[0]
    m_run, l_run, acc = float("-inf"), 0.0, np.zeros(d)
    for o_s, m_s, l_s in parts:
        m_new = max(m_run, m_s)
        with np.errstate(invalid="ignore"):
            alpha = np.exp(np.float64(m_run - m_new))
            beta = np.exp(np.float64(m_s - m_new))
        l_run = l_run * alpha + l_s * beta
        acc = acc * alpha + o_s * beta
        m_run = m_new
    return acc / l_run


def _l_not_rescaled(parts):
    d = parts[0][0].shape[0]
    m_run, l_run, acc = float("-inf"), 0.0, np.zeros(d)
    for o_s, m_s, l_s in parts:
        m_new = max(m_run, m_s)
        alpha = 0.0 if m_run == float("-inf") else math.exp(m_run - m_new)
        beta = 0.0 if m_s == float("-inf") else math.exp(m_s - m_new)
        l_run = l_run + l_s  # weights ignored for l
        acc = acc * alpha + o_s * beta
        m_run = m_new
    return acc / l_run


def _wrong_index(parts):
    # Uses the previous split's max for the incoming split (off-by-one index).
    shifted = [(parts[i][0], parts[i - 1][1] if i else parts[i][1], parts[i][2]) for i in range(len(parts))]
    return splitk.phase2(shifted)


@pytest.mark.parametrize("broken", [_no_alpha, _no_guard, _l_not_rescaled, _wrong_index])
def test_planted_merge_mistakes_are_caught(broken):
    q, k, v, bt, sl = _case(11, min_len=40, max_len=150)
    want = decode_f64(q, k, v, bt, sl)
    caught = False
    for mode, s in [("tokens", 4), ("tokens", 8), ("pages", 64)]:
        with np.errstate(all="ignore"):
            got = splitk.decode_splitk_f64(q, k, v, bt, sl, s, mode, _phase2=broken)
        if not np.all(np.isfinite(got)) or not np.allclose(got, want, rtol=1e-6, atol=1e-6):
            caught = True
    # The fold with an empty split first (test_empty_split_first_in_fold).
    rng = np.random.default_rng(0)
    qh, keys, vals = rng.normal(size=16), rng.normal(size=(30, 16)), rng.normal(size=(30, 16))
    parts = [splitk.phase1(qh, keys, vals, 0.25, a, e) for a, e in [(0, 0), (0, 10), (10, 10), (10, 30)]]
    whole = splitk.phase2([splitk.phase1(qh, keys, vals, 0.25, 0, 30)])
    with np.errstate(all="ignore"):
        got = broken(parts)
    if not np.all(np.isfinite(got)) or not np.allclose(got, whole, rtol=1e-9, atol=1e-9):
        caught = True
    assert caught, f"{broken.__name__} was not detected"

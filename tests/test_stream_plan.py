"""CPU tests of the stream-item plan (heuristics.stream_items, the restatement of the in-kernel
planner plan_stream in csrc/pa_decode.hip; the GPU tests in test_worklist.py compare the planner
kernel's work lists with it).

Pinned three ways:

* the structure every correct plan has (tests/plan_check.py): each unit's pages covered once in
  order, item slots where the merge looks for them, one owner per empty unit, <= 2 items per
  workgroup;
* a brute force on small inputs that rebuilds the items from (T, W) by walking every virtual page
  one at a time (no floor divisions, no range formulas), and known answers for equal lengths;
* the balance the plan exists for: no workgroup streams more than ceil(W / G) <= T pages, and T
  satisfies W(T) <= G * T.

Planted mistakes in a plan (a shifted page boundary, a wrong slot, a wrong item count, a wrong
entry-0 offset) are caught by the structure check.
"""

from __future__ import annotations

import random

import pytest

from paged_attention_decode_amd import heuristics as H
from tests.plan_check import check_items


def _tuples(plan):
    out = []
    for i1, i2 in plan:
        its = []
        for it in (i1, i2):
            if it is not None:
                its.append((it.b, it.kvh, it.p_begin, it.p_end, it.nsplit, it.slot0, 2, it.odd, it.slot))
        out.append(its)
    return out


def _random_pages(rng, batch, max_pages, zeros=True):
    pages = [rng.randint(0 if zeros else 1, max_pages) for _ in range(batch)]
    if zeros and batch > 2 and rng.random() < 0.5:
        pages[rng.randrange(batch)] = 0
    return pages


def _brute(pages, hkv, grid, t, w):
    """Items rebuilt from (T, W) by walking every virtual page."""
    owner = []  # virtual page -> (unit, page within unit or None for padding)
    for b, p in enumerate(pages):
        for h in range(hkv):
            for j in range(max(p, t)):
                owner.append((b * hkv + h, j if j < p else None))
    assert len(owner) == w
    # range of each virtual page: walk g while g's start <= x
    bounds = []
    for g in range(grid + 1):
        bounds.append(g * w // grid)
    rng_of = []
    g = 0
    for x in range(w):
        while bounds[g + 1] <= x:
            g += 1
        rng_of.append(g)
    items_by_g = [[] for _ in range(grid)]
    # per (g, unit): page span
    spans = {}
    for x in range(w):
        u, j = owner[x]
        g = rng_of[x]
        key = (g, u)
        if key not in spans:
            spans[key] = [None, None, x]
        if j is not None:
            if spans[key][0] is None:
                spans[key][0] = j
            spans[key][1] = j + 1
    first_x = {}
    for x in range(w):
        first_x.setdefault(owner[x][0], x)
    # units' entry ranges
    unit_groups = {}
    for (g, u), (j0, j1, x0) in sorted(spans.items()):
        p = pages[u // hkv]
        if p == 0:
            if x0 == first_x[u]:
                unit_groups.setdefault(u, []).append(g)
        elif j0 is not None:
            unit_groups.setdefault(u, []).append(g)
    for (g, u), (j0, j1, x0) in sorted(spans.items()):
        b, h = divmod(u, hkv)
        p = pages[b]
        gs = unit_groups.get(u, [])
        if g not in gs:
            continue
        second = x0 != bounds[g]  # the unit starts inside range g
        slot = 2 * g + (1 if second else 0)
        if p == 0:
            items_by_g[g].append((b, h, 0, 0, 0, slot, 2, 0, slot))
            continue
        gf = gs[0]
        odd = 1 if first_x[u] != bounds[gf] else 0
        items_by_g[g].append((b, h, j0, j1, len(gs), 2 * gf, 2, odd, slot))
    return items_by_g


@pytest.mark.parametrize("seed", range(40))
def test_mirror_matches_brute_force(seed):
    rng = random.Random(seed)
    hkv = rng.choice([1, 2, 3, 4])
    batch = rng.randint(1, 7)
    pages = _random_pages(rng, batch, rng.choice([5, 20, 60]))
    grid = rng.choice([2, 4, 8]) * batch * hkv
    min_chunk = rng.choice([1, 2])
    span = H.stream_span(pages, hkv, grid, min_chunk)
    plan = H.stream_items(pages, hkv, grid, min_chunk)
    if span is None:
        assert plan is None and sum(pages) * hkv < grid * min_chunk
        return
    t, w = span
    assert _tuples(plan) == _brute(pages, hkv, grid, t, w)


@pytest.mark.parametrize("seed", range(200))
def test_plan_structure_and_balance(seed):
    rng = random.Random(1000 + seed)
    hkv = rng.choice([1, 2, 4, 8])
    batch = rng.choice([1, 2, 3, 8, 32, 64, 100, 256])
    pages = _random_pages(rng, batch, rng.choice([4, 64, 256, 2048]))
    grid = rng.choice([2, 4, 8, 16, 64]) * batch * hkv
    min_chunk = rng.choice([1, 8, 16])
    span = H.stream_span(pages, hkv, grid, min_chunk)
    plan = H.stream_items(pages, hkv, grid, min_chunk)
    up = sum(pages) * hkv
    if span is None:
        assert plan is None and (up < grid * min_chunk or up > H.STREAM_MAX_UNIT_PAGES)
        return
    t, w = span
    assert w == hkv * sum(max(p, t) for p in pages) and w <= grid * t  # no unit fits strictly inside a range
    assert t <= max(-(-up // (grid - batch * hkv)), 1)
    items = _tuples(plan)
    check_items(items, pages, hkv, 2)
    loads = [sum(it[3] - it[2] for it in its) for its in items]
    assert max(loads) <= -(-w // grid) <= t
    assert sum(loads) == up


def test_equal_lengths_known_answer():
    # 2 sequences x 2 kv heads of 64 pages over 8 workgroups: ranges of 32 pages, two per unit.
    plan = H.stream_items([64, 64], 2, 8, 16)
    got = [(i1.b, i1.kvh, i1.p_begin, i1.p_end, i1.nsplit, i1.slot0, i1.odd, i1.slot) for i1, i2 in plan]
    assert all(i2 is None for _, i2 in plan)
    assert got == [(0, 0, 0, 32, 2, 0, 0, 0), (0, 0, 32, 64, 2, 0, 0, 2),
                   (0, 1, 0, 32, 2, 4, 0, 4), (0, 1, 32, 64, 2, 4, 0, 6),
                   (1, 0, 0, 32, 2, 8, 0, 8), (1, 0, 32, 64, 2, 8, 0, 10),
                   (1, 1, 0, 32, 2, 12, 0, 12), (1, 1, 32, 64, 2, 12, 0, 14)]


def test_spanning_known_answer():
    # One kv head, pages 3 and 5 over 2 workgroups (min_chunk 1): T = 4, W = 4 + 5 = 9, ranges [0, 4)
    # and [4, 9).  Workgroup 0: sequence 0's 3 pages (its range ends in sequence 0's padding);
    # workgroup 1: sequence 1's 5 pages, as its item 1 (the range starts where sequence 1 does).
    plan = H.stream_items([3, 5], 1, 2, 1)
    (a1, a2), (b1, b2) = plan
    assert a2 is None and b2 is None
    assert (a1.b, a1.p_begin, a1.p_end, a1.nsplit, a1.slot) == (0, 0, 3, 1, 0)
    assert (b1.b, b1.p_begin, b1.p_end, b1.nsplit, b1.slot) == (1, 0, 5, 1, 2)
    # pages 6 and 6 over 3 workgroups: T = 4, W = 12, ranges of 4: the middle one spans both sequences.
    plan = H.stream_items([6, 6], 1, 3, 1)
    (a1, a2), (b1, b2), (c1, c2) = plan
    assert (a1.b, a1.p_begin, a1.p_end, a1.nsplit, a1.slot0, a1.odd, a1.slot) == (0, 0, 4, 2, 0, 0, 0)
    assert (b1.b, b1.p_begin, b1.p_end, b1.slot) == (0, 4, 6, 2)
    assert (b2.b, b2.p_begin, b2.p_end, b2.nsplit, b2.slot0, b2.odd, b2.slot) == (1, 0, 2, 2, 2, 1, 3)
    assert (c1.b, c1.p_begin, c1.p_end, c1.slot) == (1, 2, 6, 4)


def test_structure_check_catches_planted_mistakes():
    pages, hkv, grid = [6, 6, 0, 9], 2, 12
    plan = _tuples(H.stream_items(pages, hkv, grid, 1))
    check_items(plan, pages, hkv, 2)
    spanning = next(g for g, its in enumerate(plan) if len(its) == 2)

    def mutate(g, k, field, delta):
        bad = [list(its) for its in plan]
        it = list(bad[g][k])
        it[field] += delta
        bad[g][k] = tuple(it)
        return bad

    mistakes = [
        mutate(spanning, 0, 3, -1),   # item 1 stops a page early: a page uncovered
        mutate(spanning, 1, 2, 1),    # item 2 starts a page late
        mutate(spanning, 1, 8, -1),   # item 2 in item 1's slot
        mutate(spanning, 1, 7, -1),   # entry 0 offset lost: merge would read the wrong slot
        mutate(spanning, 0, 4, 1),    # wrong item count for the unit
    ]
    zero = next((g, k) for g, its in enumerate(plan) for k, it in enumerate(its) if it[4] == 0)
    bad = [list(its) for its in plan]
    del bad[zero[0]][zero[1]]
    mistakes.append(bad)               # the empty unit's zero rows without an owner
    for bad in mistakes:
        with pytest.raises(AssertionError):
            check_items(bad, pages, hkv, 2)

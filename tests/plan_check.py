"""Structure check of a launch's work items, shared by the CPU tests (on the Python mirror of the
stream planner) and the GPU tests (on the records the planner kernel writes).

An item is (b, kvh, p_begin, p_end, nsplit, slot0, sstride, odd, slot); workgroup g holds up to two.
What must hold for any correct plan:

* every (sequence, kv head) unit's pages [0, pages) are covered by its items exactly once, in order
  of the workgroups that hold them;
* a unit with pages has nsplit items, all carrying the same nsplit, slot0, sstride and odd, and item
  e (in workgroup order) owns slot slot0 + sstride * e (+ odd for e = 0);
* an empty unit has exactly one item, with nsplit 0 (it writes the zero rows);
* an item's slot is its workgroup's own: g (per-unit items, one per workgroup) or 2g / 2g + 1
  (stream items);
* no two items share a slot, and every slot is below the launch's slot count.
"""

from __future__ import annotations


def check_items(items_by_group, pages, num_kv_heads, slots_per_group):
    """items_by_group[g] = list of items of workgroup g (each a tuple as in the module docstring)."""
    hkv = num_kv_heads
    grid = len(items_by_group)
    nslots = grid * slots_per_group
    units = {}
    used_slots = set()
    for g, items in enumerate(items_by_group):
        assert len(items) <= slots_per_group, (g, items)
        for k, it in enumerate(items):
            b, kvh, p0, p1, nsplit, slot0, sstride, odd, slot = it
            assert 0 <= b < len(pages) and 0 <= kvh < hkv, (g, it)
            if sstride == 2:  # stream items: the workgroup's two slots
                assert slots_per_group == 2 and slot in (2 * g, 2 * g + 1), (g, it)
            else:  # per-unit items (also in stream launches, when the plan falls back to them)
                assert sstride == 1 and k == 0 and slot == g, (g, it)
            assert slot not in used_slots, (g, it)
            used_slots.add(slot)
            assert 0 <= slot < nslots
            units.setdefault((b, kvh), []).append((g, slot, it))
    for b, p in enumerate(pages):
        for kvh in range(hkv):
            its = sorted(units.get((b, kvh), []))
            if p == 0:
                assert len(its) == 1 and its[0][2][4] == 0, (b, kvh, its)
                continue
            assert its, (b, kvh)
            n = its[0][2][4]
            assert len(its) == n, (b, kvh, n, len(its))
            end = 0
            for e, (g, slot, it) in enumerate(its):
                _, _, p0, p1, nsplit, slot0, sstride, odd, _ = it
                assert (nsplit, slot0, sstride, odd) == (n, its[0][2][5], its[0][2][6], its[0][2][7]), (b, kvh, e)
                assert p0 == end and p1 > p0, (b, kvh, e, it)
                end = p1
                assert slot == slot0 + sstride * e + (odd if e == 0 else 0), (b, kvh, e, it)
                assert slot0 + sstride * n <= nslots
            assert end == p, (b, kvh, end, p)

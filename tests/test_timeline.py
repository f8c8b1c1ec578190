"""The measurement build with phase stamps (libpa_decode_tl.so) and its budget.

CPU: the timeline library exports the decode entry points plus the stamp
readers of include/pa_decode_timeline.h, the product library exports none of
the readers, and the budget arithmetic (timeline.phases) gives the known
answer on hand-made stamps.  GPU: real stamps are ordered along every
workgroup's path, and the timeline build decodes like the product build.
"""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

from paged_attention_decode_amd import _native
from paged_attention_decode_amd import timeline as tl

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "pa_decode_timeline.h")


def _declared():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    return sorted(set(re.findall(r"^\s*int\s+(pad_\w+)\s*\(", text, flags=re.M)))


def _header_constants():
    text = open(HEADER).read()
    return {k: int(v) for k, v in re.findall(r"#define (PAD_TL_\w+) (\d+)", text)}


def test_header_constants_match_python():
    c = _header_constants()
    assert (c["PAD_TL_LAUNCHES"], c["PAD_TL_MAX_GROUPS"], c["PAD_TL_SLOTS"]) == (
        _native.TL_LAUNCHES, _native.TL_MAX_GROUPS, _native.TL_SLOTS)
    assert [c[f"PAD_TL_{n}"] for n in ("ENTRY", "ITEM", "LOOP_END", "PUBLISHED", "ARRIVED", "MERGED", "EXIT",
                                       "INFO")] == list(range(8))
    assert (c["PAD_TL_F_NO_ITEM"], c["PAD_TL_F_SINGLE"], c["PAD_TL_F_MERGER"], c["PAD_TL_F_GROUP"]) == (
        _native.TL_F_NO_ITEM, _native.TL_F_SINGLE, _native.TL_F_MERGER, _native.TL_F_GROUP)


def test_timeline_library_exports():
    assert _declared() == sorted(_native.TIMELINE_SIGNATURES)
    lib = _native.timeline()
    for name in list(_native.SIGNATURES) + _declared():
        assert hasattr(lib, name), name
    product = ctypes.CDLL(_native.CAPI_PATH)
    for name in _declared():
        assert not hasattr(product, name), f"{name} must not be in the product library"


def _row(entry, item, loop_end, published=0, arrived=0, merged=0, exit_=0, flags=0, xcc=0, slot=0):
    info = (slot & 0xFFFFFFFF) | (xcc << 32) | (flags << 40)
    return [entry, item, loop_end, published, arrived, merged, exit_, info]


def test_phases_known_answer():
    # Two launches of 3 workgroups (ticks of 10 ns): in each, workgroup 1 is
    # the unit's last arrival; workgroup 2 has no item.
    buf = np.zeros((2, 4, 8), dtype=np.int64)
    for k, base in enumerate((1000, 5000)):
        buf[k, 0] = _row(base + 0, base + 90, base + 1090, base + 1190, base + 1240, 0, base + 1240, 0, 3, 0)
        buf[k, 1] = _row(base + 20, base + 110, base + 1150, base + 1250, base + 1300, base + 1400, base + 1400,
                         _native.TL_F_MERGER, 5, 1)
        buf[k, 2] = _row(base + 40, base + 130, 0, 0, 0, 0, base + 135, _native.TL_F_NO_ITEM, 1, -1)
    recs = tl.phases(buf, 3, [0, 1])
    r0, r1 = recs
    assert r0["gap"] is None
    assert r1["gap"] == pytest.approx((5000 - 2400) * 0.01)
    assert r0["span"] == pytest.approx(14.0)
    assert r0["dispatch"] == pytest.approx(0.4)
    assert r0["item"] == pytest.approx(0.9)  # median of 90 and 90 ticks (workgroup 2 has no item)
    assert r0["loop"] == pytest.approx((1000 + 1040) / 2 * 0.01)
    assert r0["loop_tail"] == pytest.approx((1150 - 1120) * 0.01)
    assert (r0["publish"], r0["arrive"], r0["merge"]) == (pytest.approx(1.0), pytest.approx(0.5),
                                                          pytest.approx(1.0))
    assert r0["exit_tail"] == pytest.approx(2.5)
    assert r0["xcc_ids"] == [3, 5]
    med = tl.median_budget(recs)
    assert med["gap"] == pytest.approx(26.0) and med["span"] == pytest.approx(14.0)


@pytest.mark.gpu
def test_timeline_stamps_ordered_and_outputs_match():
    from paged_attention_decode_amd import paged_attention_decode
    from paged_attention_decode_amd import workloads as wl

    sets = [wl.make("C2", batch=16, seed=5), wl.make("C3", seed=6)]
    for w in sets:
        outs = [torch.empty_like(w.q)]
        recs, groups, plan = tl.record([w], outs, repeats=1, warmup=2)
        torch.cuda.synchronize()
        expected = paged_attention_decode(*w.args())
        torch.cuda.synchronize()
        assert torch.equal(outs[0], expected), "timeline build must decode exactly like the product build"
        for r in recs:
            for p in ("span", "item", "loop", "publish", "arrive", "merge"):
                assert r[p] is not None and r[p] >= 0, (p, r)
            assert r["span"] >= r["loop"]
        lib = _native.timeline()
        n = _native.TL_LAUNCHES
        buf = (ctypes.c_uint64 * (n * _native.TL_MAX_GROUPS * _native.TL_SLOTS))()
        assert lib.pad_timeline_read(buf, ctypes.sizeof(buf)) == 0
        a = np.frombuffer(buf, dtype=np.uint64).astype(np.int64).reshape(n, _native.TL_MAX_GROUPS, _native.TL_SLOTS)
        rows = a[n - 1, :groups]
        flags = (rows[:, _native.TL_INFO] >> 40) & 0xFF
        has = (flags & _native.TL_F_NO_ITEM) == 0
        r = rows[has]
        assert (r[:, _native.TL_ITEM] >= r[:, _native.TL_ENTRY]).all()
        assert (r[:, _native.TL_LOOP_END] >= r[:, _native.TL_ITEM]).all()
        assert (r[:, _native.TL_EXIT] >= r[:, _native.TL_LOOP_END]).all()
        m = rows[(flags & _native.TL_F_MERGER) != 0]
        assert len(m) > 0
        assert (m[:, _native.TL_MERGED] >= m[:, _native.TL_ARRIVED]).all()
        assert (m[:, _native.TL_ARRIVED] >= m[:, _native.TL_PUBLISHED]).all()

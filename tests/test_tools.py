"""Measurement tooling: the bandwidth probes, the roofline report and the split sweep.

CPU: libpa_probe.so loads, exports its entry points and rejects invalid
arguments before touching a device.  GPU: one short run of each tool, with
sanity bounds on what it reports (the numbers themselves are measurements,
not parity claims).
"""

from __future__ import annotations

import pytest
import torch

from paged_attention_decode_amd import _native


def test_probe_library_exports():
    lib = _native.probe()
    for name in _native.PROBE_SIGNATURES:
        assert hasattr(lib, name), name


def test_probe_rejects_invalid_arguments():
    lib = _native.probe()
    # null pointers, zero sizes, misaligned buffers and shapes that do not tile a wave
    assert lib.pad_probe_stream_read(None, 1 << 20, 8, 4, 2, None, None) == 1
    assert lib.pad_probe_stream_read(16, 8, 8, 4, 2, 16, None) == 1
    assert lib.pad_probe_stream_read(24, 1 << 20, 8, 4, 2, 16, None) == 1
    assert lib.pad_probe_stream_read(16, 1 << 20, 8, 17, 2, 16, None) == 1
    # row of 48 B does not divide a 64-lane wave of 16-byte loads
    assert lib.pad_probe_paged_read(16, 16, 16, 4, 2, 1, 8192, 256, 16, 48, 512, 8, 4, 2, 16, None) == 1
    # tile larger than one page
    assert lib.pad_probe_paged_read(16, 16, 16, 4, 2, 1, 4096, 256, 16, 256, 512, 8, 4, 2, 16, None) == 1
    # more than 4 loads per lane per tile (64 rows of 256 B)
    assert lib.pad_probe_paged_read(16, 16, 16, 4, 1, 1, 1 << 16, 256, 64, 256, 256, 8, 4, 2, 16, None) == 1


@pytest.mark.gpu
def test_roofline_measure_small():
    from paged_attention_decode_amd import roofline

    rec = roofline.measure("C2", 1, calls=10)
    assert rec["algorithmic_bytes"] == 4201476
    assert rec["intensity_flop_per_byte"] == pytest.approx(6.0, rel=0.01)
    for key in ("us_per_call", "gbs", "paged_read_gbs", "stream_read_gbs"):
        assert rec[key] > 0, key
    assert rec["gbs"] < 8000 and rec["paged_read_gbs"] < 8000 and rec["stream_read_gbs"] < 8000
    assert 0 < rec["pct_of_paged_read"] < 200


@pytest.mark.gpu
def test_split_sweep_small():
    from paged_attention_decode_amd import sweep

    res = sweep.sweep("C2", 1, [1, 16], trials=2, iters=3, warmup=2)
    assert [r["num_splits"] for r in res["rows"]] == ["heuristic", 1, 16]
    assert all(r["us_per_call"] > 0 for r in res["rows"])
    assert res["heuristic_plan"]["num_splits"] >= 1
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_shape_survey_small():
    from paged_attention_decode_amd import sweep

    rows = sweep.survey(cases=[(2, 12, 2, 128, 4, 256), (2, 8, 4, 96, 16, 256)], calls=3, reps=1)
    assert [r["page_size"] for r in rows] == [4, 16]
    assert all(r["us_per_call"] > 0 and 0 < r["gbs"] < 8000 for r in rows)

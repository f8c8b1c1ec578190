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


def _write_csv(path, header, rows):
    import csv
    import os

    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_profile_summary_on_synthetic_runs(tmp_path):
    # profile_summary's arithmetic on hand-made rocprofv3 outputs: kernel
    # durations, the copy-calibrated traffic and the request-size check.
    from paged_attention_decode_amd import profile_summary as ps

    root = str(tmp_path)
    kname = "void pad::pad_phase1_kernel<128, 1, 0, 0, 0>(pad::Phase1Args)"
    log = "x: 4 calls over 3 input set(s); algorithmic bytes/call 1000000 (first set), 1200000 (mean over the calls)\n"
    for run in ("trace_T", "pmc_FETCH_SIZE_T", "pmc_WRITE_SIZE_T", "pmc_REQ_T"):
        open(f"{root}/{run}.log", "w").write(log)
    trace = [[kname, 256, 2, 64, 84, 512, 1000, 1000 + d] for d in (10000, 12000, 11000, 13000)]
    _write_csv(f"{root}/trace_T/run_kernel_trace.csv",
               ["Kernel_Name", "Workgroup_Size_X", "Grid_Size_Y", "Grid_Size_Z", "VGPR_Count", "LDS_Block_Size",
                "Start_Timestamp", "End_Timestamp"], [[r[0], r[1], r[2], r[3], r[4], r[5], r[6], r[7]] for r in trace])
    # Grid_Size_X is in work-items: 2 workgroups of 256.
    import csv
    rows = list(csv.DictReader(open(f"{root}/trace_T/run_kernel_trace.csv")))
    for r in rows:
        r["Grid_Size_X"] = "512"
    _write_csv(f"{root}/trace_T/run_kernel_trace.csv", list(rows[0].keys()), [list(r.values()) for r in rows])
    _write_csv(f"{root}/trace_T/run_kernel_stats.csv", ["Name", "AverageNs"], [[kname, 11500]])
    r = ps.trace_row(root, "T")
    assert r["mean_us"] == 11.5 and r["median_us"] == 11.5 and r["min_us"] == 10.0 and r["max_us"] == 13.0
    assert r["alg_bytes"] == 1000000 and r["grid"] == (2, 2, 64) and abs(r["gbs"] - 1e6 / 11.5e3) < 1e-9
    assert ps.trace_row(root, "T", ragged=True)["alg_bytes"] == 1200000
    copy = "__amd_rocclr_copyBuffer"
    hdr = ["Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"]
    _write_csv(f"{root}/pmc_FETCH_SIZE_T/run_counter_collection.csv", hdr,
               [[copy, "131072", "FETCH_SIZE", 131072.0], [kname, "512", "FETCH_SIZE", 500.0]])
    _write_csv(f"{root}/pmc_WRITE_SIZE_T/run_counter_collection.csv", hdr,
               [[copy, "131072", "WRITE_SIZE", 262144.0], [kname, "512", "WRITE_SIZE", 10.0]])
    t = ps.traffic(root, "T")
    assert t["fetch_scale"] == 2.0 and t["write_scale"] == 1.0
    assert t["fetch_bytes"] == 500 * 2 * 1024 and t["write_bytes"] == 10 * 1024
    req = [[copy, "131072", c, v] for c, v in zip(ps.REQ_COUNTERS, (2097152, 0, 0, 2097152))]
    req += [[kname, "512", c, v] for c, v in zip(ps.REQ_COUNTERS, (8000, 0, 100, 7000))]
    _write_csv(f"{root}/pmc_REQ_T/run_counter_collection.csv", hdr, req)
    q = ps.requests(root, "T")
    assert q["bytes_if_128b"] == 7900 * 128 + 100 * 32
    assert q["fetch_size_bytes"] == 7900 * 64 + 100 * 32
    assert q["copy_ratio_128b"] == 1.0


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

"""Roofline report for the decode kernel on this GPU.

    python -m paged_attention_decode_amd.roofline [--configs C1,C2:16,C2:64,C3,C4] [--json out.json]
        [--fetch-csv run_counter_collection.csv --write-csv ... --copy-kib 262144]

The MI355X counterpart of the reference's bench/roofline.py (which read a
measured peak bandwidth from bench/measure_peak_bw.py).  For each
configuration it reports, on cold inputs (calls rotate over KV caches that
together exceed twice the 256 MB Infinity Cache):

* algorithmic bytes and FLOPs per call (K and V of every valid token, q,
  output, the page ids in use and seq_lens; FLOPs = 4 * Hq * d * sum L, the
  reference's convention, bench/roofline.py:55-59), and the intensity
  (= the GQA group, FLOP per byte, far below the MFMA ridge);
* the decode's time per call (back-to-back calls, HIP events on the launch
  stream) and achieved GB/s, as a fraction of the 8000 GB/s specification;
* two measured ceilings from libpa_probe.so (csrc/pa_probe.hip): a plain
  contiguous stream of the same byte count, and the decode's own access
  pattern without arithmetic (the K and V tiles of every used page and kv
  head, 16-byte loads, several tiles in flight per wave); the decode's GB/s
  as a fraction of the latter is the share of what this page layout allows;
* with ``--fetch-csv`` / ``--write-csv`` (rocprofv3 ``--pmc FETCH_SIZE`` /
  ``WRITE_SIZE`` runs of ``profile_run``), the HBM traffic per call, scaled
  by what the counters read for profile_run's calibration copy of
  ``--copy-kib`` KiB.
"""

from __future__ import annotations

import argparse
import csv
import json
import math
import statistics

import torch

from . import paged_attention_decode
from . import workloads as wl
from ._native import probe

PEAK_GBS = 8000.0
MFMA_FP16_TFLOPS = 2500.0  # dense fp16 MFMA peak
MALL_BYTES = 256 * 1024 * 1024


def _sets(name, batch, seed0=1):
    w0 = wl.make(name, batch=batch, seed=seed0)
    per = w0.k_cache.numel() * 4
    n = max(2, math.ceil(2 * MALL_BYTES / per) + 1)
    return [w0] + [wl.make(name, batch=batch, seed=seed0 + i) for i in range(1, n)]


def _time(fn, n_sets, calls, warmup=20):
    for i in range(warmup):
        fn(i % n_sets)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for i in range(calls):
        fn(i % n_sets)
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) * 1e3 / calls  # us


def _used_pages(w):
    """Page ids of the used pages of every sequence (int32, device)."""
    ps = w.k_cache.shape[1]
    rows = []
    for b, n in enumerate(w.seq_lens_host):
        pages = -(-int(n) // ps)
        if pages:
            rows.append(w.block_table[b, :pages])
    return torch.cat(rows).to(torch.int32).contiguous()


# (workgroups per CU, waves, tiles or loads in flight per lane) settings
# tried for each probe; the best is the ceiling.  Wider grids matter: on
# MI355X the paged pattern reads ~3% faster with 8 workgroups of 8 waves per
# CU than with one, and 4 tiles in flight per lane is far slower than 2.
PROBE_SETTINGS = ((1, 8, 2), (1, 16, 2), (1, 16, 1), (2, 8, 2), (4, 4, 2), (4, 8, 2), (8, 8, 2), (8, 4, 2))


def ceilings(sets, calls=100, groups=0):
    """Measured read ceilings for the workloads `sets` (rotated, cold).

    Returns (paged_gbs, stream_gbs, details): the best GB/s over
    PROBE_SETTINGS of the decode's access pattern without arithmetic, and of
    a contiguous stream of the same byte count (the K and the V cache of a
    set read by two back-to-back launches).  `groups` > 0 fixes the
    workgroup count instead of the per-CU multiples of PROBE_SETTINGS.
    """
    w0 = sets[0]
    nbytes = wl.bytes_of(w0)
    stream = torch.cuda.current_stream().cuda_stream
    lib = probe()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    grid_sizes = [groups if groups > 0 else mult * cus for mult, _, _ in PROBE_SETTINGS]
    sink = torch.zeros(max(grid_sizes), dtype=torch.int32, device="cuda")
    p, ps, hkv, d = w0.k_cache.shape
    pages = [_used_pages(w) for w in sets]
    rows = 16 if ps % 16 == 0 else ps
    tiles = ps // rows
    slot_bytes = hkv * d * 2
    probe_bytes = pages[0].numel() * hkv * ps * d * 2 * 2

    def paged(i, g, waves, depth):
        st = lib.pad_probe_paged_read(sets[i].k_cache.data_ptr(), sets[i].v_cache.data_ptr(), pages[i].data_ptr(),
                                      pages[i].numel(), hkv, tiles, ps * slot_bytes, d * 2, rows, d * 2, slot_bytes,
                                      g, waves, depth, sink.data_ptr(), stream)
        assert st == 0, st

    # The sets' caches differ in size when their lengths are drawn per seed
    # (C3, C5): every probe stays inside its own set's buffers.
    paged_rate = {}
    for g, (_, wv, dp) in zip(grid_sizes, PROBE_SETTINGS):
        us = _time(lambda i: paged(i, g, wv, dp), len(sets), calls)
        paged_rate[(g, wv, dp)] = sum(p.numel() for p in pages) / len(pages) * hkv * ps * d * 4 / us / 1e3

    # A contiguous stream of the same byte count: half of it from the K
    # cache, half from the V cache (capped by the smallest cache).
    span = min([nbytes // 2] + [w.k_cache.numel() * 2 for w in sets]) // 16 * 16

    def contiguous(i, g, waves, depth):
        for cache in (sets[i].k_cache, sets[i].v_cache):
            st = lib.pad_probe_stream_read(cache.data_ptr(), span, g, waves, depth, sink.data_ptr(), stream)
            assert st == 0, st

    stream_rate = {}
    for g, (_, wv, dp) in zip(grid_sizes, PROBE_SETTINGS):
        us = _time(lambda i: contiguous(i, g, wv, dp), len(sets), calls)
        stream_rate[(g, wv, dp)] = 2 * span / us / 1e3
    best_paged = max(paged_rate, key=paged_rate.get)
    best_stream = max(stream_rate, key=stream_rate.get)
    details = {"paged_best": {"groups": best_paged[0], "waves": best_paged[1], "depth": best_paged[2]},
               "stream_best": {"groups": best_stream[0], "waves": best_stream[1], "depth": best_stream[2]},
               "paged_bytes": probe_bytes, "stream_bytes": 2 * span}
    del pages
    return paged_rate[best_paged], stream_rate[best_stream], details


def measure(name, batch, calls=100, groups=0):
    sets = _sets(name, batch)
    w0 = sets[0]
    nbytes = wl.bytes_of(w0)
    flops = wl.flops_of(w0)

    def decode(i):
        paged_attention_decode(*sets[i].args())

    t_dec = _time(decode, len(sets), calls)
    paged_gbs, stream_gbs, details = ceilings(sets, calls, groups)
    gbs = nbytes / t_dec / 1e3
    group = w0.q.shape[1] // w0.k_cache.shape[2]
    rec = {
        "config": w0.name,
        "algorithmic_bytes": nbytes,
        "flops": flops,
        "intensity_flop_per_byte": round(flops / nbytes, 3),
        "gqa": group,
        "us_per_call": round(t_dec, 3),
        "gbs": round(gbs, 1),
        "pct_of_peak": round(100 * gbs / PEAK_GBS, 2),
        "gflops": round(flops / t_dec / 1e3, 1),
        "paged_read_gbs": round(paged_gbs, 1),
        "pct_of_paged_read": round(100 * gbs / paged_gbs, 2),
        "stream_read_gbs": round(stream_gbs, 1),
        "probe": details,
    }
    del sets
    torch.cuda.empty_cache()
    return rec


def _counter_median(path, counter):
    """Median per-dispatch value of `counter` for the decode kernel, and for the copy kernel."""
    dec, cpy = [], []
    with open(path) as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") != counter:
                continue
            name = row.get("Kernel_Name", "")
            val = float(row["Counter_Value"])
            if "pad_phase1_kernel" in name:
                dec.append(val)
            elif "copy" in name.lower():
                cpy.append(val)
    return (statistics.median(dec) if dec else None), (statistics.median(cpy) if cpy else None)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--configs", default="C1,C2:1,C2:16,C2:64,C3,C4")
    ap.add_argument("--calls", type=int, default=100)
    ap.add_argument("--json", default="")
    ap.add_argument("--fetch-csv", default="")
    ap.add_argument("--write-csv", default="")
    ap.add_argument("--copy-kib", type=float, default=262144.0,
                    help="KiB the calibration copy reads and writes per dispatch")
    a = ap.parse_args()
    assert torch.cuda.is_available(), "the roofline report needs a GPU"
    ridge = MFMA_FP16_TFLOPS * 1e3 / PEAK_GBS
    print(f"spec: {PEAK_GBS:.0f} GB/s HBM, {MFMA_FP16_TFLOPS:.0f} TFLOP/s dense fp16 MFMA; ridge {ridge:.0f} FLOP/B")
    print(f"{'config':10s} {'bytes':>12s} {'FLOP/B':>6s} {'us':>9s} {'GB/s':>8s} {'%peak':>6s} "
          f"{'paged-read GB/s':>15s} {'%paged':>7s} {'stream GB/s':>11s}")
    out = []
    for spec in a.configs.split(","):
        name, _, b = spec.partition(":")
        print(f"# measuring {spec}", flush=True)
        rec = measure(name, int(b) if b else None, a.calls)
        out.append(rec)
        print(f"{rec['config']:10s} {rec['algorithmic_bytes']:12d} {rec['intensity_flop_per_byte']:6.2f} "
              f"{rec['us_per_call']:9.2f} {rec['gbs']:8.1f} {rec['pct_of_peak']:6.2f} {rec['paged_read_gbs']:15.1f} "
              f"{rec['pct_of_paged_read']:7.2f} {rec['stream_read_gbs']:11.1f}", flush=True)
    if a.fetch_csv or a.write_csv:
        traffic = {}
        for path, counter, key in ((a.fetch_csv, "FETCH_SIZE", "fetch"), (a.write_csv, "WRITE_SIZE", "write")):
            if path:
                dec, cpy = _counter_median(path, counter)
                scale = (a.copy_kib / cpy) if cpy else 1.0
                traffic[key] = {"kib_raw": dec, "scale": round(scale, 4),
                                "bytes": None if dec is None else int(dec * scale * 1024)}
        print("traffic per call:", json.dumps(traffic))
        out.append({"traffic": traffic})
    if a.json:
        with open(a.json, "w") as f:
            json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()

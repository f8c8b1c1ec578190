"""Summaries of rocprofv3 runs of ``profile_run`` (the tables committed under profiles/).

Input: one rocprofv3 output directory per run, named ``<root>/<kind>_<name>``
with ``-o run`` (``run_kernel_trace.csv`` / ``run_kernel_stats.csv`` for
kernel traces, ``run_counter_collection.csv`` for counters) and the run's
stdout in ``<root>/<kind>_<name>.log`` (profile_run prints the algorithmic
bytes per call).  Kinds:

* ``trace_<name>``: ``rocprofv3 --kernel-trace --stats`` -> one table row:
  dispatches, mean (stats) / median / min / max kernel duration, algorithmic
  bytes, GB/s and % of the 8 TB/s peak, grid, workgroup size, VGPRs, LDS.
* ``pmc_FETCH_SIZE_<name>`` / ``pmc_WRITE_SIZE_<name>``: HBM bytes per call,
  each scaled by what the same counter reads for profile_run's calibration
  copy (PyTorch's copy kernel over 256 MiB, grid 131072: 262144 KiB read and
  written per dispatch).
* ``pmc_REQ_<name>``: ``TCC_EA0_RDREQ``, ``TCC_BUBBLE``, ``TCC_EA0_RDREQ_32B``
  and ``TCC_EA0_RDREQ_DRAM`` (sums) - the read requests FETCH_SIZE is built
  from on gfx950 (FETCH_SIZE = (BUBBLE*128 + (RDREQ - BUBBLE - RDREQ_32B)*64
  + RDREQ_32B*32) / 1024 in rocprofv3's counter definitions), to check the
  calibration scale against the decode kernel's own request count: with
  128-byte requests, (RDREQ - RDREQ_32B)*128 + RDREQ_32B*32 bytes were read.

Usage: ``python -m paged_attention_decode_amd.profile_summary --root DIR
[--trace N1,N2] [--traffic N1,N2] [--requests N1,N2] [--traffic-json OUT]
[--commit SHA]``.
"""

from __future__ import annotations

import argparse
import csv
import json
import os
import re
import statistics

KERNEL = "pad::pad_phase1_kernel"
COPY_GRID = "131072"
COPY_KIB = 262144.0  # 256 MiB
PEAK_GBS = 8000.0
csv.field_size_limit(1 << 30)


def _rows(path):
    with open(path) as f:
        return list(csv.DictReader(f))


def algorithmic_bytes(log_path):
    """(first set's bytes, mean over the calls, input sets) from profile_run's output."""
    txt = open(log_path).read()
    m = re.search(r"algorithmic bytes/call (\d+) \(first set\), (\d+) \(mean over the calls\)", txt)
    sets = re.search(r"(\d+) calls over (\d+) input set", txt)
    return int(m.group(1)), float(m.group(2)), int(sets.group(2))


def trace_row(root, name, ragged=False):
    d = os.path.join(root, f"trace_{name}")
    tr = [r for r in _rows(os.path.join(d, "run_kernel_trace.csv")) if KERNEL in r["Kernel_Name"]]
    st = [r for r in _rows(os.path.join(d, "run_kernel_stats.csv")) if KERNEL in r["Name"]]
    durs = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in tr]
    mean = float(st[0]["AverageNs"]) / 1e3
    first, meanb, nsets = algorithmic_bytes(os.path.join(root, f"trace_{name}.log"))
    ab = meanb if ragged else first
    wg = int(tr[0]["Workgroup_Size_X"])
    grid = (int(tr[0]["Grid_Size_X"]) // wg, int(tr[0]["Grid_Size_Y"]), int(tr[0]["Grid_Size_Z"]))
    gbs = ab / mean / 1e3
    return {"config": name, "calls": len(durs), "mean_us": mean, "median_us": statistics.median(durs),
            "min_us": min(durs), "max_us": max(durs), "alg_bytes": int(round(ab)), "gbs": gbs,
            "pct_peak": 100 * gbs / PEAK_GBS, "grid": grid, "wg": wg, "vgpr": tr[0].get("VGPR_Count", ""),
            "lds": tr[0].get("LDS_Block_Size", ""), "sets": nsets,
            "kernel": tr[0]["Kernel_Name"].split("(")[0]}


def trace_table(rows):
    w = max([8] + [len(r["config"]) for r in rows])
    hdr = (f"{'config':{w}s} {'calls':>5s} {'mean_us':>8s} {'median_us':>9s} {'min_us':>7s} {'max_us':>8s} "
           f"{'alg_bytes':>12s} {'GB/s':>6s} {'%peak':>6s}  {'grid(x,y,z)':13s} {'wg':>4s} {'vgpr':>5s} {'lds':>4s} "
           f"{'sets':>4s}  template")
    out = [hdr]
    for r in rows:
        g = "({},{},{})".format(*r["grid"])
        t = re.search(r"<([^>]*)>", r["kernel"])
        out.append(f"{r['config']:{w}s} {r['calls']:5d} {r['mean_us']:8.2f} {r['median_us']:9.2f} {r['min_us']:7.2f} "
                   f"{r['max_us']:8.2f} {r['alg_bytes']:12d} {r['gbs']:6.0f} {r['pct_peak']:6.1f}  {g:13s} "
                   f"{r['wg']:4d} {r['vgpr']:>5s} {r['lds']:>4s} {r['sets']:4d}  <{t.group(1) if t else '?'}>")
    return "\n".join(out)


def _counter(root, run, ctr):
    rs = _rows(os.path.join(root, run, "run_counter_collection.csv"))
    k = [float(r["Counter_Value"]) for r in rs if KERNEL in r["Kernel_Name"] and r["Counter_Name"] == ctr]
    c = [float(r["Counter_Value"]) for r in rs
         if "copyBuffer" in r["Kernel_Name"] and r["Grid_Size"] == COPY_GRID and r["Counter_Name"] == ctr]
    # Every copy dispatch counted must be the calibration copy of known size.
    if c and max(c) > 1.01 * min(c):
        raise ValueError(f"{run}: copy dispatches of grid {COPY_GRID} with different {ctr} ({min(c)} .. {max(c)}): "
                         "some are not the calibration copy")
    return (statistics.median(k) if k else None), (statistics.median(c) if c else None), len(k)


def traffic(root, name, ragged=False):
    fk, fc, n = _counter(root, f"pmc_FETCH_SIZE_{name}", "FETCH_SIZE")
    wk, wc, _ = _counter(root, f"pmc_WRITE_SIZE_{name}", "WRITE_SIZE")
    fs, ws = COPY_KIB / fc, COPY_KIB / wc
    fb, wb = fk * fs * 1024, wk * ws * 1024
    first, meanb, _ = algorithmic_bytes(os.path.join(root, f"pmc_FETCH_SIZE_{name}.log"))
    ab = meanb if ragged else first
    return {"bytes_per_call": int(round(fb + wb)), "fetch_bytes": int(round(fb)), "write_bytes": int(round(wb)),
            "fetch_raw_kib": fk, "write_raw_kib": wk, "fetch_scale": round(fs, 5), "write_scale": round(ws, 5),
            "algorithmic_bytes": int(round(ab)), "ratio": (fb + wb) / ab, "dispatches": n}


REQ_COUNTERS = ("TCC_EA0_RDREQ_sum", "TCC_BUBBLE_sum", "TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_DRAM_sum")


def requests(root, name, ragged=False):
    run = f"pmc_REQ_{name}"
    vals = {c: _counter(root, run, c) for c in REQ_COUNTERS}
    rd, bub, r32, dram = (vals[c][0] for c in REQ_COUNTERS)
    crd, cbub, c32, _ = (vals[c][1] for c in REQ_COUNTERS)
    first, meanb, _ = algorithmic_bytes(os.path.join(root, f"{run}.log"))
    ab = meanb if ragged else first
    as_fetch = bub * 128 + (rd - bub - r32) * 64 + r32 * 32
    as_128 = (rd - r32) * 128 + r32 * 32
    copy_128 = (crd - c32) * 128 + c32 * 32 if crd is not None else None
    return {"rdreq": rd, "bubble": bub, "rdreq_32b": r32, "rdreq_dram": dram, "fetch_size_bytes": as_fetch,
            "bytes_if_128b": as_128, "algorithmic_bytes": int(round(ab)), "ratio_128b": as_128 / ab,
            "copy_rdreq": crd, "copy_bubble": cbub, "copy_bytes_if_128b": copy_128,
            "copy_ratio_128b": (copy_128 / (COPY_KIB * 1024)) if copy_128 else None}


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--root", required=True)
    p.add_argument("--trace", default="")
    p.add_argument("--traffic", default="")
    p.add_argument("--requests", default="")
    p.add_argument("--ragged", default="C3,C5", help="configs whose bytes are the mean over the calls' input sets")
    p.add_argument("--traffic-json", default="")
    p.add_argument("--commit", default="", help="commit the runs measured (recorded in the traffic JSON)")
    a = p.parse_args()
    ragged = set(a.ragged.split(","))
    if a.trace:
        print(trace_table([trace_row(a.root, n, n in ragged) for n in a.trace.split(",")]))
    recs = {}
    for n in filter(None, a.traffic.split(",")):
        t = traffic(a.root, n, n in ragged)
        recs[n] = t
        print(f"{n + ':':8s}FETCH_SIZE {t['fetch_raw_kib']:10.1f} KiB raw -> {t['fetch_bytes']:11d} B; "
              f"WRITE_SIZE {t['write_raw_kib']:8.1f} KiB raw -> {t['write_bytes']:9d} B;\n"
              f"        traffic {t['bytes_per_call']:11d} B per call vs algorithmic {t['algorithmic_bytes']:11d} B "
              f"(ratio {t['ratio']:.4f}); scales x{t['fetch_scale']} / x{t['write_scale']}")
    for n in filter(None, a.requests.split(",")):
        r = requests(a.root, n, n in ragged)
        print(f"{n + ':':8s}RDREQ {r['rdreq']:.0f}, BUBBLE {r['bubble']:.0f}, RDREQ_32B {r['rdreq_32b']:.0f}, "
              f"RDREQ_DRAM {r['rdreq_dram']:.0f};\n"
              f"        as FETCH_SIZE counts them {r['fetch_size_bytes']:.0f} B; as 128-byte requests "
              f"{r['bytes_if_128b']:.0f} B = {r['ratio_128b']:.4f} x algorithmic {r['algorithmic_bytes']}"
              + (f";\n        calibration copy: RDREQ {r['copy_rdreq']:.0f}, BUBBLE {r['copy_bubble']:.0f} -> "
                 f"{r['copy_bytes_if_128b']:.0f} B as 128-byte requests = {r['copy_ratio_128b']:.4f} x 256 MiB"
                 if r["copy_rdreq"] else ""))
    if a.traffic_json and recs:
        for n, t in recs.items():
            t["source"] = "profiles/pad_phase1_kernel_hbm_traffic.txt"
            if a.commit:
                t["commit"] = a.commit
        with open(a.traffic_json, "w") as f:
            json.dump(recs, f, indent=1)


if __name__ == "__main__":
    main()

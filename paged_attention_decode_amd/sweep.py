"""Split-count sweep: µs per decode call for each num_splits, against the heuristic.

    python -m paged_attention_decode_amd.sweep [--config C2] [--batch 1] [--splits 1,2,4,...] [--json out.json]
    python -m paged_attention_decode_amd.sweep --survey [--json out.json]

The MI355X counterpart of the reference's bench/bench_cuda_v4_num_splits.py
(which swept num_splits 1..128 at batch 1 to choose its fixed default of 64,
src/kernel_cuda_v4.py:16).  Same measuring discipline: every setting is timed
in interleaved trials (each the best of ``--iters`` event-bracketed calls
after a warm-up), and the median over ``--trials`` trials is reported, so
clock and power-state drift hits all settings alike.  The heuristic's own
choice (``num_splits=None``: the plan of csrc/pa_decode.hip, with in-kernel
balancing of ragged batches) is timed as one more setting; the plan it picks
is printed with it.

``--survey`` times the decode (heuristic plan) over page sizes and model
shapes outside the benchmark configurations - page sizes 1-32 (the
reference's fuzz set plus 2 and 12), head_dim 32-256 and GQA ratios 1-8 -
on cold inputs (calls rotate over KV caches larger than twice the 256 MB
Infinity Cache), back-to-back calls between HIP events.
"""

from __future__ import annotations

import argparse
import json
import math
import statistics

import torch

from . import paged_attention_decode, plan
from . import workloads as wl


def _best_of(fn, iters):
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    best = float("inf")
    for _ in range(iters):
        s.record()
        fn()
        e.record()
        torch.cuda.synchronize()
        best = min(best, s.elapsed_time(e))
    return best * 1e3  # us


def sweep(name, batch, splits, trials=9, iters=30, warmup=10):
    w = wl.make(name, batch=batch, seed=7)
    settings = [None] + list(splits)
    fns = {s: (lambda s=s: paged_attention_decode(*w.args(), num_splits=s)) for s in settings}
    for s in settings:
        for _ in range(warmup):
            fns[s]()
    torch.cuda.synchronize()
    samples = {s: [] for s in settings}
    for _ in range(trials):
        for s in settings:
            samples[s].append(_best_of(fns[s], iters))
    shp = w.shape
    chosen = plan(shp["batch"], shp["num_q_heads"], shp["num_kv_heads"], shp["head_dim"], shp["page_size"],
                  shp["max_pages"], 0)
    nbytes = wl.bytes_of(w)
    rows = []
    for s in settings:
        us = statistics.median(samples[s])
        rows.append({"num_splits": "heuristic" if s is None else s, "us_per_call": round(us, 2),
                     "gbs": round(nbytes / us / 1e3, 1)})
    return {"config": w.name, "algorithmic_bytes": nbytes, "heuristic_plan": chosen, "rows": rows}


# (batch, q heads, kv heads, head_dim, page_size, seq_len) of the survey.
SURVEY_CASES = (
    [(32, 12, 2, 128, ps, 4096) for ps in (16, 32, 8, 4, 2, 1, 12, 3)] + [(64, 12, 2, 128, 24, 4096)]
    + [(32, 32, 8, 128, 16, 2048), (8, 32, 32, 128, 16, 4096), (32, 64, 8, 128, 16, 2048),
       (64, 16, 2, 64, 16, 4096), (32, 32, 8, 64, 16, 2048), (32, 24, 8, 96, 16, 2048),
       (8, 32, 32, 96, 16, 4096), (32, 16, 4, 32, 16, 4096), (32, 16, 4, 256, 16, 2048),
       (64, 32, 8, 256, 16, 2048), (8, 16, 1, 256, 16, 8192)]
    # long single-kv-head (MQA) rows: hundreds of splits, two-level merge
    + [(1, 8, 1, 128, 16, 131072), (1, 16, 1, 128, 16, 262144)]
)


def survey(cases=SURVEY_CASES, calls=40, reps=5):
    """µs per call and algorithmic GB/s for each case, cold inputs."""
    mall = 256 * 1024 * 1024
    rows = []
    for batch, hq, hkv, d, ps, seq in cases:
        lens = [seq] * batch
        w0 = wl._build(f"s{ps}", lens, hq, hkv, d, ps, 100, "cuda")
        n = max(2, math.ceil(2 * mall / (w0.k_cache.numel() * 4)) + 1)
        sets = [w0] + [wl._build(f"s{ps}", lens, hq, hkv, d, ps, 100 + i, "cuda") for i in range(1, n)]
        for i in range(10):
            paged_attention_decode(*sets[i % n].args())
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        samples = []
        for _ in range(reps):
            torch.cuda.synchronize()
            s.record()
            for i in range(calls):
                paged_attention_decode(*sets[i % n].args())
            e.record()
            torch.cuda.synchronize()
            samples.append(s.elapsed_time(e) * 1e3 / calls)
        us = statistics.median(samples)
        nbytes = wl.bytes_of(w0)
        p = plan(batch, hq, hkv, d, ps, w0.block_table.shape[1], 0)
        rows.append({"batch": batch, "num_q_heads": hq, "num_kv_heads": hkv, "head_dim": d, "page_size": ps,
                     "seq_len": seq, "algorithmic_bytes": nbytes, "us_per_call": round(us, 2),
                     "gbs": round(nbytes / us / 1e3, 1), "pct_of_peak": round(100 * nbytes / us / 1e3 / 8000, 1),
                     "plan": f"{p['num_splits']}x{p['waves_per_group']}"})
        del sets, w0
    return rows


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--config", default="C2")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--splits", default="1,2,4,8,16,32,64,128")
    ap.add_argument("--trials", type=int, default=9)
    ap.add_argument("--iters", type=int, default=30)
    ap.add_argument("--json", default="")
    ap.add_argument("--survey", action="store_true", help="time page sizes and model shapes instead")
    a = ap.parse_args()
    assert torch.cuda.is_available(), "the sweep needs a GPU"
    if a.survey:
        rows = survey()
        print("batch  Hq/Hkv  head_dim  page  seq_len      MB      us     GB/s  %peak  plan")
        for r in rows:
            print(f"{r['batch']:5d}  {r['num_q_heads']:2d}/{r['num_kv_heads']:<2d}  {r['head_dim']:8d}  {r['page_size']:4d}  "
                  f"{r['seq_len']:7d}  {r['algorithmic_bytes'] / 1e6:6.1f}  {r['us_per_call']:6.2f}  {r['gbs']:7.1f}  "
                  f"{r['pct_of_peak']:5.1f}  {r['plan']}", flush=True)
        if a.json:
            with open(a.json, "w") as f:
                json.dump(rows, f, indent=1)
        return
    res = sweep(a.config, a.batch, [int(x) for x in a.splits.split(",")], a.trials, a.iters)
    p = res["heuristic_plan"]
    print(f"{res['config']}: {res['algorithmic_bytes']} algorithmic bytes per call (warm inputs); heuristic plan: "
          f"{p['num_splits']} splits x {p['waves_per_group']} waves, {p['pages_per_split']} pages per split")
    best = min(res["rows"], key=lambda r: r["us_per_call"])
    for r in res["rows"]:
        mark = "  <- fastest" if r is best else ""
        print(f"  num_splits={str(r['num_splits']):>9s}  {r['us_per_call']:8.2f} us  {r['gbs']:8.1f} GB/s{mark}")
    if a.json:
        with open(a.json, "w") as f:
            json.dump(res, f, indent=1)


if __name__ == "__main__":
    main()

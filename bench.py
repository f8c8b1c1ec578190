"""Benchmark of the MI355X paged-attention decode path.

Metric: µs per decode call and achieved HBM GB/s (% of the
8 TB/s peak) on the GQA 12/2, head_dim 128, page 16 shape at batch 1-64,
seq_len 4096 (configuration C2).

What one run measures (one GPU; ``--gpus`` above 1 exits with a message):

* ``value``: whole-job throughput of the headline step (C2 at batch 64 by
  default) in algorithmic GB/s: K timed decode calls back to back, bracketed
  by ``torch.cuda.synchronize()``, inputs resident in HBM.  Calls rotate over
  R distinct KV caches whose total exceeds the 256 MB Infinity Cache twice,
  so the number is an HBM figure ("cold"), not a cache figure.
* ``roofline``: the decode kernel (one launch per call: split-K phase 1
  with the log-sum-exp merge fused in) - algorithmic bytes per call divided
  by the time per call, timed with HIP events on the launch stream around
  the K back-to-back calls of the timed region (``us_per_call``: it includes
  the gap between consecutive kernels, so it is at least the kernel
  duration); peak 8000 GB/s.  ``traffic`` (HBM bytes per call) is not
  measured in this run: it is the rocprofv3 FETCH_SIZE / WRITE_SIZE figure
  committed in profiles/traffic.json (``traffic_source`` names the file and
  the commit that last changed it); ``fetch_gbs`` = traffic / us_per_call,
  north_star's "FETCH_SIZE / kernel time" with the same conservative time.
  ``kernel_trace_us_committed`` is the mean kernel duration rocprofv3
  measured for the same configuration in another run, read from the
  committed profiles/pad_phase1_kernel_configs_kernel_trace.txt
  (``kernel_trace_source`` names the file and the kernel's commit);
  ``timed_region_wall_s`` is the host wall clock of the K timed calls alone
  (synchronize to synchronize, warm-up excluded).
* ``c2_sweep``: for every batch of C2, the reference's latency method
  (bench/bench_decode.py:86-112 of the reference: each call bracketed by
  events and followed by a sync, best of 30 after 10 warm-up calls, median
  of 15 trials, warm inputs; ``us_per_call_warm_trials`` holds the 15
  per-trial values) and the cold steady-state throughput of
  ``--sweep-calls`` back-to-back calls (rotated KV caches), independent of
  ``--steps`` so that the first call's host-side latency is spread over
  enough calls.
* ``cpu_baseline``: the fp32 CPU oracle (oracle/reference.py, a restatement
  of the reference's src/reference.py) timed on the host cores on the same
  headline inputs for a bounded sample (about --cpu-seconds of work), in the
  same GB/s unit.  It uses every core of the process's CPU affinity up to
  --cpu-threads (16: the share of a GPU box's cores that one GPU gets);
  ``host`` records os.cpu_count(), the affinity size and the threads used.
* ``gpu``: device metadata (torch device properties, and amd-smi's static
  and metric readings when the tool answers), as the reference's bench
  records nvidia-smi's (bench/measure_peak_bw.py:27-42).
* ``roofline.measured_ceiling_gbs``: what a read-only kernel with the
  decode's own access pattern (K and V tiles of the same pages, no
  arithmetic; libpa_probe.so via roofline.ceilings) reaches on the same
  rotated inputs - the practical ceiling for this page layout.
* ``c3_ragged``: configuration C3 (batch 32, seq_lens uniform in
  [1, 8192], page 32) through the drop-in (in-kernel planned splits),
  through the CSR page-index entry, and planned once with
  ``BatchDecodeWrapper`` then run (``*_planned``: the plan-once-run-many
  flow of the reference's FlashInfer benchmark,
  bench/bench_flashinfer.py:131-151 of the reference; the plan is made
  before the timed region, as a decoding loop makes it once per step for
  all layers), cold throughput.
* ``c2_sweep[b].us_per_call_cold_planned``: the same plan-once-run-many
  timing for each batch of C2.
* ``c2_fp8`` (``--no-fp8`` skips it): the headline step over fp8 K/V caches
  (float8_e4m3fn and float8_e5m2 codes of the same C2 inputs, per-tensor
  scales; ``paged_attention_decode_fp8``), cold throughput in GB/s of its
  own algorithmic bytes (one byte per K/V element), the time ratio to the
  fp16 headline, and batch 1 by the reference's latency method; and
  ``c2_bf16``, the same step in bfloat16 (q, caches and output).  Not the
  metric, which is quoted on fp16 caches.
* ``cpu_baseline_configs`` (``--cpu-configs``, by default C1, C3, C4 and
  C5; ``none`` skips it): the CPU oracle next to the GPU call on each listed
  configuration in the same run, with the sample sizes the reference's bench
  conventions suggest (median of at least 5 calls on C1-C3, one call on C4,
  8 seeded rows of C5); a table of it goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import statistics
import subprocess
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

METRIC = "µs/decode call + achieved HBM GB/s (% of peak), GQA 12/2 d128, batch 1–64"
PEAK_GBS = 8000.0
MALL_BYTES = 256 * 1024 * 1024


def _parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    # About 10 ms of untimed calls: a shorter warm-up left the first timed
    # region of a process ~2.5% slower than every later one.
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--batch", type=int, default=64, help="C2 batch of the headline step")
    p.add_argument("--engine", type=int, default=0, help="phase-1 engine: 0 MFMA, 1 VALU/DPP")
    p.add_argument("--num-splits", type=int, default=0, help="0 = heuristic")
    p.add_argument("--no-sweep", action="store_true", help="skip the batch sweep")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-ceiling", action="store_true", help="skip the measured read ceiling")
    p.add_argument("--no-ragged", action="store_true", help="skip the C3 ragged line")
    p.add_argument("--no-fp8", action="store_true", help="skip the fp8-cache lines")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--cpu-threads", type=int, default=16,
                   help="most CPU threads for the baseline (a GPU box grants one GPU 16 cores)")
    p.add_argument("--cpu-configs", default="C1,C3,C4,C5",
                   help="also time the CPU oracle on these configurations (e.g. C1,C2:16,C2:64,C3,C4,C5) "
                        "next to the GPU call; adds cpu_baseline_configs to the JSON line and a table on "
                        "stderr ('none' skips it)")
    p.add_argument("--trials", type=int, default=15)
    p.add_argument("--sweep-calls", type=int, default=200, help="cold back-to-back calls per C2 sweep batch")
    return p.parse_args()


def _rotation(ws_bytes: int) -> int:
    return max(2, math.ceil(2 * MALL_BYTES / max(ws_bytes, 1)) + 1)


def _make_sets(make, n, **kw):
    return [make(seed=1000 + i, **kw) for i in range(n)]


def _call(pad, w, engine, splits):
    if w.k_cache.element_size() == 1:  # fp8 caches (workloads.to_fp8)
        return pad.paged_attention_decode_fp8(*w.args(), k_scale=w.k_scale, v_scale=w.v_scale,
                                              num_splits=splits or None)
    return pad.paged_attention_decode_ex(*w.args(), num_splits=splits or None, engine=engine)


def _throughput(pad, sets, engine, splits, steps, warmup, wall=None):
    """Seconds per call over `steps` back-to-back calls (events on the launch stream).

    With a list `wall`, also appends the host wall-clock seconds of the timed
    region alone: from the synchronize before the first timed call to the
    synchronize after the last (the warm-up calls are outside it)."""
    import torch

    for i in range(warmup):
        _call(pad, sets[i % len(sets)], engine, splits)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        _call(pad, sets[i % len(sets)], engine, splits)
    end.record()
    torch.cuda.synchronize()
    if wall is not None:
        wall.append(time.perf_counter() - t0)
    return start.elapsed_time(end) / 1e3 / steps


def _throughput_planned(pad, sets, splits, steps, warmup):
    """Seconds per call of BatchDecodeWrapper.run over `steps` back-to-back calls.

    Each input set is planned once before the timed region (plan once per
    decode step, run once per layer); the timed calls only run."""
    import torch

    wraps = []
    for w in sets:
        pw = pad.BatchDecodeWrapper()
        sh = w.shape
        pw.plan_block_table(w.block_table, w.seq_lens, sh["num_q_heads"], sh["num_kv_heads"], sh["head_dim"],
                            sh["page_size"], num_splits=splits or None)
        wraps.append(pw)
    for i in range(warmup):
        j = i % len(sets)
        wraps[j].run(sets[j].q, (sets[j].k_cache, sets[j].v_cache))
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(steps):
        j = i % len(sets)
        wraps[j].run(sets[j].q, (sets[j].k_cache, sets[j].v_cache))
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / steps


def _latency_reference_method(pad, w, engine, splits, trials):
    """bench/bench_decode.py:86-112 of the reference: median of best-of-30 event timings.

    Returns (median µs, the per-trial best-of-30 values in µs)."""
    import torch

    def once():
        for _ in range(10):
            _call(pad, w, engine, splits)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        best = float("inf")
        for _ in range(30):
            s.record()
            _call(pad, w, engine, splits)
            e.record()
            torch.cuda.synchronize()
            best = min(best, s.elapsed_time(e))
        return best

    samples = [once() * 1e3 for _ in range(trials)]  # µs
    return statistics.median(samples), samples


def _git_last_commit(relpath):
    try:
        out = subprocess.run(["git", "-C", REPO, "log", "-1", "--format=%h %cs", "--", relpath],
                             capture_output=True, text=True, timeout=10)
        return out.stdout.strip() or None
    except (OSError, subprocess.SubprocessError):
        return None


def _traffic(workload_name):
    """(bytes per call, provenance) from the committed rocprofv3 traffic summary, or (None, None)."""
    rel = os.path.join("profiles", "traffic.json")
    path = os.path.join(REPO, rel)
    if not os.path.exists(path):
        return None, None
    try:
        data = json.load(open(path))
        rec = data.get(workload_name)
        if rec is None:
            return None, None
        # The summary records the commit it was measured at; the GPU box has no .git to ask.
        commit = rec.get("commit") or _git_last_commit(rel)
        src = f"{rel} ({rec.get('source', 'rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE')}"
        src += f"; fetch x{rec.get('fetch_scale')}, write x{rec.get('write_scale')}"
        src += f"; commit {commit})" if commit else ")"
        return int(rec["bytes_per_call"]), src
    except (ValueError, KeyError, TypeError):
        return None, None


def _kernel_trace_us(workload_name):
    """(mean µs, provenance) rocprofv3 recorded for this configuration in the committed kernel-trace summary.

    The number comes from the committed profile (another run, on another
    box), not from this run; the provenance names the file and the commit
    its measurement was taken at (its "commit" line)."""
    rel = os.path.join("profiles", "pad_phase1_kernel_configs_kernel_trace.txt")
    path = os.path.join(REPO, rel)
    if not os.path.exists(path):
        return None, None
    us, commit = None, None
    for line in open(path):
        f = line.split()
        m = re.search(r"kernel at commit ([0-9a-f]{7,40})", line)
        if m and commit is None:
            commit = m.group(1)
        if us is None and len(f) > 3 and f[0] == workload_name:
            try:
                us = float(f[2])
            except ValueError:
                pass
    if us is None:
        return None, None
    return us, (f"{rel} (a committed rocprofv3 --kernel-trace --stats summary of another run; kernel at commit "
                f"{commit or _git_last_commit(rel) or 'unknown'})")


def _run_json(cmd, timeout=30):
    try:
        out = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
        if out.returncode != 0:
            return None
        return json.loads(out.stdout)
    except (OSError, subprocess.SubprocessError, ValueError):
        return None


def _gpu_metadata():
    """Device properties plus amd-smi's static / metric readings (each omitted if the tool does not answer)."""
    import torch

    props = torch.cuda.get_device_properties(0)
    meta = {
        "name": props.name,
        "arch": getattr(props, "gcnArchName", None),
        "compute_units": props.multi_processor_count,
        "total_memory_gib": round(props.total_memory / 2**30, 1),
        "torch": torch.__version__,
        "hip_runtime": getattr(torch.version, "hip", None),
    }
    def pick(d, *path):
        for k in path:
            if not isinstance(d, dict) or k not in d:
                return None
            d = d[k]
        return d

    static = _run_json(["amd-smi", "static", "--gpu", "0", "--json"])
    if static is not None:
        g = (static.get("gpu_data") or [{}])[0] if isinstance(static, dict) else {}
        meta["amd_smi"] = {
            "market_name": pick(g, "asic", "market_name"),
            "device_id": pick(g, "asic", "device_id"),
            "target": pick(g, "asic", "target_graphics_version"),
            "num_compute_units": pick(g, "asic", "num_compute_units"),
            "ifwi": pick(g, "ifwi", "version"),
            "driver": pick(g, "driver", "name"),
            "vram": {k: pick(g, "vram", k) for k in ("type", "vendor", "size", "max_bandwidth")},
        }
    metric = _run_json(["amd-smi", "metric", "--gpu", "0", "--json"])
    if metric is not None:
        g = (metric.get("gpu_data") or [{}])[0] if isinstance(metric, dict) else {}
        meta.setdefault("amd_smi", {})["after_run"] = {
            "socket_power": pick(g, "power", "socket_power"),
            "gfx_clk": pick(g, "clock", "gfx_0", "clk"),
            "gfx_max_clk": pick(g, "clock", "gfx_0", "max_clk"),
            "mem_clk": pick(g, "clock", "mem_0", "clk"),
            "hotspot_temp": pick(g, "temperature", "hotspot"),
            "mem_temp": pick(g, "temperature", "mem"),
        }
    return meta


def _cpu_baseline(w, seconds, gpu_out, max_threads):
    import torch

    from oracle.reference import paged_attention_decode_reference

    cores = max(1, min(len(os.sched_getaffinity(0)), max_threads))
    torch.set_num_threads(cores)
    q = w.q.float().cpu()
    k = w.k_cache.float().cpu()
    v = w.v_cache.float().cpu()
    bt = w.block_table.cpu()
    sl = w.seq_lens.cpu()
    times = []
    out = None
    t_start = time.perf_counter()
    while not times or (time.perf_counter() - t_start < seconds and len(times) < 50):
        t0 = time.perf_counter()
        out = paged_attention_decode_reference(q, k, v, bt, sl, w.scale)
        times.append(time.perf_counter() - t0)
    err = float((gpu_out.float().cpu() - out).abs().max())
    return statistics.median(times), len(times), torch.get_num_threads(), err


def _cpu_inputs(w, rows):
    """Host fp32 inputs of batch `rows` of w: only the pages those rows use, relabelled."""
    import torch

    ps = w.k_cache.shape[1]
    bt = w.block_table[rows].cpu().to(torch.long)
    sl = w.seq_lens[rows].cpu().to(torch.long)
    cols = [bt[i, :-(-int(sl[i]) // ps)] for i in range(len(rows))]
    pages = torch.unique(torch.cat(cols)) if cols else torch.zeros(0, dtype=torch.long)
    relabel = torch.full((int(pages.max()) + 1 if pages.numel() else 1,), -1, dtype=torch.long)
    relabel[pages] = torch.arange(pages.numel())
    bt_new = torch.zeros_like(bt)
    for i, c in enumerate(cols):
        bt_new[i, :c.numel()] = relabel[c]
    idx = pages.to(w.k_cache.device)
    k = w.k_cache.index_select(0, idx).float().cpu()
    v = w.v_cache.index_select(0, idx).float().cpu()
    return w.q[rows].float().cpu(), k, v, bt_new, sl


def _cpu_configs(pad, wl, specs, engine, splits, max_threads, seconds=3.0):
    """The fp32 CPU oracle next to the GPU call on several configurations.

    Per configuration: GPU seconds per call over back-to-back cold calls
    (inputs rotated as in the sweep; C5 is one 17 GB set); CPU seconds per
    call of oracle/reference.py on the host cores after one untimed call:
    the median over at least 5 calls (C1-C3) or 1 call (C4, and C5 over 8
    seeded rows, their pages only), repeated for about `seconds` per
    configuration (at most 50 calls), compared per algorithmic byte.  Every GPU timing runs before the first
    CPU call, so the oracle's worker threads never compete with the launch
    thread.  Returns (records, table text)."""
    import random

    import torch

    from oracle.reference import paged_attention_decode_reference

    staged = []
    for spec in specs:
        name, _, b = spec.partition(":")
        batch = int(b) if b else None
        w = wl.make(name, batch=batch, seed=3000)
        n_sets = 1 if name == "C5" else _rotation(w.k_cache.numel() * 4)
        sets = [w] + [wl.make(name, batch=batch, seed=3000 + i) for i in range(1, n_sets)]
        calls = 10 if name == "C5" else 200
        # The first pass brings the clocks up after the inputs were made; the second is kept.
        _throughput(pad, sets, engine, splits, calls, 5 if name == "C5" else 20)
        gpu_s = _throughput(pad, sets, engine, splits, calls, 5 if name == "C5" else 20)
        del sets[1:]
        if name == "C5":
            rows = sorted(random.Random(3000).sample(range(w.batch), 8))
            runs, sample = 1, "8 seeded rows, their pages only"
        else:
            rows = list(range(w.batch))
            runs, sample = (1, "whole batch") if name == "C4" else (5, "whole batch")
        gpu_rows = _call(pad, w, engine, splits)[rows].float().cpu()
        staged.append((spec, w.scale, wl.bytes_of(w), dict(w.shape), w.k_cache.shape[1], gpu_s, gpu_rows, runs,
                       sample, _cpu_inputs(w, rows)))
        del w
        torch.cuda.empty_cache()
    cores = max(1, min(len(os.sched_getaffinity(0)), max_threads))
    torch.set_num_threads(cores)
    recs = []
    for spec, scale, nb_gpu, shape, ps, gpu_s, gpu_rows, runs, sample, (q, k, v, bt, sl) in staged:
        paged_attention_decode_reference(q, k, v, bt, sl, scale)  # untimed: first-touch of its buffers
        times, out = [], None
        t_start = time.perf_counter()
        while len(times) < runs or (time.perf_counter() - t_start < seconds and len(times) < 50):
            t0 = time.perf_counter()
            out = paged_attention_decode_reference(q, k, v, bt, sl, scale)
            times.append(time.perf_counter() - t0)
        cpu_s = statistics.median(times)
        hkv, hq, d = shape["num_kv_heads"], shape["num_q_heads"], shape["head_dim"]
        lens = sl.tolist()
        nb_cpu = (sum(lens) * hkv * d * 4 + 4 * len(lens) * hq * d + sum(-(-n // ps) for n in lens) * 4
                  + 4 * len(lens))
        recs.append({"config": spec, "gpu_us_per_call": round(gpu_s * 1e6, 2),
                     "gpu_gbs": round(nb_gpu / gpu_s / 1e9, 1), "cpu_ms_per_call": round(cpu_s * 1e3, 2),
                     "cpu_gbs": round(nb_cpu / cpu_s / 1e9, 3), "cpu_calls": len(times), "cpu_sample": sample,
                     "cpu_threads": torch.get_num_threads(),
                     "gpu_over_cpu": round(nb_gpu / gpu_s / (nb_cpu / cpu_s), 1),
                     "max_abs_err": float((gpu_rows - out).abs().max())})
    lines = [f"{'config':8s} {'GPU us/call':>12s} {'GPU GB/s':>9s} {'CPU ms/call':>12s} {'CPU GB/s':>9s} "
             f"{'GPU/CPU':>8s} {'max|err|':>9s}  CPU sample (calls, threads)"]
    for r in recs:
        lines.append(f"{r['config']:8s} {r['gpu_us_per_call']:12.2f} {r['gpu_gbs']:9.1f} {r['cpu_ms_per_call']:12.2f} "
                     f"{r['cpu_gbs']:9.3f} {r['gpu_over_cpu']:8.1f} {r['max_abs_err']:9.1e}  {r['cpu_sample']} "
                     f"({r['cpu_calls']}, {r['cpu_threads']})")
    return recs, "\n".join(lines)


def main():
    args = _parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} (WORLD_SIZE {world}) is not supported. "
              "The decode path shards by batch or KV head with no exchange; run one process per GPU instead.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import paged_attention_decode_amd as pad
    from paged_attention_decode_amd import workloads as wl

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    engine = args.engine
    splits = args.num_splits

    # Headline: C2 at --batch, rotated KV caches (cold).
    probe = wl.make("C2", batch=args.batch, seed=1000)
    one_set = probe.k_cache.numel() * 4
    n_sets = _rotation(one_set)
    sets = [probe] + _make_sets(wl.make, n_sets - 1, name="C2", batch=args.batch)
    nbytes = wl.bytes_of(probe)
    shp = probe.shape
    plan = pad.plan(shp["batch"], shp["num_q_heads"], shp["num_kv_heads"], shp["head_dim"], shp["page_size"],
                    shp["max_pages"], splits)

    torch.cuda.synchronize()
    wall = []
    sec = _throughput(pad, sets, engine, splits, args.steps, args.warmup, wall)
    value = nbytes / sec / 1e9
    trace_us, trace_src = _kernel_trace_us(probe.name)
    traffic, traffic_src = _traffic(probe.name)

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 q/K/V and output, fp32 accumulation; P rounded to fp16 for the PV MFMA",
        "data": "synthetic (seeded N(0,1) fp16, shuffled block tables)",
        "config": {
            "workload": f"C2: batch {args.batch}, seq_len 4096, GQA 12/2, head_dim 128, page 16; "
                        f"cold (calls rotate over {n_sets} KV caches)",
            "batch": args.batch,
            "seq_len": 4096,
            "num_q_heads": 12,
            "num_kv_heads": 2,
            "head_dim": 128,
            "page_size": 16,
            "num_splits": plan["num_splits"],
            "pages_per_split": plan["pages_per_split"],
            "waves_per_group": plan["waves_per_group"],
            "engine": "mfma" if engine == 0 else "valu",
            "algorithmic_bytes_per_call": nbytes,
        },
        "pct_of_peak": round(100.0 * value / PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": "pad_phase1_kernel",
            "achieved": round(value, 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(value / PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "fetch_gbs": round(traffic / sec / 1e9, 1) if traffic else None,
            "us_per_call": round(sec * 1e6, 3),
            "kernel_trace_us_committed": trace_us,
            "kernel_trace_source": trace_src,
            "timed_region_wall_s": round(wall[0], 6),
        },
    }
    if not args.no_ceiling:
        from paged_attention_decode_amd import roofline as rl

        paged_gbs, stream_gbs, details = rl.ceilings(sets, calls=max(20, args.steps // 2))
        result["roofline"]["measured_ceiling_gbs"] = round(paged_gbs, 1)
        result["roofline"]["frac_of_measured_ceiling"] = round(value / paged_gbs, 4)
        result["roofline"]["contiguous_stream_gbs"] = round(stream_gbs, 1)
        result["roofline"]["ceiling_probe"] = details
    del sets

    if not args.no_ragged:
        first = wl.make("C3", seed=1000)
        rs = [first] + [wl.make("C3", seed=1000 + i) for i in range(1, _rotation(first.k_cache.numel() * 4))]
        calls = args.sweep_calls
        dense = _throughput(pad, rs, engine, splits, calls, 20)
        csr_args = [pad.paged_kv_indices(w.block_table, w.seq_lens, w.k_cache.shape[1]) for w in rs]
        for i in range(10):
            j = i % len(rs)
            pad.paged_attention_decode_csr(rs[j].q, rs[j].k_cache, rs[j].v_cache, *csr_args[j])
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s_ev.record()
        for i in range(calls):
            j = i % len(rs)
            pad.paged_attention_decode_csr(rs[j].q, rs[j].k_cache, rs[j].v_cache, *csr_args[j])
        e_ev.record()
        torch.cuda.synchronize()
        csr = s_ev.elapsed_time(e_ev) / 1e3 / calls
        nb3 = sum(wl.bytes_of(w) for w in rs) / len(rs)
        planned = _throughput_planned(pad, rs, splits, calls, 20) if engine == 0 else None
        result["c3_ragged"] = {
            "workload": "C3: batch 32, seq_lens U[1, 8192], GQA 12/2, head_dim 128, page 32; cold "
                        f"(rotation over {len(rs)} seeded batches)",
            "us_per_call_dense": round(dense * 1e6, 2),
            "gbs_dense": round(nb3 / dense / 1e9, 1),
            "pct_of_peak_dense": round(100 * nb3 / dense / 1e9 / PEAK_GBS, 2),
            "us_per_call_csr": round(csr * 1e6, 2),
            "gbs_csr": round(nb3 / csr / 1e9, 1),
        }
        if planned:
            result["c3_ragged"].update({
                "us_per_call_planned": round(planned * 1e6, 2),
                "gbs_planned": round(nb3 / planned / 1e9, 1),
                "pct_of_peak_planned": round(100 * nb3 / planned / 1e9 / PEAK_GBS, 2),
            })
        del rs, csr_args

    if not args.no_fp8 and engine == 0:
        # The headline step over fp8 caches (same C2 inputs converted, one byte
        # per K/V element): not the metric, which is quoted on fp16 caches.
        fp8 = {}
        for fmt, dt in wl.FP8_NAMES.items():
            first = wl.to_fp8(wl.make("C2", batch=args.batch, seed=1000), dt)
            rs = [first] + [wl.to_fp8(wl.make("C2", batch=args.batch, seed=1000 + i), dt)
                            for i in range(1, _rotation(first.k_cache.numel() * 2))]
            t8 = _throughput(pad, rs, engine, splits, args.steps, args.warmup)
            nb8 = wl.bytes_of(first)
            w1 = wl.to_fp8(wl.make("C2", batch=1, seed=2001), dt)
            lat1, _ = _latency_reference_method(pad, w1, engine, splits, max(3, args.trials // 3))
            fp8[fmt] = {
                "us_per_call_cold": round(t8 * 1e6, 2),
                "gbs_cold": round(nb8 / t8 / 1e9, 1),
                "pct_of_peak_cold": round(100 * nb8 / t8 / 1e9 / PEAK_GBS, 2),
                "algorithmic_bytes_per_call": nb8,
                "speedup_vs_fp16_headline": round(sec / t8, 3),
                "b1_us_per_call_warm": round(lat1, 2),
            }
            del rs, first, w1
        # bfloat16 q, caches and output: the same bytes as the fp16 step.
        first = wl.to_bf16(wl.make("C2", batch=args.batch, seed=1000))
        rs = [first] + [wl.to_bf16(wl.make("C2", batch=args.batch, seed=1000 + i))
                        for i in range(1, _rotation(first.k_cache.numel() * 4))]
        tb = _throughput(pad, rs, engine, splits, args.steps, args.warmup)
        result["c2_bf16"] = {
            "workload": f"C2 batch {args.batch} in bfloat16 (q, caches, output); cold rotation",
            "us_per_call_cold": round(tb * 1e6, 2),
            "gbs_cold": round(wl.bytes_of(first) / tb / 1e9, 1),
            "pct_of_peak_cold": round(100 * wl.bytes_of(first) / tb / 1e9 / PEAK_GBS, 2),
            "time_vs_fp16_headline": round(tb / sec, 3),
        }
        del rs, first
        result["c2_fp8"] = {
            "workload": f"C2 batch {args.batch} with fp8 K/V caches (per-tensor scales, codes spanning 7/8 of the "
                        "range); cold rotation; q and output fp16",
            **fp8,
        }

    if not args.no_sweep:
        sweep = {}
        for b in wl.C2_BATCHES:
            w = wl.make("C2", batch=b, seed=2000 + b)
            lat, lat_samples = _latency_reference_method(pad, w, engine, splits, args.trials)
            rs = [w] + _make_sets(wl.make, _rotation(w.k_cache.numel() * 4) - 1, name="C2", batch=b)
            cold = _throughput(pad, rs, engine, splits, args.sweep_calls, 20)
            nb = wl.bytes_of(w)
            sweep[str(b)] = {
                "us_per_call_warm": round(lat, 2),
                "us_per_call_warm_trials": [round(x, 2) for x in lat_samples],
                "us_per_call_cold_throughput": round(cold * 1e6, 2),
                "gbs_cold": round(nb / cold / 1e9, 1),
                "pct_of_peak_cold": round(100 * nb / cold / 1e9 / PEAK_GBS, 2),
            }
            if engine == 0:
                cold_p = _throughput_planned(pad, rs, splits, args.sweep_calls, 20)
                sweep[str(b)]["us_per_call_cold_planned"] = round(cold_p * 1e6, 2)
                sweep[str(b)]["pct_of_peak_cold_planned"] = round(100 * nb / cold_p / 1e9 / PEAK_GBS, 2)
            del rs, w
        result["c2_sweep"] = sweep

    # Before the headline's CPU baseline: its timings are all GPU ones first.
    if args.cpu_configs and args.cpu_configs != "none" and not args.no_cpu:
        recs, table = _cpu_configs(pad, wl, [s for s in args.cpu_configs.split(",") if s], engine, splits,
                                   args.cpu_threads)
        result["cpu_baseline_configs"] = recs
        print(table, file=sys.stderr, flush=True)
    if not args.no_cpu:
        gpu_out = _call(pad, probe, engine, splits)
        torch.cuda.synchronize()
        med, n, threads, err = _cpu_baseline(probe, args.cpu_seconds, gpu_out, args.cpu_threads)
        result["cpu_baseline"] = {
            "value": round(nbytes / med / 1e9, 3),
            "unit": "GB/s",
            "cores": threads,
            "kind": "port",
            "sample": f"oracle/reference.py fp32 on the headline C2 batch-{args.batch} inputs, "
                      f"{n} full call(s), median {med * 1e3:.1f} ms/call, torch threads {threads}",
            "ms_per_call": round(med * 1e3, 2),
            "gpu_vs_cpu_max_abs_err": err,
        }
    result["host"] = {
        "os_cpu_count": os.cpu_count(),
        "affinity_cores": len(os.sched_getaffinity(0)),
        "cpu_baseline_threads": result.get("cpu_baseline", {}).get("cores"),
        "why_capped": f"a GPU box grants one GPU {args.cpu_threads} cores (OMP_NUM_THREADS={os.environ.get('OMP_NUM_THREADS')})",
    }
    result["gpu"] = _gpu_metadata()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()

"""A short, fixed workload to run under rocprofv3.

    python -m paged_attention_decode_amd.profile_run --config C2 --batch 64 --calls 50

``--shape B/HQ/HKV/D/L[/PS]`` replaces the configuration by B sequences of L
tokens (page size PS, default 16) with HQ / HKV heads of head_dim D.
``--tp N`` / ``--sp N`` run one GPU's share of the configuration when it is
sharded over N GPUs by kv heads or by ranges of each sequence's pages
(workloads.make).

Runs a calibration copy first (``--copy-mb`` MiB read and written by
PyTorch's copy kernel, 3 dispatches: the bytes a FETCH_SIZE / WRITE_SIZE
counter should report for a plain stream of known size), then ``--calls``
decode calls of the named configuration, rotating over enough distinct KV
caches that the 256 MB Infinity Cache cannot serve repeats ("cold"), or on
one set of inputs with ``--warm``.  Prints the per-call algorithmic bytes.

``--kv e4m3fn`` (or ``e5m2``) converts every input set's caches to fp8
(workloads.to_fp8) and calls ``paged_attention_decode_fp8``; the printed
algorithmic bytes then count one byte per K/V element.  ``--kv bf16``
rounds q and the caches to bfloat16 (workloads.to_bf16) and calls
``paged_attention_decode_ex``.  With an fp8 ``--kv``, ``--q bf16`` rounds q
to bfloat16 (fp8 caches with bf16 q and output).

``--planned`` plans every input set once with ``BatchDecodeWrapper``
(the work-list planner kernel, one dispatch per set, before the timed
calls) and then makes the ``--calls`` decode calls through ``run()``.

``--timeline`` instead runs each configuration of ``--configs`` (e.g.
``C2:16,C2:32,C3``) through ``libpa_decode_tl.so`` (the decode library with
per-workgroup phase stamps) in groups of 4 back-to-back cold launches and
prints the median per-phase budget (timeline.py), one line per
configuration; ``--json`` also writes the table as JSON.
"""

from __future__ import annotations

import argparse
import json
import math

import torch

from . import paged_attention_decode_ex, paged_attention_decode_fp8
from . import workloads as wl


def _sets(make, warm: bool):
    w0 = make(1)
    n_sets = 1 if warm else max(2, math.ceil(512 * (1 << 20) / (w0.k_cache.numel() * 4)) + 1)
    return [w0] + [make(1 + i) for i in range(1, n_sets)]


def run_timeline(a) -> None:
    from . import timeline as tl

    rows = {}
    cols = ("span", "gap", "dispatch", "item", "loop", "loop_tail", "publish", "arrive", "merge", "exit_tail")
    print("timeline budget, us (medians over %d groups of 4 back-to-back cold launches)" % a.repeats, flush=True)
    print(f"{'config':8s} {'grid':>6s} {'S':>3s} {'nw':>3s} " + " ".join(f"{c:>9s}" for c in cols), flush=True)
    for cfg in a.configs.split(","):
        name, _, b = cfg.partition(":")
        batch = int(b) if b else None
        sets = _sets(lambda seed: wl.make(name, batch=batch, seed=seed), a.warm)
        outs = [torch.empty_like(w.q) for w in sets]
        recs, groups, plan = tl.record(sets, outs, a.num_splits, a.engine, repeats=a.repeats)
        med = tl.median_budget(recs)
        xcc = sorted(set(x for r in recs for x in r["xcc_ids"]))
        rows[cfg] = {"grid": groups, "num_splits": plan.num_splits, "waves": plan.waves_per_group, **med,
                     "xcc_ids_seen": xcc}
        fmt = lambda v: f"{v:9.2f}" if v is not None else f"{'-':>9s}"
        print(f"{cfg:8s} {groups:6d} {plan.num_splits:3d} {plan.waves_per_group:3d} "
              + " ".join(fmt(med[c]) for c in cols), flush=True)
        del sets, outs
        torch.cuda.empty_cache()
    if a.json:
        with open(a.json, "w") as f:
            json.dump(rows, f, indent=1)


def main() -> None:
    p = argparse.ArgumentParser()
    p.add_argument("--config", default="C2", choices=["C1", "C2", "C3", "C4", "C5"])
    p.add_argument("--batch", type=int, default=64)
    p.add_argument("--calls", type=int, default=50)
    p.add_argument("--engine", type=int, default=0)
    p.add_argument("--num-splits", type=int, default=0)
    p.add_argument("--copy-mb", type=int, default=256)
    p.add_argument("--warm", action="store_true")
    p.add_argument("--shape", default="", help="B/HQ/HKV/D/L[/PS]: uniform lengths instead of --config")
    p.add_argument("--tp", type=int, default=1, help="--config: one GPU's share over N GPUs by kv heads")
    p.add_argument("--sp", type=int, default=1, help="--config: one GPU's share over N GPUs by page ranges")
    p.add_argument("--timeline", action="store_true", help="per-phase budget from libpa_decode_tl.so")
    p.add_argument("--configs", default="C2:16,C2:32,C2:64,C3,C4", help="--timeline: configurations")
    p.add_argument("--repeats", type=int, default=8, help="--timeline: groups of 4 launches")
    p.add_argument("--json", default="", help="--timeline: write the table here")
    p.add_argument("--kv", default="fp16", choices=["fp16", "bf16", "e4m3fn", "e5m2"], help="q/K/V format")
    p.add_argument("--q", default="fp16", choices=["fp16", "bf16"], help="q format with fp8 caches")
    p.add_argument("--planned", action="store_true",
                   help="plan every input set once (BatchDecodeWrapper), then time only run() calls")
    a = p.parse_args()
    if a.timeline:
        run_timeline(a)
        return

    if a.copy_mb > 0:
        n = a.copy_mb * (1 << 20) // 2
        src = torch.randn(n, device="cuda", dtype=torch.float16)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"calibration copy: {a.copy_mb} MiB read + {a.copy_mb} MiB written per dispatch", flush=True)
        del src, dst

    if a.shape:
        f = [int(x) for x in a.shape.split("/")]
        b, hq, hkv, d, seq = f[:5]
        ps = f[5] if len(f) > 5 else 16

        def make(seed):
            return wl._build(f"shape {a.shape}", [seq] * b, hq, hkv, d, ps, seed, "cuda")
    else:
        def make(seed):
            return wl.make(a.config, batch=a.batch, seed=seed, tp=a.tp, sp=a.sp)
    if a.kv != "fp16":
        assert not a.planned, "--planned runs fp16 caches"
        make16 = make

        def make(seed):
            if a.kv == "bf16":
                return wl.to_bf16(make16(seed))
            w8 = wl.to_fp8(make16(seed), wl.FP8_NAMES[a.kv])
            if a.q == "bf16":
                w8.q = w8.q.bfloat16()
            return w8
    sets = _sets(make, a.warm)
    w0, n_sets = sets[0], len(sets)
    wraps = []
    if a.planned:
        from . import BatchDecodeWrapper

        for w in sets:
            pw = BatchDecodeWrapper()
            sh = w.shape
            pw.plan_block_table(w.block_table, w.seq_lens, sh["num_q_heads"], sh["num_kv_heads"], sh["head_dim"],
                                sh["page_size"], num_splits=a.num_splits or None)
            wraps.append(pw)
    torch.cuda.synchronize()
    for i in range(a.calls):
        w = sets[i % n_sets]
        if a.planned:
            wraps[i % n_sets].run(w.q, (w.k_cache, w.v_cache))
        elif a.kv in ("e4m3fn", "e5m2"):
            paged_attention_decode_fp8(*w.args(), k_scale=w.k_scale, v_scale=w.v_scale,
                                       num_splits=a.num_splits or None)
        else:
            paged_attention_decode_ex(*w.args(), num_splits=a.num_splits or None, engine=a.engine)
    torch.cuda.synchronize()
    used = [sets[i % n_sets] for i in range(a.calls)]
    mean_bytes = sum(wl.bytes_of(w) for w in used) / len(used)
    print(f"{w0.name}: {a.calls} calls over {n_sets} input set(s); algorithmic bytes/call {wl.bytes_of(w0)} "
          f"(first set), {mean_bytes:.0f} (mean over the calls)", flush=True)


if __name__ == "__main__":
    main()

"""Per-phase time budget of the decode kernel from its timeline stamps.

``libpa_decode_tl.so`` (the decode library compiled with ``-DPAD_TIMELINE``,
include/pa_decode_timeline.h) has thread 0 of every workgroup store
``s_memrealtime`` stamps (100 MHz) at fixed points of its path, for a ring of
the last 4 launches.  :func:`record` runs back-to-back launches through that
library and returns the stamps; :func:`phases` turns one group of launches
into the budget that explains a call's time:

* ``gap``: last workgroup exit of one launch -> first workgroup entry of
  the next (back-to-back launches on one stream);
* ``dispatch``: first -> last workgroup entry of a launch;
* ``item``: entry -> work item known (median over workgroups with an item);
* ``loop``: item known -> every wave's streaming loop done (median);
* ``loop_tail``: median -> latest loop end over the launch;
* ``publish`` / ``arrive`` / ``merge``: for the workgroups that merged a
  unit (its last arrival): loop end -> partial stores complete, -> arrival
  atomic returned, -> merged output written (medians);
* ``exit_tail``: latest loop end -> latest workgroup exit;
* ``span``: first entry -> last exit.

The reference kept its phase-1 / phase-2 split from Nsight Compute
(profiles/notes.md:848-883 of the reference); this is the same budget for
the fused kernel.  Measurement tooling only: the decode path never loads
the timeline library.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _native

TICK_US = 0.01  # s_memrealtime runs at 100 MHz

PHASES = ("span", "gap", "dispatch", "item", "loop", "loop_tail", "publish", "arrive", "merge", "exit_tail")


def _us(x):
    return float(x) * TICK_US


def phases(stamps: np.ndarray, groups: int, order) -> list[dict]:
    """Budget of each launch in ``order`` (ring entries in launch order) over its first ``groups`` rows.

    ``stamps`` is the raw buffer viewed as ``[launches, max_groups, slots]`` int64.
    """
    out = []
    prev_exit = None
    for k in order:
        r = stamps[k, :groups]
        entry = r[:, _native.TL_ENTRY]
        exit_ = r[:, _native.TL_EXIT]
        info = r[:, _native.TL_INFO]
        flags = (info >> 40) & 0xFF
        has_item = (flags & _native.TL_F_NO_ITEM) == 0
        rec = {}
        t0 = entry.min()
        last_exit = exit_.max()
        rec["span"] = _us(last_exit - t0)
        rec["gap"] = None if prev_exit is None else _us(t0 - prev_exit)
        prev_exit = last_exit
        rec["dispatch"] = _us(entry.max() - t0)
        item = r[has_item, _native.TL_ITEM] - entry[has_item]
        rec["item"] = _us(np.median(item)) if item.size else None
        loop_end = r[has_item, _native.TL_LOOP_END]
        ok = loop_end > 0
        loop = loop_end[ok] - r[has_item, _native.TL_ITEM][ok]
        rec["loop"] = _us(np.median(loop)) if loop.size else None
        rec["loop_tail"] = _us(loop_end[ok].max() - np.median(loop_end[ok])) if loop.size else None
        merger = (flags & _native.TL_F_MERGER) != 0
        if merger.any():
            m = r[merger]
            rec["publish"] = _us(np.median(m[:, _native.TL_PUBLISHED] - m[:, _native.TL_LOOP_END]))
            rec["arrive"] = _us(np.median(m[:, _native.TL_ARRIVED] - m[:, _native.TL_PUBLISHED]))
            rec["merge"] = _us(np.median(m[:, _native.TL_MERGED] - m[:, _native.TL_ARRIVED]))
        else:
            rec["publish"] = rec["arrive"] = rec["merge"] = None
        rec["exit_tail"] = _us(last_exit - loop_end[ok].max()) if loop.size else None
        rec["xcc_ids"] = sorted(set(int(x) for x in ((info[has_item] >> 32) & 0xF)))
        out.append(rec)
    return out


def median_budget(records: list[dict]) -> dict:
    """Median of each phase over launches (``gap`` over the launches that have one)."""
    res = {}
    for p in PHASES:
        vals = [r[p] for r in records if r.get(p) is not None]
        res[p] = round(float(np.median(vals)), 2) if vals else None
    return res


def record(sets, outs, num_splits: int = 0, engine: int = 0, repeats: int = 8, warmup: int = 20):
    """Run ``repeats`` groups of 4 back-to-back launches through libpa_decode_tl.so; per-launch budgets."""
    import torch

    lib = _native.timeline()
    dims = [_native.dims_for(*w.args(), o) for w, o in zip(sets, outs)]
    ws_need, cnt_need = 0, 0
    for d in dims:
        ws = ctypes.c_size_t()
        nc = ctypes.c_int64()
        assert lib.pad_decode_workspace_bytes(ctypes.byref(d), num_splits, 0, ctypes.byref(ws)) == 0
        assert lib.pad_decode_counters_needed(ctypes.byref(d), num_splits, 0, ctypes.byref(nc)) == 0
        ws_need, cnt_need = max(ws_need, ws.value), max(cnt_need, nc.value)
    wsb = torch.empty(max(ws_need, 256), dtype=torch.uint8, device="cuda")
    cnt = torch.zeros(max(cnt_need, 1), dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    plan = _native.PadPlan()
    assert lib.pad_decode_plan(ctypes.byref(dims[0]), num_splits, 0, ctypes.byref(plan)) == 0
    s0 = sets[0].shape
    groups = plan.num_splits * s0["num_kv_heads"] * s0["batch"]
    assert groups <= _native.TL_MAX_GROUPS, "grid larger than the timeline buffer"

    def call(i):
        j = i % len(sets)
        w = sets[j]
        st = lib.pad_decode_launch_ex(w.q.data_ptr(), w.k_cache.data_ptr(), w.v_cache.data_ptr(),
                                      w.block_table.data_ptr(), w.seq_lens.data_ptr(), outs[j].data_ptr(),
                                      wsb.data_ptr(), wsb.numel(), cnt.data_ptr(), cnt.numel(), ctypes.byref(dims[j]),
                                      ctypes.c_float(w.scale), num_splits, engine, None, stream)
        assert st == 0, st

    n = _native.TL_LAUNCHES
    buf = (ctypes.c_uint64 * (n * _native.TL_MAX_GROUPS * _native.TL_SLOTS))()
    records = []
    i = 0
    for _ in range(repeats):
        for _ in range(warmup):
            call(i)
            i += 1
        torch.cuda.synchronize()
        assert lib.pad_timeline_reset() == 0
        for _ in range(n):
            call(i)
            i += 1
        torch.cuda.synchronize()
        assert lib.pad_timeline_read(buf, ctypes.sizeof(buf)) == 0
        a = np.frombuffer(buf, dtype=np.uint64).astype(np.int64).reshape(n, _native.TL_MAX_GROUPS, _native.TL_SLOTS)
        records.extend(phases(a, groups, range(n)))
    return records, groups, plan

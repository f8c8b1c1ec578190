"""CPU checks of bench.py's host-side logic (no GPU).

``_cpu_inputs`` copies only the pages a subset of batch rows uses and
relabels their block-table columns onto that compact page set, so the CPU
baseline on C5 never upcasts the whole 17 GB cache.  The relabelled inputs
must decode exactly as the full ones do for those rows.
"""

from __future__ import annotations

import importlib.util
import os

import torch

from oracle.reference import paged_attention_decode_reference
from paged_attention_decode_amd import workloads as wl

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(REPO, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_row_subset_inputs_decode_like_the_full_batch():
    bench = _bench()
    w = wl.make("C3", seed=7, device="cpu")  # ragged lengths, page 32, shuffled table
    rows = [0, 5, 17, 31]
    q, k, v, bt, sl = bench._cpu_inputs(w, rows)
    used = sum(-(-int(w.seq_lens[r]) // w.k_cache.shape[1]) for r in rows)
    assert k.shape[0] == len(torch.unique(torch.cat(
        [w.block_table[r, :-(-int(w.seq_lens[r]) // w.k_cache.shape[1])] for r in rows]))) <= used
    assert torch.equal(sl, w.seq_lens[rows].to(torch.long))
    sub = paged_attention_decode_reference(q, k, v, bt, sl, w.scale)
    full = paged_attention_decode_reference(w.q.float(), w.k_cache.float(), w.v_cache.float(), w.block_table,
                                            w.seq_lens, w.scale)
    torch.testing.assert_close(sub, full[rows], rtol=0, atol=0)


def test_row_subset_with_an_empty_row():
    bench = _bench()
    w = wl.make("C2", batch=3, seed=8, device="cpu")
    w.seq_lens[1] = 0
    q, k, v, bt, sl = bench._cpu_inputs(w, [0, 1])
    out = paged_attention_decode_reference(q, k, v, bt, sl, w.scale)
    assert torch.all(out[1] == 0)
    full = paged_attention_decode_reference(w.q.float(), w.k_cache.float(), w.v_cache.float(), w.block_table,
                                            w.seq_lens, w.scale)
    torch.testing.assert_close(out[0], full[0], rtol=0, atol=0)


def test_committed_kernel_trace_is_labelled_with_its_source():
    bench = _bench()
    us, src = bench._kernel_trace_us("C2_b64")
    assert us is not None and us > 0
    assert "profiles/pad_phase1_kernel_configs_kernel_trace.txt" in src and "commit" in src
    assert bench._kernel_trace_us("no_such_config") == (None, None)


def test_per_config_cpu_baseline_is_on_by_default():
    import sys

    bench = _bench()
    argv = sys.argv
    try:
        sys.argv = ["bench.py"]
        args = bench._parse()
    finally:
        sys.argv = argv
    assert set(args.cpu_configs.split(",")) >= {"C1", "C3", "C4"}


def test_fp8_workload_conversion():
    # to_fp8 keeps the inputs, stores K / k_scale and V / v_scale as fp8 codes
    # that span the format's range, and counts one byte per K/V element.
    import torch

    w = wl.make("C2", batch=2, seed=3, device="cpu")
    for name, dt in wl.FP8_NAMES.items():
        w8 = wl.to_fp8(w, dt)
        assert w8.k_cache.dtype == dt and w8.v_cache.dtype == dt and w8.name.endswith(name)
        assert w8.q is w.q and w8.block_table is w.block_table
        top = float(w8.k_cache.float().abs().max())
        assert abs(top - 0.875 * wl.FP8_MAX[dt]) <= 0.07 * wl.FP8_MAX[dt]
        deq = w8.k_cache.float() * w8.k_scale
        rel = 2.0 ** -3 if name == "e4m3fn" else 2.0 ** -2  # half an ulp of a 3- / 2-bit mantissa
        big = w.k_cache.float().abs() > 0.1
        assert torch.all((deq - w.k_cache.float()).abs()[big] <= rel / 2 * w.k_cache.float().abs()[big] + 1e-6)
        kv16 = 2 * 4096 * 2 * 128 * 2 * 2  # batch x seq x kv heads x head_dim x fp16 x (K, V)
        assert wl.bytes_of(w) - wl.bytes_of(w8) == kv16 // 2


def test_shard_shares_of_a_configuration():
    # One GPU's share of a sharded configuration (workloads.make tp= / sp=).
    # Page ranges: counting every token of a sequence onto GPU (t // ps) // c,
    # with c = ceil(pages / sp) pages per GPU, gives GPU 0's share, and the
    # shares of all GPUs add up to the sequence.
    g = torch.Generator().manual_seed(0)
    for _ in range(200):
        n = int(torch.randint(1, 5000, (1,), generator=g))
        ps = int(torch.randint(1, 40, (1,), generator=g))
        sp = int(torch.randint(1, 10, (1,), generator=g))
        c = -(-(-(-n // ps)) // sp)
        owner = [(t // ps) // c for t in range(n)]
        assert wl.shard_lens([n], ps, sp) == [owner.count(0)]
        assert sum(owner.count(i) for i in range(sp)) == n and max(owner) < sp
    # kv heads: 1/tp of the heads with the same lengths, 1/tp of the K/V bytes.
    full, share = wl.make("C2", batch=4, seed=5, device="cpu"), wl.make("C2", batch=4, seed=5, device="cpu", tp=2)
    assert share.q.shape == (4, 6, 128) and share.k_cache.shape[2] == 1 and share.name == "C2_b4_tp2"
    assert torch.equal(share.seq_lens, full.seq_lens)
    kv = lambda w: w.k_cache[0, 0].numel() * 2 * 2 * int(w.seq_lens.sum())  # noqa: E731  (K, V) fp16
    assert kv(full) == 2 * kv(share)
    c4 = wl.make("C4", device="cpu", sp=8)
    assert c4.seq_lens.tolist() == [16384] and c4.block_table.shape == (1, 1024) and c4.q.shape == (1, 32, 128)
    c3 = wl.make("C3", seed=2, device="cpu", sp=2)
    assert c3.block_table.shape[1] == 128 and all(0 < n <= 4096 for n in c3.seq_lens.tolist())
    # no sharding: the configuration itself
    assert torch.equal(wl.make("C1", seed=4, device="cpu", tp=1, sp=1).k_cache, wl.make("C1", seed=4, device="cpu").k_cache)
    for bad in ({"tp": 3}, {"tp": 0}, {"sp": 0}):
        try:
            wl.make("C2", batch=1, device="cpu", **bad)
        except ValueError:
            continue
        raise AssertionError(bad)

"""Seeded synthetic inputs for the benchmark configurations, built on the GPU.

Configurations (all fp16 N(0,1) q/K/V, scale 1/sqrt(head_dim), pages handed
out by one seeded global shuffle so physical pages are non-contiguous across
and within sequences; unused block_table columns point at valid pages):

* ``C1`` batch 1, 12 Q / 2 KV heads, head_dim 128, page 16, seq_len 1024.
* ``C2`` the same GQA shape, every seq_len 4096, batch from the sweep
  {1, 2, 4, 8, 16, 32, 64}.
* ``C3`` batch 32, 12/2, page 32, seq_lens uniform in [1, 8192] with one
  forced to 1 and several not multiples of 32; two keys per sequence
  scaled x8 (every kv head) to stress the softmax range.
* ``C4`` batch 1, 32 Q / 8 KV heads, page 16, seq_len 131072.
* ``C5`` batch 256, 64 Q / 8 KV heads, page 16, seq_lens uniform in
  [512, 32768] (about 17 GB of fp16 K+V).

``algorithmic_bytes`` is the byte count the roofline uses: K and V of every
valid token, the q read and the output write, the block_table entries of the
used pages and seq_lens (the split workspace is excluded as overhead).

``make(..., tp=N)`` and ``make(..., sp=N)`` build one GPU's share of a
configuration sharded over N GPUs, by kv heads or by ranges of each
sequence's pages.

``to_bf16`` rounds q and the caches to bfloat16.  ``to_fp8`` turns a
workload's caches into fp8 codes (float8_e4m3fn or
float8_e5m2) of K / k_scale and V / v_scale, per-tensor scales chosen so the
largest magnitude lands at 7/8 of the format's range; its algorithmic bytes
count one byte per K/V element.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

C2_BATCHES = (1, 2, 4, 8, 16, 32, 64)


@dataclass
class Workload:
    name: str
    q: torch.Tensor
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    block_table: torch.Tensor
    seq_lens: torch.Tensor
    seq_lens_host: list = field(default_factory=list)
    scale: float = 0.0
    k_scale: float = 1.0  # fp8 caches: they hold K / k_scale and V / v_scale
    v_scale: float = 1.0

    @property
    def batch(self) -> int:
        return self.q.shape[0]

    @property
    def shape(self) -> dict:
        b, hq, d = self.q.shape
        p, ps, hkv, _ = self.k_cache.shape
        return dict(batch=b, num_q_heads=hq, num_kv_heads=hkv, head_dim=d, page_size=ps,
                    max_pages=self.block_table.shape[1], num_pages=p)

    def args(self):
        return self.q, self.k_cache, self.v_cache, self.block_table, self.seq_lens


def algorithmic_bytes(seq_lens, num_q_heads, num_kv_heads, head_dim, page_size, kv_elem_bytes=2) -> int:
    """K+V of valid tokens + q read + out write + used block_table entries + seq_lens."""
    lens = [int(x) for x in seq_lens]
    kv = sum(lens) * num_kv_heads * head_dim * kv_elem_bytes * 2
    qo = 2 * len(lens) * num_q_heads * head_dim * 2
    bt = sum(-(-n // page_size) for n in lens) * 4
    return kv + qo + bt + 4 * len(lens)


def algorithmic_flops(seq_lens, num_q_heads, head_dim) -> int:
    return 4 * num_q_heads * head_dim * sum(int(x) for x in seq_lens)


def _build(name, lens, hq, hkv, d, ps, seed, device, max_pages=None, key_boost=0):
    g_cpu = torch.Generator().manual_seed(seed)
    pages = [-(-n // ps) for n in lens]
    width = max_pages if max_pages is not None else max(max(pages), 1)
    total = sum(pages)
    num_pages = max(total, 1)
    perm = torch.randperm(num_pages, generator=g_cpu).to(torch.int32)
    bt = torch.empty(len(lens), width, dtype=torch.int32)
    cur = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[cur:cur + n]
        if n < width:
            bt[b, n:] = perm[(cur + n) % num_pages]  # valid page, never read
        cur += n
    g_dev = torch.Generator(device=device).manual_seed(seed)
    k = torch.randn(num_pages, ps, hkv, d, generator=g_dev, device=device, dtype=torch.float16)
    v = torch.randn(num_pages, ps, hkv, d, generator=g_dev, device=device, dtype=torch.float16)
    q = torch.randn(len(lens), hq, d, generator=g_dev, device=device, dtype=torch.float16)
    if key_boost:
        # Scale a few seeded key rows x8 (all kv heads) inside each sequence.
        for b, n in enumerate(lens):
            for _ in range(key_boost):
                t = int(torch.randint(0, n, (1,), generator=g_cpu))
                page = int(bt[b, t // ps])
                k[page, t % ps] *= 8.0
    sl = torch.tensor(lens, dtype=torch.int32)
    return Workload(name, q, k, v, bt.to(device), sl.to(device), list(lens), 1.0 / math.sqrt(d))


def c3_seq_lens(seed: int, batch: int = 32, max_len: int = 8192, page_size: int = 32):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(1, max_len + 1, (batch,), generator=g).tolist()
    lens[0] = 1
    for i in range(1, 4):  # at least three lengths that are not page multiples
        if lens[i] % page_size == 0:
            lens[i] -= 1
    return lens


def _spec(name: str, batch: int | None, seed: int):
    """(label, seq_lens, hq, hkv, head_dim, page_size, extra _build arguments) of a configuration."""
    if name == "C1":
        return "C1", [1024], 12, 2, 128, 16, {}
    if name == "C2":
        b = 64 if batch is None else batch
        return f"C2_b{b}", [4096] * b, 12, 2, 128, 16, {}
    if name == "C3":
        return "C3", c3_seq_lens(seed), 12, 2, 128, 32, {"max_pages": 256, "key_boost": 2}
    if name == "C4":
        return "C4", [131072], 32, 8, 128, 16, {}
    if name == "C5":
        g = torch.Generator().manual_seed(seed)
        lens = torch.randint(512, 32768 + 1, (256,), generator=g).tolist()
        return "C5", lens, 64, 8, 128, 16, {"max_pages": 2048}
    raise ValueError(f"unknown workload {name}")


def shard_lens(lens, page_size: int, sp: int) -> list[int]:
    """Tokens of each sequence on the first of ``sp`` GPUs that hold consecutive ranges of its
    pages, ceil(pages / sp) pages each (the last GPU holding the remainder): one GPU's share."""
    out = []
    for n in lens:
        pages = -(-n // page_size)
        out.append(min(n, -(-pages // sp) * page_size))
    return out


def make(name: str, batch: int | None = None, seed: int = 0, device: str = "cuda", tp: int = 1,
         sp: int = 1) -> Workload:
    """Configuration ``name``, or one GPU's share of it when it is sharded: ``tp`` GPUs each holding
    num_kv_heads / tp kv heads and their query groups (tensor parallel over heads), or ``sp`` GPUs
    each holding a range of every sequence's pages (``shard_lens``; the split-K merge of the
    shares would follow on each GPU)."""
    label, lens, hq, hkv, d, ps, kw = _spec(name, batch, seed)
    if tp < 1 or sp < 1 or hkv % tp:
        raise ValueError(f"{name}: tp {tp} must divide {hkv} kv heads, sp {sp} must be >= 1")
    if tp > 1:
        label, hq, hkv = f"{label}_tp{tp}", hq // tp, hkv // tp
    if sp > 1:
        label, lens = f"{label}_sp{sp}", shard_lens(lens, ps, sp)
        if "max_pages" in kw:
            kw = dict(kw, max_pages=-(-kw["max_pages"] // sp))
    return _build(label, lens, hq, hkv, d, ps, seed, device, **kw)


def bytes_of(w: Workload) -> int:
    s = w.shape
    return algorithmic_bytes(w.seq_lens_host, s["num_q_heads"], s["num_kv_heads"], s["head_dim"], s["page_size"],
                             w.k_cache.element_size())


def flops_of(w: Workload) -> int:
    s = w.shape
    return algorithmic_flops(w.seq_lens_host, s["num_q_heads"], s["head_dim"])


FP8_MAX = {torch.float8_e4m3fn: 448.0, torch.float8_e5m2: 57344.0}
FP8_NAMES = {"e4m3fn": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def to_fp8(w: Workload, dtype=torch.float8_e4m3fn) -> Workload:
    """The same workload with fp8 caches (codes of K / k_scale, V / v_scale)."""

    def quant(x):
        scale = float(x.abs().max()) / (0.875 * FP8_MAX[dtype]) or 1.0
        out = torch.empty(x.shape, dtype=dtype, device=x.device)
        flat_in, flat_out = x.view(x.shape[0], -1), out.view(x.shape[0], -1)
        step = max(1, (1 << 26) // max(flat_in.shape[1], 1))  # bounded fp32 temporaries
        for i in range(0, x.shape[0], step):
            # copy_ with a dtype change is an elementwise cast, never a device
            # memcpy (a profile's copy-kernel calibration counts those).
            flat_out[i:i + step].copy_(flat_in[i:i + step].float().div_(scale))
        return out, scale

    k8, ks = quant(w.k_cache)
    v8, vs = quant(w.v_cache)
    name = w.name + "_" + next(n for n, t in FP8_NAMES.items() if t == dtype)
    return Workload(name, w.q, k8, v8, w.block_table, w.seq_lens, list(w.seq_lens_host), w.scale, ks, vs)


def to_bf16(w: Workload) -> Workload:
    """The same workload in bfloat16 (q and both caches rounded)."""
    return Workload(w.name + "_bf16", w.q.bfloat16(), w.k_cache.bfloat16(), w.v_cache.bfloat16(), w.block_table,
                    w.seq_lens, list(w.seq_lens_host), w.scale)

"""Shared case builders, an independent SDPA check and parity assertions.

Tolerances:
* PARITY_RTOL / PARITY_ATOL = 2e-3: the contract (GPU fp16 output vs the
  fp32 oracle on the same fp16-rounded inputs).
* REF_RTOL / REF_ATOL = 1e-2 / 1e-3: the reference's own kernel-vs-oracle
  tolerance (tests/kernel_test_utils.py:20), checked as well.
"""

from __future__ import annotations

import math
import random

import torch
import torch.nn.functional as F

PARITY_RTOL = 2e-3
PARITY_ATOL = 2e-3
REF_RTOL = 1e-2
REF_ATOL = 1e-3


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


def make_cache(num_pages, page_size, num_kv_heads, head_dim, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(num_pages, page_size, num_kv_heads, head_dim, generator=g, dtype=torch.float32)
    v = torch.randn(num_pages, page_size, num_kv_heads, head_dim, generator=g, dtype=torch.float32)
    return k.to(dtype), v.to(dtype)


def contiguous_table(seq_lens, page_size, extra_cols=0, fill=None):
    """Block table with pages laid out in logical order; unused columns get `fill`."""
    needed = [cdiv(s, page_size) for s in seq_lens]
    width = max(max(needed), 1) + extra_cols
    total = sum(needed)
    bt = torch.zeros(len(seq_lens), width, dtype=torch.int32)
    cur = 0
    for b, n in enumerate(needed):
        for j in range(n):
            bt[b, j] = cur
            cur += 1
        for j in range(n, width):
            bt[b, j] = (cur if fill is None else fill) % max(total + 1, 1)
    return bt, total


def shuffled_table(seq_lens, page_size, spare_pages, extra_cols, seed):
    """Block table over a shuffled physical layout with never-referenced pages.

    Unused columns point at valid pages that hold different data, so reading
    one by mistake changes the result.
    """
    rng = random.Random(seed)
    needed = [cdiv(s, page_size) if s > 0 else 0 for s in seq_lens]
    width = max(max(needed), 1) + extra_cols
    num_pages = sum(needed) + spare_pages
    ids = list(range(num_pages))
    rng.shuffle(ids)
    bt = torch.zeros(len(seq_lens), width, dtype=torch.int32)
    cur = 0
    for b, n in enumerate(needed):
        for j in range(n):
            bt[b, j] = ids[cur]
            cur += 1
        for j in range(n, width):
            bt[b, j] = ids[(cur + j) % num_pages]
    return bt, num_pages


def random_case(seed, *, kv_heads=(1, 2, 4), gqa=(1, 2, 4, 6, 8), head_dims=(32, 64, 128),
                page_sizes=(1, 4, 8, 16, 32), max_batch=4, min_len=0, max_len=200):
    """Ragged batch, shuffled physical pages, spare pages and unused columns."""
    rng = random.Random(seed)
    hkv = rng.choice(kv_heads)
    group = rng.choice(gqa)
    d = rng.choice(head_dims)
    ps = rng.choice(page_sizes)
    batch = rng.randint(1, max_batch)
    lens = [rng.randint(min_len, max_len) for _ in range(batch)]
    bt, num_pages = shuffled_table(lens, ps, spare_pages=rng.randint(2, 5), extra_cols=rng.randint(0, 2),
                                   seed=seed + 7919)
    k, v = make_cache(num_pages, ps, hkv, d, seed)
    g = torch.Generator().manual_seed(seed + 1)
    q = torch.randn(batch, hkv * group, d, generator=g)
    return q, k, v, bt, torch.tensor(lens, dtype=torch.int32)


def sdpa_check(q, k_cache, v_cache, block_table, seq_lens, scale=None):
    """Independent check: walk pages one by one, then F.scaled_dot_product_attention.

    Shares no code with oracle/ (the reference's tests/oracle_sdpa.py plays
    the same role for its oracle).
    """
    batch, hq, d = q.shape
    page_size, hkv = k_cache.shape[1], k_cache.shape[2]
    group = hq // hkv
    out = torch.zeros_like(q)
    for b in range(batch):
        n = int(seq_lens[b])
        if n == 0:
            continue
        ks, vs, col, remaining = [], [], 0, n
        while remaining > 0:
            take = min(page_size, remaining)
            page = int(block_table[b, col])
            ks.append(k_cache[page, :take])
            vs.append(v_cache[page, :take])
            remaining -= take
            col += 1
        kk = torch.cat(ks).repeat_interleave(group, dim=1).transpose(0, 1).contiguous()  # [hq, n, d]
        vv = torch.cat(vs).repeat_interleave(group, dim=1).transpose(0, 1).contiguous()
        o = F.scaled_dot_product_attention(q[b].unsqueeze(1), kk, vv, scale=scale)
        out[b] = o.squeeze(1)
    return out


def assert_parity(actual, expected, rtol=PARITY_RTOL, atol=PARITY_ATOL, ref_tol=True):
    """GPU result (any dtype/device) vs CPU fp32/fp64 expectation."""
    a = actual.detach().float().cpu()
    e = torch.as_tensor(expected).float()
    assert a.shape == e.shape, (a.shape, e.shape)
    assert torch.isfinite(a).all(), "non-finite output"
    torch.testing.assert_close(a, e, rtol=rtol, atol=atol)
    if ref_tol:
        torch.testing.assert_close(a, e, rtol=REF_RTOL, atol=REF_ATOL)


def default_scale(d):
    return 1.0 / math.sqrt(d)

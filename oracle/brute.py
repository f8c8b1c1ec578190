"""float64 brute-force paged decode - test infrastructure only.

Written from the operator's definition, sharing no code with
``oracle.reference``: the pages of each sequence are walked one at a time
(the way tests/oracle_sdpa.py:17-58 walks them), and the attention is
evaluated in float64 numpy with an explicit exp / sum, per query head.
Used to cross-check ``oracle.reference`` and to write the golden fixtures
under tests/golden/.
"""

from __future__ import annotations

import math

import numpy as np


def gather_tokens(cache: np.ndarray, block_table_row: np.ndarray, n_tok: int) -> np.ndarray:
    """Tokens 0..n_tok-1 of one sequence, [n_tok, Hkv, d], by walking its pages."""
    page_size = cache.shape[1]
    chunks = []
    remaining = n_tok
    col = 0
    while remaining > 0:
        page = int(block_table_row[col])
        if page < 0 or page >= cache.shape[0]:
            raise ValueError(f"page id {page} outside the cache")
        take = min(page_size, remaining)
        chunks.append(cache[page, :take])
        remaining -= take
        col += 1
    if not chunks:
        return np.zeros((0,) + cache.shape[2:], dtype=cache.dtype)
    return np.concatenate(chunks, axis=0)


def decode_f64(q, k_cache, v_cache, block_table, seq_lens, scale=None) -> np.ndarray:
    """out[b, h] = softmax(scale * q[b,h] . K_b^T) V_b in float64 (zeros if seq_len 0)."""
    q = np.asarray(q, dtype=np.float64)
    k_cache = np.asarray(k_cache, dtype=np.float64)
    v_cache = np.asarray(v_cache, dtype=np.float64)
    block_table = np.asarray(block_table)
    seq_lens = np.asarray(seq_lens)
    batch, num_q_heads, head_dim = q.shape
    num_kv_heads = k_cache.shape[2]
    group = num_q_heads // num_kv_heads
    s = 1.0 / math.sqrt(head_dim) if scale is None else float(scale)
    out = np.zeros((batch, num_q_heads, head_dim), dtype=np.float64)
    for b in range(batch):
        n_tok = int(seq_lens[b])
        if n_tok == 0:
            continue
        keys = gather_tokens(k_cache, block_table[b], n_tok)
        vals = gather_tokens(v_cache, block_table[b], n_tok)
        for h in range(num_q_heads):
            kv = h // group
            logits = (keys[:, kv, :] @ q[b, h]) * s
            w = np.exp(logits - logits.max())
            out[b, h] = (w @ vals[:, kv, :]) / w.sum()
    return out

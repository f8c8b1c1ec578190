"""float64 model of split-K decode - test infrastructure only.

Restates analysis/split_k_derivation.md of the reference:

* phase 1 (:16-35): for the tokens [start, end) of one split,
  ``m_s = max score``, ``l_s = sum exp(score - m_s)``,
  ``O_s = sum exp(score - m_s) V`` (unnormalised); an empty split is
  ``(O, m, l) = (0, -inf, 0)``;
* phase 2 (:37-65): the running fold
  ``m_new = max(m_run, m_s); alpha = exp(m_run - m_new);
  beta = exp(m_s - m_new); l = l*alpha + l_s*beta; acc = acc*alpha + O_s*beta``,
  then ``out = acc / l``;
* the ``-inf`` guard (:67-86): ``beta = 0`` for an empty split (and, as the
  reference's Triton phase 2 also does, ``alpha = 0`` while the running max
  is still ``-inf``; src/kernel_v4_split_k.py:195-196);
* ``num_splits = 1`` reduces to the unsplit computation (:88-99).

Two ways to cut a sequence into splits are modelled: the reference CUDA
kernel's token chunks of ``ceil(L/S)`` (cuda/kernel_v4_split_k.cu:73-75) and
this build's page-aligned chunks of ``ceil(max_pages/S)`` pages.
"""

from __future__ import annotations

import math

import numpy as np

from .brute import gather_tokens

NEG_INF = float("-inf")


def phase1(qh: np.ndarray, keys: np.ndarray, vals: np.ndarray, scale: float, start: int, end: int):
    """Partial (O, m, l) of one query head over tokens [start, end)."""
    if end <= start:
        return np.zeros(vals.shape[-1]), NEG_INF, 0.0
    logits = (keys[start:end] @ qh) * scale
    m = float(logits.max())
    p = np.exp(logits - m)
    return p @ vals[start:end], m, float(p.sum())


def phase2(partials) -> np.ndarray:
    """Fold a list of (O_s, m_s, l_s) into the normalised output."""
    d = partials[0][0].shape[0]
    m_run, l_run, acc = NEG_INF, 0.0, np.zeros(d)
    for o_s, m_s, l_s in partials:
        m_new = max(m_run, m_s)
        alpha = 0.0 if m_run == NEG_INF else math.exp(m_run - m_new)
        beta = 0.0 if m_s == NEG_INF else math.exp(m_s - m_new)
        l_run = l_run * alpha + l_s * beta
        acc = acc * alpha + o_s * beta
        m_run = m_new
    if l_run == 0.0:
        return np.zeros(d)
    return acc / l_run


def split_bounds(n_tok: int, num_splits: int, mode: str, page_size: int = 1, max_pages: int = 0):
    """Token ranges of the splits of one sequence.

    mode "tokens": chunks of ceil(L/S) tokens (cuda/kernel_v4_split_k.cu:73-75).
    mode "pages": chunks of ceil(max_pages/S) whole pages, clipped to L.
    """
    if mode == "tokens":
        chunk = -(-n_tok // num_splits) if n_tok > 0 else 0
        return [(min(s * chunk, n_tok), min((s + 1) * chunk, n_tok)) for s in range(num_splits)]
    if mode == "pages":
        pps = max(1, -(-max(max_pages, 1) // num_splits))
        step = pps * page_size
        return [(min(s * step, n_tok), min((s + 1) * step, n_tok)) for s in range(num_splits)]
    raise ValueError(mode)


def decode_splitk_f64(q, k_cache, v_cache, block_table, seq_lens, num_splits, mode="pages", scale=None,
                      _phase2=phase2):
    """Whole decode through phase 1 + phase 2 in float64."""
    q = np.asarray(q, dtype=np.float64)
    k_cache = np.asarray(k_cache, dtype=np.float64)
    v_cache = np.asarray(v_cache, dtype=np.float64)
    block_table = np.asarray(block_table)
    seq_lens = np.asarray(seq_lens)
    batch, num_q_heads, head_dim = q.shape
    page_size, num_kv_heads = k_cache.shape[1], k_cache.shape[2]
    group = num_q_heads // num_kv_heads
    s = 1.0 / math.sqrt(head_dim) if scale is None else float(scale)
    out = np.zeros((batch, num_q_heads, head_dim))
    for b in range(batch):
        n_tok = int(seq_lens[b])
        keys = gather_tokens(k_cache, block_table[b], n_tok)
        vals = gather_tokens(v_cache, block_table[b], n_tok)
        bounds = split_bounds(n_tok, num_splits, mode, page_size, block_table.shape[1])
        for h in range(num_q_heads):
            kv = h // group
            parts = [phase1(q[b, h], keys[:, kv], vals[:, kv], s, a, e) for a, e in bounds]
            out[b, h] = _phase2(parts)
    return out

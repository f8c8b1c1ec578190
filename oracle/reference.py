"""fp32 CPU restatement of the reference oracle - test infrastructure only.

Restates ``paged_attention_decode_reference`` (src/reference.py:8-54) and
``_validate_inputs`` (src/reference.py:57-112) of Kare0638/paged-attention-
decode.  Same algorithm, step for step: per sequence, gather its pages,
expand the KV heads to the query heads (GQA), scores -> subtract the row
max -> softmax -> weighted sum of V, all in fp32; ``seq_len == 0`` gives
zeros.  Same error classes for the same invalid inputs (ValueError /
TypeError).

It is used as the parity oracle on fp16-rounded inputs (the protocol of
tests/kernel_test_utils.py:47-51) and, timed on the host cores, as the CPU
baseline.  It never ships in the product path.  decode_bf16_protocol and
decode_fp8_protocol apply the same oracle to bfloat16-rounded and to
dequantised fp8 inputs; tests/test_oracle_formats.py pins their own part
(unit scales, the roles of k_scale, v_scale and q's rounding).
"""

from __future__ import annotations

import math

import torch


def validate_inputs(q, k_cache, v_cache, block_table, seq_lens) -> None:
    """Shape/dtype/device/value checks of src/reference.py:57-112."""
    if q.ndim != 3:
        raise ValueError(f"q must be [batch, num_q_heads, head_dim], got {tuple(q.shape)}")
    if k_cache.ndim != 4:
        raise ValueError(
            "k_cache must be [num_pages, page_size, num_kv_heads, head_dim], "
            f"got {tuple(k_cache.shape)}"
        )
    if v_cache.shape != k_cache.shape:
        raise ValueError(f"v_cache shape {tuple(v_cache.shape)} must equal k_cache {tuple(k_cache.shape)}")
    if block_table.ndim != 2:
        raise ValueError(f"block_table must be [batch, max_pages], got {tuple(block_table.shape)}")
    if seq_lens.ndim != 1:
        raise ValueError(f"seq_lens must be [batch], got {tuple(seq_lens.shape)}")

    batch, num_q_heads, head_dim = q.shape
    _, page_size, num_kv_heads, cache_head_dim = k_cache.shape
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        if t.dtype != torch.float32:
            raise TypeError(f"{name} must be torch.float32 (got {t.dtype})")
    if block_table.dtype not in (torch.int32, torch.int64):
        raise TypeError("block_table must be int32 or int64")
    if seq_lens.dtype not in (torch.int32, torch.int64):
        raise TypeError("seq_lens must be int32 or int64")
    if q.device != k_cache.device or q.device != v_cache.device:
        raise ValueError("q, k_cache and v_cache must be on one device")
    if block_table.shape[0] != batch:
        raise ValueError("block_table batch dimension must equal q's")
    if seq_lens.shape[0] != batch:
        raise ValueError("seq_lens batch dimension must equal q's")
    if head_dim != cache_head_dim:
        raise ValueError("q head_dim must equal the KV cache head_dim")
    if page_size <= 0:
        raise ValueError("page_size must be positive")
    if num_kv_heads <= 0:
        raise ValueError("num_kv_heads must be positive")
    if num_q_heads % num_kv_heads != 0:
        raise ValueError("num_q_heads must be a multiple of num_kv_heads (GQA)")
    if bool((seq_lens < 0).any()):
        raise ValueError("seq_lens must be non-negative")
    capacity = block_table.shape[1] * page_size
    if bool((seq_lens > capacity).any()):
        raise ValueError("a seq_len exceeds what block_table can address")


def paged_attention_decode_reference(q, k_cache, v_cache, block_table, seq_lens, scale=None):
    """fp32 paged decode attention (src/reference.py:8-54).

    q [B, Hq, d], k_cache/v_cache [P, page_size, Hkv, d] (all fp32),
    block_table [B, max_pages], seq_lens [B] (int32/int64) -> [B, Hq, d] fp32.
    """
    validate_inputs(q, k_cache, v_cache, block_table, seq_lens)
    batch, num_q_heads, head_dim = q.shape
    num_pages, page_size, num_kv_heads, _ = k_cache.shape
    group = num_q_heads // num_kv_heads
    softmax_scale = 1.0 / math.sqrt(head_dim) if scale is None else float(scale)

    out = torch.empty_like(q)
    for b in range(batch):
        n_tok = int(seq_lens[b])
        if n_tok == 0:  # src/reference.py:32-34
            out[b] = 0.0
            continue
        n_pg = -(-n_tok // page_size)
        pages = block_table[b, :n_pg].to(torch.long)
        if bool(((pages < 0) | (pages >= num_pages)).any()):  # src/reference.py:40-41
            raise ValueError("block_table holds a physical page id outside the cache")
        # Gather the sequence's tokens in logical order: [n_tok, Hkv, d].
        keys = k_cache.index_select(0, pages).reshape(n_pg * page_size, num_kv_heads, head_dim)[:n_tok]
        vals = v_cache.index_select(0, pages).reshape(n_pg * page_size, num_kv_heads, head_dim)[:n_tok]
        # GQA: query head h reads kv head h // group (src/reference.py:46-47).
        keys = keys.unsqueeze(2).expand(n_tok, num_kv_heads, group, head_dim).reshape(n_tok, num_q_heads, head_dim)
        vals = vals.unsqueeze(2).expand(n_tok, num_kv_heads, group, head_dim).reshape(n_tok, num_q_heads, head_dim)
        logits = torch.einsum("hd,thd->ht", q[b], keys) * softmax_scale
        logits = logits - logits.amax(dim=-1, keepdim=True)
        weights = torch.softmax(logits, dim=-1)
        out[b] = torch.einsum("ht,thd->hd", weights, vals)
    return out


def decode_fp16_protocol(q, k_cache, v_cache, block_table, seq_lens, scale=None):
    """Oracle on fp16-rounded inputs upcast to fp32 (tests/kernel_test_utils.py:47-51).

    Accepts fp16 or fp32 tensors on any device; computes on the CPU.
    """
    q32 = q.detach().to("cpu").half().float()
    k32 = k_cache.detach().to("cpu").half().float()
    v32 = v_cache.detach().to("cpu").half().float()
    return paged_attention_decode_reference(q32, k32, v32, block_table.detach().to("cpu"),
                                            seq_lens.detach().to("cpu"), scale)


def decode_bf16_protocol(q, k_cache, v_cache, block_table, seq_lens, scale=None):
    """Oracle on bfloat16-rounded inputs upcast to fp32 (the fp16 protocol with bf16 rounding).

    The reference computes in fp16 only (src/kernel_cuda_v4.py:37-48); this
    applies its oracle to the values a bfloat16 caller holds.
    """
    q32 = q.detach().to("cpu").bfloat16().float()
    k32 = k_cache.detach().to("cpu").bfloat16().float()
    v32 = v_cache.detach().to("cpu").bfloat16().float()
    return paged_attention_decode_reference(q32, k32, v32, block_table.detach().to("cpu"),
                                            seq_lens.detach().to("cpu"), scale)


def decode_fp8_protocol(q, k_cache, v_cache, block_table, seq_lens, k_scale=1.0, v_scale=1.0, scale=None,
                        q_dtype=torch.float16):
    """Oracle for fp8 caches: the fp32 oracle on the dequantised caches.

    k_cache / v_cache are torch.float8_e4m3fn or torch.float8_e5m2 holding
    K / k_scale and V / v_scale (per-tensor scales); the oracle decodes each
    code with PyTorch's float8 -> float32 conversion, multiplies by the
    scale in fp32 and runs ``paged_attention_decode_reference`` on q rounded
    to ``q_dtype`` (fp16, or bfloat16 for a bf16 caller).  The reference's
    caches are fp16 only (src/kernel_cuda_v4.py:37-48); this extends its
    oracle to the dequantised values.
    """
    q32 = q.detach().to("cpu").to(q_dtype).float()
    k32 = k_cache.detach().to("cpu").float() * float(k_scale)
    v32 = v_cache.detach().to("cpu").float() * float(v_scale)
    return paged_attention_decode_reference(q32, k32, v32, block_table.detach().to("cpu"),
                                            seq_lens.detach().to("cpu"), scale)


def decode_rows_fp16_protocol(q, k_cache, v_cache, block_table, seq_lens, rows, scale=None):
    """The oracle for a subset of batch rows, gathering only those rows' pages.

    For caches too large to upcast whole (tens of GB): only the pages the
    selected rows reference are copied to the host and upcast, and the
    block table is relabelled onto that compact page set.  Returns
    [len(rows), Hq, d] fp32.
    """
    page_size = k_cache.shape[1]
    rows = list(rows)
    bt_rows = block_table[rows].detach().to("cpu").to(torch.long)
    sl_rows = seq_lens[rows].detach().to("cpu").to(torch.long)
    used = []
    for i in range(len(rows)):
        n_pg = -(-int(sl_rows[i]) // page_size)
        used.append(bt_rows[i, :n_pg])
    uniq = torch.unique(torch.cat(used)) if used else torch.zeros(0, dtype=torch.long)
    remap = {int(p): j for j, p in enumerate(uniq.tolist())}
    idx = uniq.to(k_cache.device)
    k_sub = k_cache.index_select(0, idx).to("cpu").half().float()
    v_sub = v_cache.index_select(0, idx).to("cpu").half().float()
    bt_new = torch.zeros_like(bt_rows)
    for i in range(len(rows)):
        n_pg = -(-int(sl_rows[i]) // page_size)
        for j in range(n_pg):
            bt_new[i, j] = remap[int(bt_rows[i, j])]
    q_rows = q[rows].detach().to("cpu").half().float()
    if k_sub.shape[0] == 0:  # every selected row is empty
        k_sub = torch.zeros(1, *k_cache.shape[1:])
        v_sub = torch.zeros(1, *k_cache.shape[1:])
    return paged_attention_decode_reference(q_rows, k_sub, v_sub, bt_new, sl_rows, scale)

"""Drop-in Python surface of the decode operator.

``paged_attention_decode`` keeps the signature and behaviour of the
reference's ``paged_attention_decode_cuda_v4`` (src/kernel_cuda_v4.py:19-65):

    fn(q, k_cache, v_cache, block_table, seq_lens, num_splits=None, scale=None)
        -> Tensor  # fp16, shape of q

* q fp16 [batch, num_q_heads, head_dim]; k_cache / v_cache fp16
  [num_pages, page_size, num_kv_heads, head_dim]; block_table [batch,
  max_pages] and seq_lens [batch] in int32 or int64 (cast to int32 as the
  reference does, src/kernel_cuda_v4.py:58-59).
* ``scale`` defaults to 1/sqrt(head_dim) (src/kernel_cuda_v4.py:60).
* ``num_splits=None`` picks the split count from shapes (heuristics.py)
  instead of the reference's constant 64; an explicit value is honoured.
* Argument problems visible from metadata raise AssertionError, as the
  reference's asserts do (src/kernel_cuda_v4.py:37-48); the native layer
  raises RuntimeError.  Nothing here reads tensor values, so a call never
  synchronises with the device.  Preconditions left unchecked, as in the
  reference (src/kernel_cuda_v1.py:25-28): page ids in range and
  seq_len <= max_pages * page_size (the kernels clamp both so that a
  violation cannot fault).
"""

from __future__ import annotations

import math

import torch

from ._native import ext

SUPPORTED_HEAD_DIMS = (32, 64, 96, 128, 256)
MAX_GQA = 16
ENGINE_MFMA = 0
ENGINE_VALU = 1


def _check(q, k_cache, v_cache, block_table, seq_lens):
    assert q.is_cuda and k_cache.is_cuda and v_cache.is_cuda, "paged_attention_decode requires GPU tensors"
    assert block_table.is_cuda and seq_lens.is_cuda, "block_table and seq_lens must be GPU tensors"
    assert q.dtype == torch.float16 and k_cache.dtype == torch.float16 and v_cache.dtype == torch.float16, (
        "paged_attention_decode expects fp16 q/k_cache/v_cache"
    )
    assert q.dim() == 3 and k_cache.dim() == 4 and v_cache.shape == k_cache.shape, "bad q / cache shapes"
    batch, num_q_heads, head_dim = q.shape
    _, _, num_kv_heads, cache_head_dim = k_cache.shape
    assert cache_head_dim == head_dim, "q head_dim must match the KV cache head_dim"
    assert num_kv_heads > 0 and num_q_heads % num_kv_heads == 0, (
        "num_q_heads must be divisible by num_kv_heads (GQA)"
    )
    assert num_q_heads // num_kv_heads <= MAX_GQA, f"GQA group larger than {MAX_GQA}"
    assert head_dim in SUPPORTED_HEAD_DIMS, f"head_dim must be one of {SUPPORTED_HEAD_DIMS}"
    assert block_table.dim() == 2 and block_table.shape[0] == batch, "block_table must be [batch, max_pages]"
    assert seq_lens.dim() == 1 and seq_lens.shape[0] == batch, "seq_lens must be [batch]"
    assert k_cache.stride(3) == 1 and v_cache.stride(3) == 1, "K/V caches need a contiguous head_dim"
    return head_dim


def _aligned_q(q):
    # 16-byte rows are required by the kernels; q is small, so copy if needed.
    if q.stride(2) != 1 or q.stride(1) % 8 or q.stride(0) % 8 or q.data_ptr() % 16:
        return q.contiguous()
    return q


def paged_attention_decode_ex(q, k_cache, v_cache, block_table, seq_lens, num_splits=None, scale=None,
                              engine: int = ENGINE_MFMA):
    """``paged_attention_decode`` with the phase-1 engine selectable (0 MFMA, 1 VALU/DPP)."""
    head_dim = _check(q, k_cache, v_cache, block_table, seq_lens)
    if num_splits is None:
        num_splits = 0
    else:
        num_splits = int(num_splits)
        assert num_splits >= 1, "num_splits must be >= 1"
    if block_table.dtype != torch.int32:
        block_table = block_table.to(torch.int32)
    if seq_lens.dtype != torch.int32:
        seq_lens = seq_lens.to(torch.int32)
    scale = float(scale) if scale is not None else 1.0 / math.sqrt(head_dim)
    return ext().forward(_aligned_q(q), k_cache, v_cache, block_table, seq_lens, scale, num_splits, int(engine))


def paged_attention_decode(q, k_cache, v_cache, block_table, seq_lens, num_splits=None, scale=None):
    """Paged-attention decode on the GPU (drop-in for src/kernel_cuda_v4.py:19-65)."""
    return paged_attention_decode_ex(q, k_cache, v_cache, block_table, seq_lens, num_splits, scale)


# The reference's public name for the same operator.
paged_attention_decode_cuda_v4 = paged_attention_decode


def plan(batch, num_q_heads, num_kv_heads, head_dim, page_size, max_pages, num_splits=0, num_cus=0):
    """Split plan the native launcher would use (host only), as a dict."""
    return ext().plan(batch, num_q_heads, num_kv_heads, head_dim, page_size, max_pages, num_splits, num_cus)

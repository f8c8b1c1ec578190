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


def _check(q, k_cache, v_cache, block_table, seq_lens, dtypes=(torch.float16,)):
    assert q.is_cuda and k_cache.is_cuda and v_cache.is_cuda, "paged_attention_decode requires GPU tensors"
    assert block_table.is_cuda and seq_lens.is_cuda, "block_table and seq_lens must be GPU tensors"
    assert q.dtype in dtypes and k_cache.dtype == q.dtype and v_cache.dtype == q.dtype, (
        "paged_attention_decode expects fp16 q/k_cache/v_cache" if dtypes == (torch.float16,)
        else f"q, k_cache and v_cache must share one dtype of {dtypes}"
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
    """``paged_attention_decode`` with the phase-1 engine selectable (0 MFMA, 1 VALU/DPP), and bfloat16 too.

    q, k_cache and v_cache are all fp16, or all bfloat16 (MFMA engine; the
    output is then bfloat16 and P is rounded to bf16 for the PV product)."""
    head_dim = _check(q, k_cache, v_cache, block_table, seq_lens, (torch.float16, torch.bfloat16))
    assert q.dtype == torch.float16 or engine == ENGINE_MFMA, "bfloat16 runs on the MFMA engine"
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
    """Paged-attention decode on the GPU (drop-in for src/kernel_cuda_v4.py:19-65).

    fp16 only, as the reference asserts (src/kernel_cuda_v4.py:37-48);
    :func:`paged_attention_decode_ex` also takes bfloat16."""
    _check(q, k_cache, v_cache, block_table, seq_lens)
    return paged_attention_decode_ex(q, k_cache, v_cache, block_table, seq_lens, num_splits, scale)


# The reference's public name for the same operator.
paged_attention_decode_cuda_v4 = paged_attention_decode

FP8_CACHE_DTYPES = (torch.float8_e4m3fn, torch.float8_e5m2)
FP8_HEAD_DIMS = (64, 128, 256)
# PAD_KV_* codes of include/pa_decode.h by cache dtype (bfloat16: q, caches and output).
_KV_FORMATS = {torch.float16: 0, torch.float8_e4m3fn: 1, torch.float8_e5m2: 2, torch.bfloat16: 3}
_KV_NAMES = {"float16": torch.float16, "fp16": torch.float16, "half": torch.float16,
             "bfloat16": torch.bfloat16, "bf16": torch.bfloat16,
             "float8_e4m3fn": torch.float8_e4m3fn, "e4m3fn": torch.float8_e4m3fn, "e4m3": torch.float8_e4m3fn,
             "float8_e5m2": torch.float8_e5m2, "e5m2": torch.float8_e5m2}


def _kv_dtype(kv_data_type, default=torch.float16):
    """A dtype given as a torch dtype or a name (None: ``default``)."""
    if kv_data_type is None:
        return default
    if isinstance(kv_data_type, str):
        assert kv_data_type in _KV_NAMES, f"unknown data type {kv_data_type!r}"
        return _KV_NAMES[kv_data_type]
    assert kv_data_type in _KV_FORMATS, f"data type must be one of {tuple(_KV_FORMATS)}"
    return kv_data_type


def _pair_ok(q_dtype, kv_dtype):
    """fp16 q with fp16 or fp8 caches, or bfloat16 q with bfloat16 or fp8 caches."""
    if q_dtype == torch.bfloat16:
        return kv_dtype != torch.float16
    return q_dtype == torch.float16 and kv_dtype != torch.bfloat16


def _format_code(q_dtype, kv_dtype):
    """PAD_KV_* code of a call (fp8 caches with bfloat16 q: the ``_BF16`` codes 4 and 5)."""
    code = _KV_FORMATS[kv_dtype]
    return code + 3 if q_dtype == torch.bfloat16 and kv_dtype in FP8_CACHE_DTYPES else code


def _cache_format(q, k_cache, v_cache, head_dim, engine, k_scale, v_scale):
    """(PAD_KV_* code, k_scale, v_scale) of a call; fp8 and bf16 need the MFMA engine, fp8 head_dim 64/128/256."""
    assert k_cache.dtype in _KV_FORMATS and v_cache.dtype == k_cache.dtype, (
        "k_cache and v_cache must both be float16, bfloat16, float8_e4m3fn or float8_e5m2"
    )
    assert _pair_ok(q.dtype, k_cache.dtype), (
        "q must be float16 (with float16 or fp8 caches) or bfloat16 (with bfloat16 or fp8 caches)"
    )
    fmt = _format_code(q.dtype, k_cache.dtype)
    if fmt in (0, 3):
        assert k_scale in (None, 1.0) and v_scale in (None, 1.0), "k_scale / v_scale apply to fp8 caches only"
        assert fmt == 0 or engine == ENGINE_MFMA, "bfloat16 runs on the MFMA engine"
        return fmt, 1.0, 1.0
    assert head_dim in FP8_HEAD_DIMS, f"fp8 caches: head_dim must be one of {FP8_HEAD_DIMS}"
    assert engine == ENGINE_MFMA, "fp8 caches run on the MFMA engine"
    k_scale = 1.0 if k_scale is None else float(k_scale)
    v_scale = 1.0 if v_scale is None else float(v_scale)
    assert k_scale > 0 and v_scale > 0 and math.isfinite(k_scale) and math.isfinite(v_scale), (
        "k_scale and v_scale must be finite and positive"
    )
    return fmt, k_scale, v_scale


def paged_attention_decode_fp8(q, k_cache, v_cache, block_table, seq_lens, k_scale=1.0, v_scale=1.0,
                               num_splits=None, scale=None):
    """Decode over fp8 K/V caches: the same operator with half the cache bytes.

    ``k_cache`` / ``v_cache`` are ``torch.float8_e4m3fn`` or
    ``torch.float8_e5m2`` (both the same), laid out as the fp16 caches
    ``[num_pages, page_size, num_kv_heads, head_dim]``, and hold
    ``K / k_scale`` and ``V / v_scale`` (per-tensor scales, Python floats).
    The result equals the fp16 (bfloat16) operator on the dequantised caches
    ``k_cache.float() * k_scale`` and ``v_cache.float() * v_scale``: every fp8
    code widens to fp16 and to bf16 exactly.  q and the output are fp16 or
    bfloat16; head_dim 64, 128 or 256; the MFMA engine only.  No counterpart
    in the reference, whose caches are fp16 only (src/kernel_cuda_v4.py:37-48).
    """
    assert q.is_cuda and k_cache.is_cuda and v_cache.is_cuda, "paged_attention_decode requires GPU tensors"
    assert block_table.is_cuda and seq_lens.is_cuda, "block_table and seq_lens must be GPU tensors"
    assert q.dtype in (torch.float16, torch.bfloat16), "q must be fp16 or bf16"
    assert k_cache.dtype in FP8_CACHE_DTYPES and v_cache.dtype == k_cache.dtype, (
        "k_cache and v_cache must both be float8_e4m3fn or both float8_e5m2"
    )
    assert q.dim() == 3 and k_cache.dim() == 4 and v_cache.shape == k_cache.shape, "bad q / cache shapes"
    batch, num_q_heads, head_dim = q.shape
    num_kv_heads = k_cache.shape[2]
    assert k_cache.shape[3] == head_dim, "q head_dim must match the KV cache head_dim"
    assert num_kv_heads > 0 and num_q_heads % num_kv_heads == 0, (
        "num_q_heads must be divisible by num_kv_heads (GQA)"
    )
    assert num_q_heads // num_kv_heads <= MAX_GQA, f"GQA group larger than {MAX_GQA}"
    assert head_dim in FP8_HEAD_DIMS, f"fp8 caches: head_dim must be one of {FP8_HEAD_DIMS}"
    assert block_table.dim() == 2 and block_table.shape[0] == batch, "block_table must be [batch, max_pages]"
    assert seq_lens.dim() == 1 and seq_lens.shape[0] == batch, "seq_lens must be [batch]"
    assert k_cache.stride(3) == 1 and v_cache.stride(3) == 1, "K/V caches need a contiguous head_dim"
    k_scale, v_scale = float(k_scale), float(v_scale)
    assert k_scale > 0 and v_scale > 0 and math.isfinite(k_scale) and math.isfinite(v_scale), (
        "k_scale and v_scale must be finite and positive"
    )
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
    return ext().forward_kv8(_aligned_q(q), k_cache, v_cache, block_table, seq_lens, scale, k_scale, v_scale,
                             num_splits)


def paged_kv_indices(block_table, seq_lens, page_size: int):
    """Dense ``block_table [B, max_pages]`` + ``seq_lens [B]`` -> CSR ``(indptr, indices, last_page_len)``.

    The conversion of the reference's FlashInfer adapter,
    ``_paged_kv_indices`` (src/flashinfer_adapter.py:40-65): sequence b uses
    its first ``ceil(seq_lens[b] / page_size)`` pages, ``indptr`` is the
    running page count (int32, ``[B + 1]``), ``indices`` the used page ids in
    order (int32) and ``last_page_len[b] = seq_lens[b] - (pages_b - 1) *
    page_size`` (int32; in [1, page_size] for a non-empty sequence).  Done
    with tensor ops on the tables' device; sizing ``indices`` reads the total
    page count back to the host once.
    """
    assert block_table.dim() == 2 and seq_lens.dim() == 1 and block_table.shape[0] == seq_lens.shape[0], (
        "block_table must be [batch, max_pages] and seq_lens [batch]"
    )
    assert page_size >= 1, "page_size must be >= 1"
    device = block_table.device
    lens = seq_lens.to(torch.int64)
    pages = (lens + page_size - 1) // page_size
    indptr = torch.zeros(seq_lens.shape[0] + 1, dtype=torch.int32, device=device)
    indptr[1:] = torch.cumsum(pages, dim=0).to(torch.int32)
    cols = torch.arange(block_table.shape[1], device=device)
    used = cols.unsqueeze(0) < pages.unsqueeze(1)
    indices = block_table[used].to(torch.int32)
    last_page_len = (lens - (pages - 1) * page_size).to(torch.int32)
    return indptr, indices, last_page_len


def paged_attention_decode_csr(q, k_cache, v_cache, indptr, indices, last_page_len, num_splits=None, scale=None,
                               engine: int = ENGINE_MFMA, k_scale=None, v_scale=None):
    """Paged-attention decode over a CSR page index (no dense block table).

    Sequence b's page ids are ``indices[indptr[b]:indptr[b+1]]`` and its last
    page holds ``last_page_len[b]`` tokens - FlashInfer's paged-KV index, which
    the reference builds in src/flashinfer_adapter.py:40-65 and hands to
    ``BatchDecodeWithPagedKVCacheWrapper.plan/run`` (:100-112).  Same caches,
    ``scale`` and ``num_splits`` as :func:`paged_attention_decode`; returns
    fp16 shaped like q.  Index tensors may be int32 or int64 (cast to int32).
    The caches may also be fp8 with ``k_scale`` / ``v_scale``, as for
    :func:`paged_attention_decode_fp8`.
    """
    assert q.is_cuda and k_cache.is_cuda and v_cache.is_cuda, "paged_attention_decode requires GPU tensors"
    assert indptr.is_cuda and indices.is_cuda and last_page_len.is_cuda, "CSR index tensors must be GPU tensors"
    assert q.dtype in (torch.float16, torch.bfloat16), "paged_attention_decode expects fp16 or bf16 q"
    assert q.dim() == 3 and k_cache.dim() == 4 and v_cache.shape == k_cache.shape, "bad q / cache shapes"
    batch, num_q_heads, head_dim = q.shape
    num_kv_heads = k_cache.shape[2]
    assert k_cache.shape[3] == head_dim, "q head_dim must match the KV cache head_dim"
    assert num_q_heads % num_kv_heads == 0, "num_q_heads must be divisible by num_kv_heads (GQA)"
    assert num_q_heads // num_kv_heads <= MAX_GQA, f"GQA group larger than {MAX_GQA}"
    assert head_dim in SUPPORTED_HEAD_DIMS, f"head_dim must be one of {SUPPORTED_HEAD_DIMS}"
    assert indptr.dim() == 1 and indptr.shape[0] == batch + 1, "indptr must be [batch + 1]"
    assert last_page_len.dim() == 1 and last_page_len.shape[0] == batch, "last_page_len must be [batch]"
    assert indices.dim() == 1, "indices must be 1-D"
    assert k_cache.stride(3) == 1 and v_cache.stride(3) == 1, "K/V caches need a contiguous head_dim"
    if num_splits is None:
        num_splits = 0
    else:
        num_splits = int(num_splits)
        assert num_splits >= 1, "num_splits must be >= 1"
    indptr = indptr.to(torch.int32).contiguous()
    indices = indices.to(torch.int32).contiguous()
    last_page_len = last_page_len.to(torch.int32).contiguous()
    _, k_scale, v_scale = _cache_format(q, k_cache, v_cache, head_dim, engine, k_scale, v_scale)
    scale = float(scale) if scale is not None else 1.0 / math.sqrt(head_dim)
    return ext().forward_csr(_aligned_q(q), k_cache, v_cache, indptr, indices, last_page_len, scale, num_splits,
                             int(engine), k_scale, v_scale)


def plan(batch, num_q_heads, num_kv_heads, head_dim, page_size, max_pages, num_splits=0, num_cus=0, csr=False):
    """Split plan the native launcher would use (host only), as a dict.

    With ``csr=True``, the plan of :func:`paged_attention_decode_csr` whose ``indices`` hold ``max_pages``
    entries (all sequences' pages)."""
    return ext().plan(batch, num_q_heads, num_kv_heads, head_dim, page_size, max_pages, num_splits, num_cus,
                      bool(csr))


class BatchDecodeWrapper:
    """Plan once per decode step, run once per layer.

    The split the reference's FlashInfer adapter drives
    (``BatchDecodeWithPagedKVCacheWrapper``: ``plan(indptr, indices,
    last_page_len, num_qo_heads, num_kv_heads, head_dim, page_size, ...)``
    then ``run(q, (k_cache, v_cache))``, src/flashinfer_adapter.py:100-112;
    plan-once-run-many in bench/bench_flashinfer.py:131-151).  ``plan()``
    queues one small kernel that writes the launch's work list: for every
    workgroup of the decode grid, the (sequence, kv head) unit and page range
    it processes and the page ids its waves read first.  ``run()`` decodes
    from that list instead of working it out from the sequence lengths at
    the start of every launch, and returns exactly what
    :func:`paged_attention_decode_csr` (or, after :meth:`plan_block_table`,
    :func:`paged_attention_decode`) returns for the same arguments.

    The list encodes the lengths and page ids: plan again when they change
    (in a decoding loop, once per step, before the first layer).  The index
    tensors given to ``plan()`` are kept and read again by every ``run()``.

    Data types, with FlashInfer's argument names: ``q_data_type`` (float16
    by default, or bfloat16) and ``kv_data_type`` (q's type by default).
    fp8 caches: plan with ``kv_data_type=torch.float8_e4m3fn`` (or
    ``torch.float8_e5m2``, or their names; q float16 or bfloat16) and pass
    ``k_scale`` / ``v_scale`` to ``run()``; the result equals
    :func:`paged_attention_decode_fp8` (or the CSR call) on the same inputs.
    bfloat16: ``q_data_type=torch.bfloat16``; q and output bfloat16, caches
    bfloat16 unless ``kv_data_type`` names an fp8 type.
    """

    def __init__(self):
        self._plan = None

    def plan(self, indptr, indices, last_page_len, num_qo_heads, num_kv_heads, head_dim, page_size,
             sm_scale=None, num_splits=None, kv_data_type=None, q_data_type=None):
        """Plan over a CSR page index (FlashInfer's layout, see :func:`paged_kv_indices`)."""
        assert indptr.is_cuda and indices.is_cuda and last_page_len.is_cuda, "CSR index tensors must be GPU tensors"
        assert indptr.dim() == 1 and last_page_len.dim() == 1 and indptr.shape[0] == last_page_len.shape[0] + 1, (
            "indptr must be [batch + 1] and last_page_len [batch]"
        )
        assert indices.dim() == 1, "indices must be 1-D"
        q_dtype, kv_dtype = self._check_geometry(num_qo_heads, num_kv_heads, head_dim, page_size, kv_data_type,
                                                 q_data_type)
        indptr = indptr.to(torch.int32).contiguous()
        indices = indices.to(torch.int32).contiguous()
        last_page_len = last_page_len.to(torch.int32).contiguous()
        splits = self._splits(num_splits)
        wl = ext().plan_worklist_csr(indptr, indices, last_page_len, num_qo_heads, num_kv_heads, head_dim,
                                     page_size, splits, _format_code(q_dtype, kv_dtype))
        self._plan = ("csr", (indptr, indices, last_page_len), wl, splits,
                      (int(last_page_len.shape[0]), num_qo_heads, num_kv_heads, head_dim, page_size),
                      self._scale(sm_scale, head_dim), q_dtype, kv_dtype)

    def plan_block_table(self, block_table, seq_lens, num_qo_heads, num_kv_heads, head_dim, page_size,
                         sm_scale=None, num_splits=None, kv_data_type=None, q_data_type=None):
        """Plan over the reference's dense ``block_table [B, max_pages]`` and ``seq_lens [B]``."""
        assert block_table.is_cuda and seq_lens.is_cuda, "block_table and seq_lens must be GPU tensors"
        assert block_table.dim() == 2 and seq_lens.dim() == 1 and block_table.shape[0] == seq_lens.shape[0], (
            "block_table must be [batch, max_pages] and seq_lens [batch]"
        )
        q_dtype, kv_dtype = self._check_geometry(num_qo_heads, num_kv_heads, head_dim, page_size, kv_data_type,
                                                 q_data_type)
        if block_table.dtype != torch.int32:
            block_table = block_table.to(torch.int32)
        if seq_lens.dtype != torch.int32:
            seq_lens = seq_lens.to(torch.int32)
        splits = self._splits(num_splits)
        wl = ext().plan_worklist(block_table, seq_lens, num_qo_heads, num_kv_heads, head_dim, page_size, splits,
                                 _format_code(q_dtype, kv_dtype))
        self._plan = ("dense", (block_table, seq_lens), wl, splits,
                      (int(seq_lens.shape[0]), num_qo_heads, num_kv_heads, head_dim, page_size),
                      self._scale(sm_scale, head_dim), q_dtype, kv_dtype)

    def run(self, q, paged_kv_cache, k_scale=None, v_scale=None):
        """Decode ``q [batch, num_qo_heads, head_dim]`` against ``(k_cache, v_cache)``; q's dtype, shaped like q.

        ``k_scale`` / ``v_scale``: the per-tensor scales of fp8 caches (the
        caches hold K / k_scale and V / v_scale)."""
        assert self._plan is not None, "call plan() or plan_block_table() before run()"
        kind, index, wl, splits, geometry, scale, q_dtype, kv_dtype = self._plan
        k_cache, v_cache = paged_kv_cache
        assert q.is_cuda and k_cache.is_cuda and v_cache.is_cuda, "paged_attention_decode requires GPU tensors"
        assert q.dtype == q_dtype, f"q must be {q_dtype}, the q_data_type the plan was made for"
        assert k_cache.dtype == kv_dtype and v_cache.dtype == kv_dtype, (
            f"the caches must be {kv_dtype}, the kv_data_type the plan was made for"
        )
        assert q.dim() == 3 and k_cache.dim() == 4 and v_cache.shape == k_cache.shape, "bad q / cache shapes"
        batch, num_qo_heads, num_kv_heads, head_dim, page_size = geometry
        assert tuple(q.shape) == (batch, num_qo_heads, head_dim), "q does not match the planned shapes"
        assert k_cache.shape[1] == page_size and k_cache.shape[2] == num_kv_heads and k_cache.shape[3] == head_dim, (
            "k_cache does not match the planned page size / heads / head_dim"
        )
        assert k_cache.stride(3) == 1 and v_cache.stride(3) == 1, "K/V caches need a contiguous head_dim"
        _, k_scale, v_scale = _cache_format(q, k_cache, v_cache, head_dim, ENGINE_MFMA, k_scale, v_scale)
        if kind == "csr":
            return ext().forward_worklist_csr(_aligned_q(q), k_cache, v_cache, *index, wl, scale, splits, k_scale,
                                              v_scale)
        return ext().forward_worklist(_aligned_q(q), k_cache, v_cache, *index, wl, scale, splits, k_scale, v_scale)

    @staticmethod
    def _check_geometry(num_qo_heads, num_kv_heads, head_dim, page_size, kv_data_type=None, q_data_type=None):
        assert num_kv_heads > 0 and num_qo_heads % num_kv_heads == 0, (
            "num_qo_heads must be divisible by num_kv_heads (GQA)"
        )
        assert num_qo_heads // num_kv_heads <= MAX_GQA, f"GQA group larger than {MAX_GQA}"
        assert head_dim in SUPPORTED_HEAD_DIMS, f"head_dim must be one of {SUPPORTED_HEAD_DIMS}"
        assert page_size >= 1, "page_size must be >= 1"
        q_dtype = _kv_dtype(q_data_type)
        kv_dtype = _kv_dtype(kv_data_type, q_dtype)
        assert _pair_ok(q_dtype, kv_dtype), (
            "q_data_type float16 (with float16 or fp8 caches) or bfloat16 (with bfloat16 or fp8 caches)"
        )
        if kv_dtype in FP8_CACHE_DTYPES:
            assert head_dim in FP8_HEAD_DIMS, f"fp8 caches: head_dim must be one of {FP8_HEAD_DIMS}"
        return q_dtype, kv_dtype

    @staticmethod
    def _splits(num_splits):
        if num_splits is None:
            return 0
        num_splits = int(num_splits)
        assert num_splits >= 1, "num_splits must be >= 1"
        return num_splits

    @staticmethod
    def _scale(sm_scale, head_dim):
        return float(sm_scale) if sm_scale is not None else 1.0 / math.sqrt(head_dim)

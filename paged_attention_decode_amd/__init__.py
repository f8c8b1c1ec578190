"""MI355X-native paged-attention decode.

Drop-in replacement for the decode operator of Kare0638/paged-attention-decode
(``paged_attention_decode_cuda_v4``, src/kernel_cuda_v4.py:19-65), running
hand-written gfx950 HIP kernels through the C ABI in include/pa_decode.h.
"""

from .ops import (  # noqa: F401
    BatchDecodeWrapper,
    ENGINE_MFMA,
    ENGINE_VALU,
    FP8_CACHE_DTYPES,
    FP8_HEAD_DIMS,
    SUPPORTED_HEAD_DIMS,
    paged_attention_decode,
    paged_attention_decode_csr,
    paged_attention_decode_cuda_v4,
    paged_attention_decode_ex,
    paged_attention_decode_fp8,
    paged_kv_indices,
    plan,
)

__all__ = [
    "BatchDecodeWrapper",
    "paged_attention_decode",
    "paged_attention_decode_cuda_v4",
    "paged_attention_decode_ex",
    "paged_attention_decode_csr",
    "paged_attention_decode_fp8",
    "paged_kv_indices",
    "plan",
    "ENGINE_MFMA",
    "ENGINE_VALU",
    "SUPPORTED_HEAD_DIMS",
    "FP8_CACHE_DTYPES",
    "FP8_HEAD_DIMS",
]

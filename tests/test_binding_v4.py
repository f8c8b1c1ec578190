"""GPU tests of the torch binding's reference-signature entry, forward_v4.

forward_v4(q, k_cache, v_cache, block_table, seq_lens, scale, gqa_ratio,
head_dim, page_size, num_splits) keeps the argument list of the reference's
binding (cuda/binding.cpp:13-14, cuda/kernels.h:60-70), for code that called
the extension directly.  Parity: the primary shape of
tests/test_kernel_cuda_v4.py:36-59 against the fp32 oracle on the same fp16
inputs, atol = rtol = 2e-3 (and the reference's own 1e-2 / 1e-3).  Errors:
RuntimeError when gqa_ratio, head_dim or page_size disagree with the tensors
and when num_splits < 1 (cuda/kernel_v4_split_k.cu:216-223 checks
num_splits >= 1 with TORCH_CHECK as well).
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle.reference import decode_fp16_protocol
from tests.helpers import assert_parity, contiguous_table, make_cache

pytestmark = pytest.mark.gpu

HKV, GQA, D, PS = 2, 6, 128, 16
LENS = [1, 17, 256, 4000]


def _case():
    bt, total = contiguous_table(LENS, PS)
    k, v = make_cache(total + 3, PS, HKV, D, seed=0)
    q = torch.randn(len(LENS), HKV * GQA, D, generator=torch.Generator().manual_seed(0))
    return q, k, v, bt, torch.tensor(LENS, dtype=torch.int32)


def _dev(*ts):
    return [t.half().cuda() if t.is_floating_point() else t.cuda() for t in ts]


@pytest.mark.parametrize("num_splits", [1, 8, 64])
def test_forward_v4_matches_oracle(num_splits):
    from paged_attention_decode_amd._native import ext

    q, k, v, bt, sl = _case()
    scale = 1.0 / math.sqrt(D)
    expected = decode_fp16_protocol(q, k, v, bt, sl, scale)
    qd, kd, vd, btd, sld = _dev(q, k, v, bt, sl)
    out = ext().forward_v4(qd, kd, vd, btd, sld, scale, GQA, D, PS, num_splits)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and out.shape == q.shape
    assert_parity(out, expected)


def test_forward_v4_equals_drop_in():
    """Same kernel, plan and split count as the Python drop-in: bit-identical output."""
    import paged_attention_decode_amd as pad
    from paged_attention_decode_amd._native import ext

    q, k, v, bt, sl = _case()
    qd, kd, vd, btd, sld = _dev(q, k, v, bt, sl)
    a = ext().forward_v4(qd, kd, vd, btd, sld, 1.0 / math.sqrt(D), GQA, D, PS, 8)
    b = pad.paged_attention_decode_cuda_v4(qd, kd, vd, btd, sld, num_splits=8)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize(
    "field,value,match",
    [
        ("gqa_ratio", GQA - 1, "gqa_ratio"),
        ("gqa_ratio", 0, "gqa_ratio"),
        ("head_dim", 64, "head_dim"),
        ("page_size", 32, "page_size"),
        ("num_splits", 0, "num_splits"),
        ("num_splits", -3, "num_splits"),
    ],
)
def test_forward_v4_rejects_inconsistent_arguments(field, value, match):
    from paged_attention_decode_amd._native import ext

    q, k, v, bt, sl = _case()
    qd, kd, vd, btd, sld = _dev(q, k, v, bt, sl)
    args = {"gqa_ratio": GQA, "head_dim": D, "page_size": PS, "num_splits": 8}
    args[field] = value
    with pytest.raises(RuntimeError, match=match):
        ext().forward_v4(qd, kd, vd, btd, sld, 1.0 / math.sqrt(D), args["gqa_ratio"], args["head_dim"],
                         args["page_size"], args["num_splits"])
    torch.cuda.synchronize()

"""Pins for the oracle's data-format protocols (oracle/reference.py).

decode_fp8_protocol and decode_bf16_protocol feed the pinned fp32 oracle
(test_oracle_pins.py) with dequantised or rounded inputs.  What is checked
here is their own part, each against something independent of its code:

* unit scales on fp8 codes reduce to the fp16 protocol on the same values
  (every fp8 value is an fp16 value; PyTorch's float8 -> float16 cast);
* k_scale acts on the scores: it equals folding the factor into the softmax
  scale (a swapped or dropped k_scale fails);
* v_scale acts on the output linearly: scaling it by 2 doubles the output
  exactly, and leaves the attention weights alone (a v_scale applied to K
  fails);
* q is rounded to the requested type (fp16 or bf16) before the oracle;
* the bf16 protocol on values both formats hold exactly equals the fp16
  protocol, and on others differs by the bf16 rounding of the inputs only
  (the float64 brute force on the same rounded inputs agrees).
"""

from __future__ import annotations

import pytest
import torch

from oracle.brute import decode_f64
from oracle.reference import decode_bf16_protocol, decode_fp8_protocol, decode_fp16_protocol
from tests.helpers import make_cache, shuffled_table

FP8 = [torch.float8_e4m3fn, torch.float8_e5m2]


def _case(seed, lens=(5, 40, 0, 33), ps=8, hkv=2, gqa=3, d=16):
    bt, n = shuffled_table(list(lens), ps, spare_pages=2, extra_cols=1, seed=seed)
    k, v = make_cache(n, ps, hkv, d, seed=seed)
    q = torch.randn(len(lens), hkv * gqa, d, generator=torch.Generator().manual_seed(seed + 1))
    return q, k, v, bt, torch.tensor(list(lens), dtype=torch.int32)


@pytest.mark.parametrize("dt", FP8)
def test_fp8_unit_scales_are_the_fp16_protocol_on_the_codes(dt):
    q, k, v, bt, sl = _case(1)
    k8, v8 = k.to(dt), v.to(dt)
    a = decode_fp8_protocol(q, k8, v8, bt, sl)
    b = decode_fp16_protocol(q, k8.to(torch.float16), v8.to(torch.float16), bt, sl)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dt", FP8)
def test_k_scale_acts_on_the_scores(dt):
    q, k, v, bt, sl = _case(2)
    k8, v8 = (k / 0.05).to(dt), (v / 0.05).to(dt)
    ks, s = 0.037, 0.25
    a = decode_fp8_protocol(q, k8, v8, bt, sl, k_scale=ks, v_scale=1.0, scale=s)
    b = decode_fp8_protocol(q, k8, v8, bt, sl, k_scale=1.0, v_scale=1.0, scale=s * ks)
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6)
    c = decode_fp8_protocol(q, k8, v8, bt, sl, k_scale=1.0, v_scale=ks, scale=s)  # the scale on V instead
    assert (a - c).abs().max() > 1e-2


@pytest.mark.parametrize("dt", FP8)
def test_v_scale_acts_linearly_on_the_output(dt):
    q, k, v, bt, sl = _case(3)
    k8, v8 = (k / 0.05).to(dt), (v / 0.05).to(dt)
    a = decode_fp8_protocol(q, k8, v8, bt, sl, k_scale=0.05, v_scale=0.05)
    b = decode_fp8_protocol(q, k8, v8, bt, sl, k_scale=0.05, v_scale=0.1)
    assert torch.equal(b, 2 * a)  # doubling a power-of-two factor is exact in fp32
    c = decode_fp8_protocol(q, k8, v8, bt, sl, k_scale=0.1, v_scale=0.05)  # the factor on K instead
    assert (c - a).abs().max() > 1e-2


def test_q_is_rounded_to_the_requested_type():
    q, k, v, bt, sl = _case(4)
    k8, v8 = k.to(torch.float8_e4m3fn), v.to(torch.float8_e4m3fn)
    a = decode_fp8_protocol(q, k8, v8, bt, sl, q_dtype=torch.bfloat16)
    b = decode_fp8_protocol(q.bfloat16().float(), k8, v8, bt, sl, q_dtype=torch.float32)
    c = decode_fp8_protocol(q, k8, v8, bt, sl)  # fp16 rounding
    assert torch.equal(a, b)
    assert not torch.equal(a, c)


def test_bf16_protocol_on_values_both_formats_hold():
    q, k, v, bt, sl = _case(5)
    q, k, v = [(t * 8).round().clamp(-32, 32) / 8 for t in (q, k, v)]
    assert torch.equal(decode_bf16_protocol(q, k, v, bt, sl), decode_fp16_protocol(q, k, v, bt, sl))


def test_bf16_protocol_against_the_float64_brute_force():
    q, k, v, bt, sl = _case(6)
    out = decode_bf16_protocol(q, k, v, bt, sl)
    ref = decode_f64(q.bfloat16().double(), k.bfloat16().double(), v.bfloat16().double(), bt, sl)
    torch.testing.assert_close(out.double(), torch.from_numpy(ref), rtol=1e-5, atol=1e-6)
    # and it is not the fp16 protocol on general values
    assert not torch.equal(out, decode_fp16_protocol(q, k, v, bt, sl))

"""GPU tests of the decode with bfloat16 q, caches and output.

No counterpart in the reference, whose operator is fp16 only
(src/kernel_cuda_v4.py:37-48).  The kernel runs the fp16 path on bf16 MFMAs:
the scores and the fold are fp32, P is rounded to bf16 for the PV product
(as the fp16 path rounds it to fp16), and the output is rounded to bf16.

Tolerance: atol = rtol = 1e-2 against the fp32 oracle on the same
bf16-rounded inputs (oracle/reference.py decode_bf16_protocol).  A bf16
output alone is within half an ulp, 2^-9 = 0.2% relative, of the exact
value; the rounded P adds about as much.  Structural checks: split
invariance to 1e-2, the CSR index and the work list bit-identical to the
dense one-shot call, and a ~2^-8 relative agreement with the fp16 kernel on
inputs exact in both formats.
"""

from __future__ import annotations

import pytest
import torch

from oracle.reference import decode_bf16_protocol
from tests.helpers import make_cache, random_case, shuffled_table

pytestmark = pytest.mark.gpu

BF16_ATOL = BF16_RTOL = 1e-2


def _close(actual, expected, atol=BF16_ATOL, rtol=BF16_RTOL):
    a = actual.float().cpu()
    e = expected.float().cpu()
    assert a.shape == e.shape and torch.isfinite(a).all()
    err = (a - e).abs()
    bound = atol + rtol * e.abs()
    assert bool((err <= bound).all()), f"max excess {(err - bound).max().item():.3e}, max err {err.max().item():.3e}"


def _case(lens, ps, hkv, gqa, d, seed, spare=2, extra=1):
    bt, n = shuffled_table(lens, ps, spare_pages=spare, extra_cols=extra, seed=seed)
    k, v = make_cache(n, ps, hkv, d, seed=seed)
    q = torch.randn(len(lens), hkv * gqa, d, generator=torch.Generator().manual_seed(seed))
    return q, k, v, bt, torch.tensor(lens, dtype=torch.int32)


def _dev(q, k, v, bt, sl):
    return q.bfloat16().cuda(), k.bfloat16().cuda(), v.bfloat16().cuda(), bt.cuda(), sl.cuda()


@pytest.mark.parametrize("d", [32, 64, 96, 128, 256])
@pytest.mark.parametrize("ps", [16, 1, 12])
def test_bf16_matches_oracle(d, ps):
    import paged_attention_decode_amd as pad

    lens = [1, ps + 3, 150, 777, 0]
    q, k, v, bt, sl = _case(lens, ps, 2, 6, d, seed=ps + d)
    expected = decode_bf16_protocol(q, k, v, bt, sl)
    qd, kd, vd, btd, sld = _dev(q, k, v, bt, sl)
    for splits in (None, 1, 5, 60):
        out = pad.paged_attention_decode_ex(qd, kd, vd, btd, sld, num_splits=splits)
        torch.cuda.synchronize()
        assert out.dtype == torch.bfloat16 and out.shape == q.shape
        _close(out, expected)
        assert torch.all(out[4] == 0)  # the empty row


@pytest.mark.parametrize("hkv,gqa", [(1, 1), (4, 2), (2, 8), (1, 16)])
def test_bf16_group_sizes(hkv, gqa):
    import paged_attention_decode_amd as pad

    q, k, v, bt, sl = _case([33, 2000, 5], 16, hkv, gqa, 128, seed=hkv * 31 + gqa)
    expected = decode_bf16_protocol(q, k, v, bt, sl)
    qd, kd, vd, btd, sld = _dev(q, k, v, bt, sl)
    for splits in (None, 64):
        _close(pad.paged_attention_decode_ex(qd, kd, vd, btd, sld, num_splits=splits), expected)


def test_bf16_close_to_the_fp16_kernel_on_shared_values():
    # Inputs that both formats hold exactly (multiples of 1/8 in [-4, 4]):
    # the two kernels differ only by P's and the output's rounding.
    import paged_attention_decode_amd as pad

    q, k, v, bt, sl = _case([300, 1500, 64], 16, 2, 4, 128, seed=7)
    q, k, v = [(t * 8).round().clamp(-32, 32) / 8 for t in (q, k, v)]
    a = pad.paged_attention_decode_ex(*_dev(q, k, v, bt, sl))
    b = pad.paged_attention_decode(q.half().cuda(), k.half().cuda(), v.half().cuda(), bt.cuda(), sl.cuda())
    torch.cuda.synchronize()
    _close(a, b.float(), atol=2e-2 * 2.0 ** -2, rtol=2.0 ** -7)


def test_bf16_csr_and_work_list_equal_the_dense_call():
    import paged_attention_decode_amd as pad
    from oracle.csr import paged_kv_indices as ref_indices

    lens = [4096, 300, 2500, 1, 777, 0, 1500, 64]
    q, k, v, bt, sl = _case(lens, 16, 2, 6, 128, seed=41)
    qd, kd, vd, btd, sld = _dev(q, k, v, bt, sl)
    indptr, indices, last = [t.cuda() for t in ref_indices(bt, sl, 16)]
    dense = pad.BatchDecodeWrapper()
    dense.plan_block_table(btd, sld, 12, 2, 128, 16, q_data_type=torch.bfloat16)
    csr = pad.BatchDecodeWrapper()
    csr.plan(indptr, indices, last, 12, 2, 128, 16, q_data_type="bf16")
    a = pad.paged_attention_decode_ex(qd, kd, vd, btd, sld)
    b = dense.run(qd, (kd, vd))
    c = pad.paged_attention_decode_csr(qd, kd, vd, indptr, indices, last)
    e = csr.run(qd, (kd, vd))
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(c, e)
    expected = decode_bf16_protocol(q, k, v, bt, sl)
    _close(a, expected)
    _close(c, expected)
    with pytest.raises(AssertionError, match="q_data_type"):
        dense.run(q.half().cuda(), (kd, vd))


def test_bf16_rejections():
    import paged_attention_decode_amd as pad
    from paged_attention_decode_amd._native import ext

    q, k, v, bt, sl = _case([20], 16, 2, 2, 128, seed=1)
    qd, kd, vd, btd, sld = _dev(q, k, v, bt, sl)
    with pytest.raises(AssertionError, match="MFMA"):
        pad.paged_attention_decode_ex(qd, kd, vd, btd, sld, engine=1)
    with pytest.raises(AssertionError, match="fp16"):
        pad.paged_attention_decode(qd, kd, vd, btd, sld)  # the drop-in keeps the reference's fp16 contract
    with pytest.raises(RuntimeError, match="bfloat16"):
        ext().forward(qd, kd.half(), vd.half(), btd, sld, 0.1, 0, 0)
    with pytest.raises(RuntimeError, match="unsupported K/V cache format"):
        ext().forward(qd, kd, vd, btd, sld, 0.1, 0, 1)
    with pytest.raises(AssertionError, match="q_data_type"):
        pad.BatchDecodeWrapper().plan_block_table(btd, sld, 4, 2, 128, 16, q_data_type=torch.bfloat16,
                                                  kv_data_type=torch.float16)
    torch.cuda.synchronize()


FUZZ = int(__import__("os").environ.get("PAD_KERNEL_FUZZ_ITERS", "20"))


@pytest.mark.parametrize("seed", range(FUZZ))
def test_bf16_fuzz_matrix(seed):
    # Every head_dim, group sizes to 16, every block mode, ragged batches
    # with empty rows; the heuristic plan, 4 and 60 splits.
    import paged_attention_decode_amd as pad

    q, k, v, bt, sl = random_case(11000 + seed, kv_heads=(1, 2, 4), gqa=(1, 3, 8, 16),
                                  head_dims=(32, 64, 96, 128, 256),
                                  page_sizes=(1, 2, 3, 4, 8, 12, 16, 24, 32), min_len=0, max_len=400)
    expected = decode_bf16_protocol(q, k, v, bt, sl)
    qd, kd, vd, btd, sld = _dev(q, k, v, bt, sl)
    for s in (None, 4, 60):
        _close(pad.paged_attention_decode_ex(qd, kd, vd, btd, sld, num_splits=s), expected)


def test_bf16_strided_inputs():
    import paged_attention_decode_amd as pad

    lens = [40, 90]
    q, k, v, bt, sl = _case(lens, 16, 2, 6, 128, seed=41, spare=1, extra=0)
    expected = decode_bf16_protocol(q, k, v, bt, sl)
    n = k.shape[0]
    qw = torch.zeros(2, 12, 256, dtype=torch.bfloat16, device="cuda")
    qw[:, :, 64:192] = q.bfloat16().cuda()
    kw = torch.zeros(n, 16, 3, 136, dtype=torch.bfloat16, device="cuda")
    vw = torch.zeros(n, 16, 3, 136, dtype=torch.bfloat16, device="cuda")
    kw[:, :, :2, :128] = k.bfloat16().cuda()
    vw[:, :, :2, :128] = v.bfloat16().cuda()
    out = pad.paged_attention_decode_ex(qw[:, :, 64:192], kw[:, :, :2, :128], vw[:, :, :2, :128], bt.cuda(),
                                        sl.cuda())
    torch.cuda.synchronize()
    _close(out, expected)


def test_bf16_graph_capture_replays():
    import paged_attention_decode_amd as pad

    lens = [4096, 300, 2500, 1]
    q, k, v, bt, sl = _case(lens, 16, 2, 6, 128, seed=93)
    dev = [k.bfloat16().cuda(), v.bfloat16().cuda(), bt.cuda(), sl.cuda()]
    qs = [torch.randn(len(lens), 12, 128, generator=torch.Generator().manual_seed(94 + i)).bfloat16().cuda()
          for i in range(3)]
    q_static = qs[0].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            pad.paged_attention_decode_ex(q_static, *dev)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out_static = pad.paged_attention_decode_ex(q_static, *dev)
    torch.cuda.synchronize()
    for rep in range(2):
        for qn in qs:
            q_static.copy_(qn)
            graph.replay()
            torch.cuda.synchronize()
            eager = pad.paged_attention_decode_ex(qn, *dev)
            torch.cuda.synchronize()
            assert torch.equal(out_static, eager), f"replay {rep} differs from the eager call"

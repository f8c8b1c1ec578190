"""A compiled C++ caller of the C ABI (tests/capi_consumer.cpp), run as its own process.

It is what a runtime written in C or C++ would do (include/pa_decode.h plus
HIP runtime calls for memory and a stream; no Python, no PyTorch): size the
scratch with the pure-host queries, zero the counters once, launch twice on
its own stream.  Its output must equal the Python drop-in's bit for bit (same
kernel, same plan) and match the fp32 oracle at the parity tolerance.
"""

from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest
import torch

from oracle.reference import decode_fp16_protocol
from tests.helpers import assert_parity, make_cache, shuffled_table

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_bin", "capi_consumer")


@pytest.mark.parametrize("splits", [0, 1, 7])
def test_compiled_caller_matches_the_drop_in_and_the_oracle(tmp_path, splits):
    import paged_attention_decode_amd as pad

    assert os.path.exists(BIN), f"{BIN} is missing: run python -m paged_attention_decode_amd.build"
    lens = [1, 77, 400, 1000, 0]
    hq, hkv, d, ps = 12, 2, 128, 16
    bt, n = shuffled_table(lens, ps, spare_pages=3, extra_cols=1, seed=71)
    k, v = make_cache(n, ps, hkv, d, seed=71)
    q = torch.randn(len(lens), hq, d, generator=torch.Generator().manual_seed(71))
    sl = torch.tensor(lens, dtype=torch.int32)
    header = np.array([len(lens), hq, hkv, d, ps, bt.shape[1], n, splits], dtype=np.int64)
    src = tmp_path / "in.bin"
    with open(src, "wb") as f:
        f.write(header.tobytes())
        for t in (q.half(), k.half(), v.half()):
            f.write(t.contiguous().view(torch.int16).numpy().tobytes())
        f.write(bt.contiguous().numpy().astype(np.int32).tobytes())
        f.write(sl.numpy().astype(np.int32).tobytes())
    dst = tmp_path / "out.bin"
    run = subprocess.run([BIN, str(src), str(dst)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stderr
    out = torch.from_numpy(np.fromfile(dst, dtype=np.int16)).view(torch.float16).view(q.shape)
    assert_parity(out, decode_fp16_protocol(q, k, v, bt, sl))
    drop_in = pad.paged_attention_decode(q.half().cuda(), k.half().cuda(), v.half().cuda(), bt.cuda(), sl.cuda(),
                                         num_splits=splits or None)
    torch.cuda.synchronize()
    assert torch.equal(out, drop_in.cpu())

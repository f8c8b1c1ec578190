"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: each fixture's expected output is reproduced by the float64 brute force
(to the last bits) and by the fp32 oracle restatement (1e-5), so neither the
data nor the oracles can drift silently.  GPU: the HIP decode path matches
every fixture within atol = rtol = 2e-3 (and the reference's 1e-2 / 1e-3),
at the heuristic split count and at forced ones.
"""

from __future__ import annotations

import glob
import math
import os

import numpy as np
import pytest
import torch

from oracle.brute import decode_f64
from oracle.reference import paged_attention_decode_reference
from tests.helpers import assert_parity

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "*.npz")))


def _load(path):
    z = np.load(path)
    scale = float(z["scale"])
    return {k: z[k] for k in z.files}, (None if math.isnan(scale) else scale)


def test_fixtures_present():
    assert len(GOLDEN) >= 10


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_fixture_matches_oracles(path):
    f, scale = _load(path)
    f64 = decode_f64(f["q"].astype(np.float64), f["k_cache"].astype(np.float64), f["v_cache"].astype(np.float64),
                     f["block_table"], f["seq_lens"], scale)
    np.testing.assert_allclose(f64, f["expected"], rtol=1e-12, atol=1e-12)
    ref = paged_attention_decode_reference(torch.from_numpy(f["q"]).float(), torch.from_numpy(f["k_cache"]).float(),
                                           torch.from_numpy(f["v_cache"]).float(), torch.from_numpy(f["block_table"]),
                                           torch.from_numpy(f["seq_lens"]), scale)
    np.testing.assert_allclose(ref.numpy(), f["expected"], rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_kernel_matches_fixture(path):
    import paged_attention_decode_amd as pad

    f, scale = _load(path)
    dev = [torch.from_numpy(f[k]).cuda() for k in ("q", "k_cache", "v_cache", "block_table", "seq_lens")]
    for splits in (None, 1, 3):
        out = pad.paged_attention_decode(*dev, num_splits=splits, scale=scale)
        assert_parity(out, torch.from_numpy(f["expected"]))

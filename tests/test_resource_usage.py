"""Compiler-reported register use of the decode kernels (CPU: hipcc only, no GPU).

Every pad_phase1_kernel instantiation must run without scratch memory: no
VGPR spills and a scratch size of zero (SGPR spills go to VGPR lanes and are
allowed).  One compile of pa_decode.hip for gfx950, about a minute.
"""

import os
import shutil

import pytest

from paged_attention_decode_amd import build, resource_usage

pytestmark = pytest.mark.skipif(not os.path.exists(os.path.join(build.ROCM, "bin", "hipcc"))
                                and shutil.which("hipcc") is None, reason="hipcc not installed")


@pytest.fixture(scope="module")
def rows():
    return [r for r in resource_usage.collect() if "pad_phase1_kernel" in r["name"]]


def test_every_instantiation_is_reported(rows):
    # 5 head_dims x 6 block modes of the MFMA engine, plus the VALU engine's
    # (head_dim 64/128) x (uniform, other) x group sizes {1, 2, 4, 6, 8},
    # plus 2 fp8 cache formats x head_dim {64, 128, 256} x 6 block modes,
    # plus bfloat16 x 5 head_dims x 6 block modes, plus the 2 fp8 formats
    # with bfloat16 q x 3 head_dims x 6 block modes.
    assert len(rows) >= 152
    assert any(r["template"] == "<128, 1, 0, 0>" for r in rows)  # the benchmark's kernel
    assert any(r["template"] == "<128, 1, 0, 0, e4m3fn>" for r in rows)
    assert any(r["template"] == "<128, 1, 0, 0, e5m2>" for r in rows)
    assert any(r["template"] == "<96, 0, 0, 0, bf16>" for r in rows)
    assert any(r["template"] == "<256, 2, 0, 0, e5m2/bf16>" for r in rows)


def test_no_scratch_memory_in_any_instantiation(rows):
    bad = [(r["template"], r.get("vgpr_spill"), r.get("scratch")) for r in rows
           if r.get("vgpr_spill", 0) or r.get("scratch", 0)]
    assert not bad, f"VGPR spills / scratch: {bad}"


def test_headline_kernel_fits_three_waves_per_simd(rows):
    # head_dim 128 with whole-page blocks: 168 VGPRs or fewer, so a CU can
    # hold three 4-wave workgroups when the grid oversubscribes it (C5).
    r = next(r for r in rows if r["template"] == "<128, 1, 0, 0>")
    assert r["occupancy"] >= 3 and r["vgpr"] + r.get("agpr", 0) <= 168

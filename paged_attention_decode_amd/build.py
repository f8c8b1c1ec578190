"""Build the native parts of the package in-tree.

Four shared libraries, all written next to this file (and one test program,
below):

* ``libpa_decode.so`` - the C-ABI library (``include/pa_decode.h``): gfx950
  kernels plus ``extern "C"`` entry points, compiled by ``hipcc`` from
  ``csrc/pa_decode.hip``.
* ``_pa_decode_ext<EXT_SUFFIX>`` - the thin PyTorch binding
  (``csrc/pa_torch.cpp``), host-only C++ compiled by ``g++`` against
  PyTorch's headers and linked to ``libpa_decode.so`` through an
  ``$ORIGIN`` rpath.
* ``libpa_probe.so`` - bandwidth probes for the roofline report
  (``csrc/pa_probe.hip``, ``roofline.py``); not on the decode path.
* ``libpa_decode_tl.so`` - the same source as ``libpa_decode.so`` compiled
  with ``-DPAD_TIMELINE``: every workgroup stamps the phases of its path
  (``include/pa_decode_timeline.h``) for ``profile_run --timeline``.
  Measurement only; the decode path never loads it.

And one test program: ``tests/_bin/capi_consumer`` (``tests/capi_consumer.cpp``,
host C++ linked to ``libpa_decode.so`` and the HIP runtime), a compiled
caller of the C ABI that ``tests/test_capi_consumer.py`` runs.

Usage: ``python -m paged_attention_decode_amd.build`` (or ``build()`` from
``__graft_entry__``).  Every call recompiles; the three hipcc builds run in
parallel.
"""

from __future__ import annotations

import os
import shlex
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

CAPI_LIB = os.path.join(PKG_DIR, "libpa_decode.so")
PROBE_LIB = os.path.join(PKG_DIR, "libpa_probe.so")
TIMELINE_LIB = os.path.join(PKG_DIR, "libpa_decode_tl.so")
CONSUMER_BIN = os.path.join(REPO_DIR, "tests", "_bin", "capi_consumer")
EXT_NAME = "_pa_decode_ext"
EXT_LIB = os.path.join(PKG_DIR, EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))

# Device code: gfx950 only; packed-FP32 VALU forms are disabled.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the online-softmax rescale is VALU work on
    # them, and AGPR<->VGPR copies around it cost more than they save.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]


def _run(cmd: list[str]) -> None:
    print("+ " + " ".join(shlex.quote(c) for c in cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    lines = [ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln]
    if lines:
        print("\n".join(lines), flush=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {cmd[0]}")


def build_capi() -> str:
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    tmp = CAPI_LIB + ".tmp"
    _run([hipcc, *HIP_FLAGS, f"-I{INCLUDE}", os.path.join(CSRC, "pa_decode.hip"), "-o", tmp])
    os.replace(tmp, CAPI_LIB)
    return CAPI_LIB


def build_timeline() -> str:
    """libpa_decode_tl.so: the decode library with per-workgroup phase stamps (measurement only)."""
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    tmp = TIMELINE_LIB + ".tmp"
    _run([hipcc, *HIP_FLAGS, "-DPAD_TIMELINE", f"-I{INCLUDE}", os.path.join(CSRC, "pa_decode.hip"), "-o", tmp])
    os.replace(tmp, TIMELINE_LIB)
    return TIMELINE_LIB


def build_probe() -> str:
    """libpa_probe.so: the bandwidth probes of the roofline report (roofline.py)."""
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    tmp = PROBE_LIB + ".tmp"
    _run([hipcc, *HIP_FLAGS, os.path.join(CSRC, "pa_probe.hip"), "-o", tmp])
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def build_torch_ext() -> str:
    import torch
    from torch.utils import cpp_extension

    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    includes = cpp_extension.include_paths(device_type="cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = EXT_LIB + ".tmp"
    cmd = [
        os.environ.get("CXX", "g++"),
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-w",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        f"-DTORCH_EXTENSION_NAME={EXT_NAME}",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        f"-I{INCLUDE}",
        *[f"-I{p}" for p in includes],
        f"-I{sysconfig.get_paths()['include']}",
        os.path.join(CSRC, "pa_torch.cpp"),
        "-o",
        tmp,
        f"-L{PKG_DIR}",
        "-lpa_decode",
        f"-L{torch_lib}",
        "-ltorch_python",
        "-ltorch",
        "-ltorch_cpu",
        "-lc10_hip",
        "-lc10",
        "-lamdhip64",
        "-Wl,-rpath,$ORIGIN",
        f"-Wl,-rpath,{torch_lib}",
    ]
    _run(cmd)
    os.replace(tmp, EXT_LIB)
    return EXT_LIB


def build_capi_consumer() -> str:
    """tests/_bin/capi_consumer: a compiled C ABI caller for tests/test_capi_consumer.py (host code only)."""
    os.makedirs(os.path.dirname(CONSUMER_BIN), exist_ok=True)
    tmp = CONSUMER_BIN + ".tmp"
    _run([
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__=1", f"-I{ROCM}/include",
        f"-I{INCLUDE}", os.path.join(REPO_DIR, "tests", "capi_consumer.cpp"), "-o", tmp, f"-L{PKG_DIR}",
        "-lpa_decode", f"-L{ROCM}/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN/../../paged_attention_decode_amd",
        f"-Wl,-rpath,{ROCM}/lib",
    ])
    os.replace(tmp, CONSUMER_BIN)
    return CONSUMER_BIN


def build_all() -> list[str]:
    with ThreadPoolExecutor(max_workers=3) as pool:
        hip = [pool.submit(build_capi), pool.submit(build_timeline), pool.submit(build_probe)]
        capi = hip[0].result()
        ext = build_torch_ext()  # links against libpa_decode.so
        consumer = build_capi_consumer()
        return [capi, ext, consumer, hip[1].result(), hip[2].result()]


if __name__ == "__main__":
    for path in build_all():
        print("built", path)
    sys.exit(0)

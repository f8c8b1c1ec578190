"""Register and scratch use of every decode-kernel instantiation, from the compiler.

Compiles ``csrc/pa_decode.hip`` for gfx950 (device code only, the product
flags of ``build.py``) with ``-Rpass-analysis=kernel-resource-usage`` and
parses the remarks: per kernel VGPRs, AGPRs, SGPRs, scratch bytes per lane,
SGPR and VGPR spill counts, occupancy (waves per SIMD) and static LDS.

SGPR spills go to lanes of a VGPR (``v_writelane``), not to memory; VGPR
spills and a non-zero scratch size mean scratch-memory traffic, which a
bandwidth-bound kernel pays for in its loop.

Usage: ``python -m paged_attention_decode_amd.resource_usage [--define NAME]``.
"""

from __future__ import annotations

import argparse
import os
import re
import subprocess

from . import build

FIELDS = {
    "VGPRs": "vgpr",
    "AGPRs": "agpr",
    "TotalSGPRs": "sgpr",
    "ScratchSize [bytes/lane]": "scratch",
    "SGPRs Spill": "sgpr_spill",
    "VGPRs Spill": "vgpr_spill",
    "Occupancy [waves/SIMD]": "occupancy",
    "LDS Size [bytes/block]": "lds",
}


def _demangle_args(name: str) -> str:
    # _ZN3pad17pad_phase1_kernelILi128ELi1ELi0ELi0ELi0EEEvNS_10Phase1ArgsE -> <128, 1, 0, 0> (fp16 caches);
    # a fifth argument of 1-5 is printed as e4m3fn / e5m2 (fp8 caches, fp16 q),
    # bf16, e4m3fn/bf16 / e5m2/bf16 (fp8 caches, bfloat16 q).
    args = re.findall(r"Li(\d+)E", name)
    if len(args) == 5:
        kvf = args.pop()
        if kvf != "0":
            args.append({"1": "e4m3fn", "2": "e5m2", "3": "bf16", "4": "e4m3fn/bf16",
                         "5": "e5m2/bf16"}.get(kvf, kvf))
    return "<" + ", ".join(args) + ">" if args else name


def collect(defines: tuple[str, ...] = ()) -> list[dict]:
    """One dict per kernel of pa_decode.hip (name, template args and FIELDS)."""
    hipcc = os.path.join(build.ROCM, "bin", "hipcc")
    flags = [f for f in build.HIP_FLAGS if f != "-shared"]
    cmd = [hipcc, *flags, *[f"-D{d}" for d in defines], f"-I{build.INCLUDE}", "--cuda-device-only", "-c",
           os.path.join(build.CSRC, "pa_decode.hip"), "-o", os.devnull, "-Rpass-analysis=kernel-resource-usage"]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError("compile failed:\n" + proc.stdout[-4000:])
    rows: list[dict] = []
    for line in proc.stdout.splitlines():
        m = re.search(r"remark:\s+(.*?): (.*?) \[-Rpass-analysis", line)
        if not m:
            continue
        key, val = m.group(1).strip(), m.group(2).strip()
        if key == "Function Name":
            rows.append({"name": val, "template": _demangle_args(val)})
        elif rows and key in FIELDS:
            rows[-1][FIELDS[key]] = int(val)
    return rows


def table(rows: list[dict]) -> str:
    out = [f"{'kernel':22s} {'template':18s} {'VGPR':>4s} {'AGPR':>4s} {'SGPR':>4s} {'scratch':>7s} "
           f"{'sgpr_spill':>10s} {'vgpr_spill':>10s} {'waves/SIMD':>10s} {'LDS':>5s}"]
    for r in rows:
        kern = next((k for k in ("pad_phase1_kernel", "pad_plan_kernel", "pad_zero_i32_kernel") if k in r["name"]), r["name"][:22])
        tmpl = r["template"] if r["template"].startswith("<") else "-"
        out.append(f"{kern:22s} {tmpl:18s} {r.get('vgpr', 0):4d} {r.get('agpr', 0):4d} "
                   f"{r.get('sgpr', 0):4d} {r.get('scratch', 0):7d} {r.get('sgpr_spill', 0):10d} "
                   f"{r.get('vgpr_spill', 0):10d} {r.get('occupancy', 0):10d} {r.get('lds', 0):5d}")
    return "\n".join(out)


def main() -> None:
    p = argparse.ArgumentParser()
    p.add_argument("--define", action="append", default=[], help="extra -D for the compile (e.g. PAD_TIMELINE)")
    a = p.parse_args()
    rows = collect(tuple(a.define))
    print(table(rows))
    phase1 = [r for r in rows if "pad_phase1_kernel" in r["name"]]
    spilled = [r for r in phase1 if r.get("vgpr_spill", 0) or r.get("scratch", 0)]
    print(f"\n{len(phase1)} pad_phase1_kernel instantiations; {len(spilled)} with VGPR spills or scratch")


if __name__ == "__main__":
    main()

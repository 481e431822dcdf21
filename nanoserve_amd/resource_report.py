"""Per-kernel register, spill, LDS and occupancy table of the gfx950 build, from the compiler's
resource-usage remarks (hipcc -Rpass-analysis=kernel-resource-usage), as a markdown table.

    python -m nanoserve_amd.resource_report > profiles/kernel_resources.md

The flags are the Makefile's. Kernel names are demangled and shortened to their template
arguments; LDS is the static allocation (kernels that size LDS at launch add a dynamic part,
noted in the last column when the kernel declares extern shared memory).
"""
from __future__ import annotations

import glob
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature",
         "-Xclang", "-packed-fp32-ops", "-Rpass-analysis=kernel-resource-usage"]
FIELDS = ("VGPRs", "AGPRs", "TotalSGPRs", "VGPRs Spill", "SGPRs Spill", "LDS Size [bytes/block]",
          "Occupancy [waves/SIMD]")


def demangle(names):
    out = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True,
                         check=True).stdout.splitlines()
    short = []
    for n in out:
        n = re.sub(r"ns::\(anonymous namespace\)::", "", n)
        n = re.sub(r"\(.*\)$", "", n)  # drop the parameter list
        short.append(n)
    return short


def kernels_of(src):
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", os.devnull]
    text = subprocess.run(cmd, capture_output=True, text=True).stderr
    rows, cur = [], None
    for line in text.splitlines():
        m = re.search(r"remark:\s+Function Name: (\S+)", line)
        if m:
            cur = {"name": m.group(1)}
            rows.append(cur)
            continue
        m = re.search(r"remark:\s+([A-Za-z \[\]/]+): (\d+)", line)
        if m and cur is not None and m.group(1).strip() in FIELDS:
            cur[m.group(1).strip()] = int(m.group(2))
    return rows


HEADER = """# Per-kernel registers, spills, LDS and occupancy (gfx950 build)

Compiler resource-usage remarks for every kernel instantiated in `nanoserve_amd/csrc/*.hip`, with the
flags the library is built with:

    python -m nanoserve_amd.resource_report > profiles/kernel_resources.md

VGPR / AGPR: vector / accumulation registers per lane (the waves on a SIMD share 512 per lane);
waves/SIMD is the compiler's occupancy bound from registers and LDS. Static LDS excludes the
LDS that the W4 GEMV kernels (w4_gemv.hip, w4_packed.hip) size at launch for the activation.
"""


def main():
    srcs = sorted(glob.glob(os.path.join(HERE, "csrc", "*.hip")))
    print(HEADER)
    print("| source | kernel | VGPR | AGPR | SGPR | VGPR spill | SGPR spill | static LDS (B) "
          "| waves/SIMD |")
    print("|---|---|---:|---:|---:|---:|---:|---:|---:|")
    for src in srcs:
        rows = [r for r in kernels_of(src) if r["name"].startswith("_Z")]
        if not rows:
            continue
        for r, name in zip(rows, demangle([r["name"] for r in rows])):
            print(f"| {os.path.basename(src)} | `{name}` | {r.get('VGPRs', '')} | "
                  f"{r.get('AGPRs', '')} | {r.get('TotalSGPRs', '')} | {r.get('VGPRs Spill', '')} | "
                  f"{r.get('SGPRs Spill', '')} | {r.get('LDS Size [bytes/block]', '')} | "
                  f"{r.get('Occupancy [waves/SIMD]', '')} |")
    sys.stdout.flush()


if __name__ == "__main__":
    main()

"""Build the native library in-tree: garuda_amd/libgaruda_moe.so for gfx950.

hipcc cross-compiles without a GPU, so this runs anywhere the ROCm toolchain is.
`python -m garuda_amd.build` or `garuda_amd.build.build()`.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libgaruda_moe.so"
ARCH = os.environ.get("GMOE_ARCH", "gfx950")

SOURCES = ["gmoe_kernels.hip", "gmoe_api.cpp", "gmoe_quant.cpp"]

COMMON = [
    "-O3", "-fPIC", "-std=c++20", "-ffp-contract=off", "-fno-fast-math",
    "-Wall", "-Wno-unused-function",
]
# Packed-FP32 instructions are kept out of the device code entirely.
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        sys.stderr.write(out + "\n")
        raise RuntimeError(f"build step failed: {' '.join(cmd)}")


def build(verbose: bool = False) -> Path:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    objs = []
    for src in SOURCES:
        obj = objdir / (src + ".o")
        cmd = [hipcc, *COMMON, "-c", str(CSRC / src), "-o", str(obj)]
        if src.endswith(".hip"):
            cmd[1:1] = DEVICE
        else:
            cmd[1:1] = ["-D__HIP_PLATFORM_AMD__"]
        if verbose:
            print(" ".join(cmd))
        _run(cmd)
        objs.append(str(obj))
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *objs, "-lpthread"])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))

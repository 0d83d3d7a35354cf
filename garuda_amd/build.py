"""Build the native library in-tree: garuda_amd/libgaruda_moe.so for gfx950.

hipcc cross-compiles without a GPU, so this runs anywhere the ROCm toolchain is.
`python -m garuda_amd.build` or `garuda_amd.build.build()`.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libgaruda_moe.so"
ARCH = os.environ.get("GMOE_ARCH", "gfx950")

SOURCES = ["gmoe_kernels.hip", "gmoe_api.cpp", "gmoe_quant.cpp", "gmoe_gguf.cpp", "gmoe_predict.cpp", "gmoe_kv.cpp",
           "gmoe_attn.hip", "gmoe_glue.hip", "gmoe_model.cpp", "gmoe_noalloc.hip", "gmoe_l2.cpp"]
# gmoe_units.hip is built once per block type (ggml type ids), each object holding one
# type's expert kernels; gmoe_prefill.hip likewise for the types with MFMA prefill.
UNIT_TYPES = {"f32": 0, "f16": 1, "q4_0": 2, "q8_0": 8, "q2_k": 10, "q3_k": 11, "q4_k": 12, "q5_k": 13, "q6_k": 14}
PREFILL_TYPES = {k: v for k, v in UNIT_TYPES.items() if k != "f32"}

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


def _jobs(hipcc: str, objdir: Path) -> list[tuple[list[str], Path]]:
    jobs = []
    for src in SOURCES:
        obj = objdir / (src + ".o")
        extra = DEVICE if src.endswith(".hip") else ["-D__HIP_PLATFORM_AMD__"]
        jobs.append(([hipcc, *extra, *COMMON, "-c", str(CSRC / src), "-o", str(obj)], obj))
    for name, qt in UNIT_TYPES.items():
        obj = objdir / f"gmoe_units_{name}.o"
        jobs.append(([hipcc, *DEVICE, *COMMON, f"-DGMOE_QT={qt}", "-c", str(CSRC / "gmoe_units.hip"), "-o", str(obj)], obj))
    for name, qt in PREFILL_TYPES.items():
        obj = objdir / f"gmoe_prefill_{name}.o"
        jobs.append(([hipcc, *DEVICE, *COMMON, f"-DGMOE_QT={qt}", "-c", str(CSRC / "gmoe_prefill.hip"), "-o", str(obj)], obj))
    return jobs


def build(verbose: bool = False) -> Path:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    jobs = _jobs(hipcc, objdir)
    if verbose:
        for cmd, _ in jobs:
            print(" ".join(cmd))
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        list(ex.map(lambda j: _run(j[0]), jobs))
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *[str(o) for _, o in jobs], "-lpthread"])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))

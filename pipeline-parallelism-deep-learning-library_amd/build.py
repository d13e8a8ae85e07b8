"""Builds liblinalg_hip.so (host planner + gfx950 kernels) in place.

Every source is compiled with hipcc for gfx950 only. Device code is built with
`-ffp-contract=off` (alpha*acc and beta*C round separately, as the reference's scalar rules
are written) and with packed-FP32 instruction selection disabled. Run as a script or call
`build()`; it always recompiles.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
OBJ = HERE / "_build"
LIB = HERE / "liblinalg_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = [
    "abi.cpp",
    "backend.cpp",
    "contraction.cpp",
    "permutation.cpp",
    "wire.cpp",
    "contraction_kernels.hip",
    "contraction_f16_kernels.hip",
    "permutation_kernels.hip",
    "training_kernels.hip",
]

COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
          f"-I{REPO / 'include'}", f"-I{CSRC}"]
DEVICE = [f"--offload-arch={ARCH}", "-ffp-contract=off",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _compile(src: str) -> Path:
    path = CSRC / src
    out = OBJ / (src + ".o")
    cmd = [HIPCC, *COMMON]
    if src.endswith(".hip"):
        cmd += DEVICE
    cmd += ["-c", str(path), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return out


def build(verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *[str(o) for o in objs]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

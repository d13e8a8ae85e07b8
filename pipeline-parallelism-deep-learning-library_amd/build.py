"""Builds liblinalg_hip.so (host planner + gfx950 kernels) in place.

Every source is compiled with hipcc for gfx950 only. Device code is built with
`-ffp-contract=off` (alpha*acc and beta*C round separately, as the reference's scalar rules
are written) and with packed-FP32 instruction selection disabled. Run as a script or call
`build()`; it always recompiles.

`python build.py --host-sanitize DIR` builds a second library into DIR whose host code
(planner, validation, wire parser, backend checks) carries AddressSanitizer and
UndefinedBehaviorSanitizer, device code unchanged; the CPU test suite runs against it with
  LD_PRELOAD=<clang asan runtime> PYTHONMALLOC=malloc ASAN_OPTIONS=detect_leaks=0 \
  LINALG_HIP_LIB=DIR/liblinalg_hip.so python -m pytest tests -m "not gpu"
(the runtime: /opt/rocm/llvm/lib/clang/<version>/lib/linux/libclang_rt.asan-x86_64.so).
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
    "contraction_noalloc.hip",
    "contraction_f16_kernels.hip",
    "permutation_kernels.hip",
    "training_kernels.hip",
    "backend_gemm16_kernels.hip",
]

COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
          f"-I{REPO / 'include'}", f"-I{CSRC}"]
DEVICE = [f"--offload-arch={ARCH}", "-ffp-contract=off",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


SANITIZE = ["-Xarch_host", "-fsanitize=address,undefined", "-Xarch_host",
            "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer", "-g"]


def _compile(src: str, obj: Path = OBJ, sanitize: bool = False) -> Path:
    path = CSRC / src
    out = obj / (src + ".o")
    cmd = [HIPCC, *COMMON]
    if src.endswith(".hip"):
        cmd += DEVICE
    elif sanitize:
        cmd += SANITIZE
    cmd += ["-c", str(path), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return out


def check_stubs(lib: Path) -> None:
    """Fails when a kernel's host-side launch stub is left undefined: clang emits no stub for a
    kernel template whose host-side instantiation it drops, and the library would then load
    nowhere."""
    res = subprocess.run(["nm", "-D", "--undefined-only", str(lib)], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"nm failed on {lib}: {res.stderr}")
    missing = [ln.split()[-1] for ln in res.stdout.splitlines() if "__device_stub__" in ln]
    if missing:
        raise RuntimeError(f"{lib}: kernels without a launch stub: {missing}")


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
    check_stubs(tmp)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def build_host_sanitized(out_dir: Path) -> Path:
    out_dir = Path(out_dir)
    obj = out_dir / "_build"
    obj.mkdir(parents=True, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as pool:
        objs = list(pool.map(lambda s: _compile(s, obj, True), SOURCES))
    lib = out_dir / "liblinalg_hip.so"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-shared-libasan",
           "-Xarch_host", "-fsanitize=address,undefined", "-o", str(lib), *[str(o) for o in objs]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    print(f"built {lib}")
    return lib


if __name__ == "__main__":
    if len(sys.argv) == 3 and sys.argv[1] == "--host-sanitize":
        build_host_sanitized(Path(sys.argv[2]))
    else:
        build(verbose=True)
    sys.exit(0)

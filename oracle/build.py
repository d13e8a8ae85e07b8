"""Builds oracle/liboracle.so from oracle.c with gcc.

-O2 -ffp-contract=off and no fast-math: every multiply and add rounds once, in the order
written, which is what the restated reference loops require.
"""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent


def build() -> Path:
    out = HERE / "liboracle.so"
    tmp = HERE / "liboracle.so.tmp"
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-std=c11", "-fPIC", "-shared",
           "-pthread", str(HERE / "oracle.c"), "-o", str(tmp), "-lm"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed: {' '.join(cmd)}\n{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build())

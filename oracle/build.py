"""Build recipe for the CPU oracle (test infrastructure only).

gcc -O2 -ffp-contract=off -fPIC -shared oracle/aq_oracle.c -> oracle/_build/liboracle.so
The reference tree's own kernels are CUDA and cannot be compiled in this
image (no nvcc), so there is no oracle/_ref build.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "_build" / "liboracle.so"
SRC = HERE / "aq_oracle.c"
FLAGS = ["-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
         "-Wall", "-Wno-unused-function"]


def build() -> Path:
    cc = shutil.which("gcc") or "gcc"
    OUT.parent.mkdir(exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    res = subprocess.run([cc, *FLAGS, str(SRC), "-o", str(tmp), "-lm"],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())

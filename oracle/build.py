"""Build the CPU oracle (test infrastructure only) into oracle/liboracle.so.

gcc -O2 -fopenmp on oracle.c. The reference itself (Rust/candle) cannot be
compiled in this image, so there is no oracle/_ref build.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"


def build() -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-fopenmp", "-fPIC", "-shared", "-std=c11",
           "-Wall", "-o", str(tmp), str(HERE / "oracle.c"), "-lm"]
    subprocess.run(cmd, check=True)
    tmp.replace(LIB)
    return LIB


if __name__ == "__main__":
    print(build())

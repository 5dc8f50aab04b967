"""Build tests/cpp/backend_tests: the C++ mirror's tests (include/vapi_kv.hpp)
linked against vapi_amd/libvapi_kv.so. Host code only (hipcc for the HIP
runtime headers); the binary finds the library through its rpath.

Usage: python tests/cpp/build.py
"""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
OUT = HERE / "_build" / "backend_tests"


def build() -> Path:
    OUT.parent.mkdir(exist_ok=True)
    tmp = OUT.with_suffix(".tmp")
    cmd = ["/opt/rocm/bin/hipcc", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror",
           f"-I{ROOT / 'include'}", str(HERE / "backend_tests.cpp"), "-o", str(tmp),
           f"-L{ROOT / 'vapi_amd'}", "-lvapi_kv", "-Wl,-rpath,$ORIGIN/../../../vapi_amd"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("build of backend_tests failed")
    tmp.replace(OUT)
    return OUT


if __name__ == "__main__":
    print(build())

"""Build tests/cpp/backend_tests: the C++ mirror's tests (include/vapi_kv.hpp)
linked against vapi_amd/libvapi_kv.so. Host code only (hipcc for the HIP
runtime headers); the binary finds the library through its rpath.

Usage: python tests/cpp/build.py
"""
from __future__ import annotations

import hashlib
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
OUT = HERE / "_build" / "backend_tests"
STAMP = HERE / "_build" / "backend_tests.sources"
# What the binary is compiled from: a binary built against another version
# of the C header passes descriptors of another layout to the library.
SOURCES = [ROOT / "include" / "vapi_kv.h", ROOT / "include" / "vapi_kv.hpp",
           HERE / "backend_tests.cpp"]


def sources_digest() -> str:
    h = hashlib.sha256()
    for p in SOURCES:
        h.update(p.read_bytes())
    return h.hexdigest()


def is_current() -> bool:
    """The binary exists and was built from the sources as they are now."""
    return OUT.exists() and STAMP.exists() and STAMP.read_text().strip() == sources_digest()


def build() -> Path:
    OUT.parent.mkdir(exist_ok=True)
    digest = sources_digest()
    tmp = OUT.with_suffix(".tmp")
    cmd = ["/opt/rocm/bin/hipcc", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror",
           f"-I{ROOT / 'include'}", str(HERE / "backend_tests.cpp"), "-o", str(tmp),
           f"-L{ROOT / 'vapi_amd'}", "-lvapi_kv", "-Wl,-rpath,$ORIGIN/../../../vapi_amd"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("build of backend_tests failed")
    tmp.replace(OUT)
    STAMP.write_text(digest + "\n")
    return OUT


if __name__ == "__main__":
    print(build())

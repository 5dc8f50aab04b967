"""Build libvapi_kv.so (gfx950) in-tree with hipcc.

Usage: python -m vapi_amd.build        (or vapi_amd.build.build() from Python)

Every HIP source is compiled for gfx950 only, with packed-FP32 instruction
selection turned off (-Xclang -target-feature -Xclang -packed-fp32-ops), and
linked into vapi_amd/libvapi_kv.so next to this file.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
ROOT = HERE.parent
LIB = HERE / "libvapi_kv.so"
# The benchmark's HBM ceiling probes, outside the product library.
PROBE_LIB = HERE / "libvapi_probe.so"
PROBE_SOURCES = ["probes.hip"]
OBJ_DIR = HERE / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
]

SOURCES = ["kv_ops.hip", "attention.hip", "attn_decode.hip", "attn_prefill.hip",
           "attn_prefill_f32.hip", "attn_generic.hip", "host.cpp", "spill.cpp"]

# The MFMA attention kernels never produce NaN from finite K/V/Q (masked
# scores are -inf, running maxima start finite), so fmaxf on MFMA results
# needs no operand quieting: -fno-honor-nans drops one instruction per score.
EXTRA_FLAGS = {"attn_decode.hip": ["-fno-honor-nans", "-Rpass-analysis=kernel-resource-usage"],
               "attn_prefill.hip": ["-fno-honor-nans", "-Rpass-analysis=kernel-resource-usage"],
               "attn_prefill_f32.hip": ["-fno-honor-nans",
                                        "-Rpass-analysis=kernel-resource-usage"]}

# The prefill kernel's step barrier counts its own vector-memory operations
# (the direct loads into LDS) with an explicit vmcnt wait, and the decode
# publishes its partials after an explicit vmcnt(0); a register spill would
# add scratch traffic to those counts (and slow the stream), so a build
# whose attention kernels use scratch is refused.
NO_SCRATCH = {"attn_prefill.hip": ("paged_prefill_tiled", "paged_mixed_stream"),
              "attn_decode.hip": ("paged_decode_stream",),
              "attn_prefill_f32.hip": ("paged_prefill_f32",)}


def _check_no_scratch(src: Path, remarks: str) -> None:
    kernels = NO_SCRATCH.get(src.name)
    if not kernels:
        return
    current = None
    for line in remarks.splitlines():
        if "Function Name:" in line:
            current = line.split("Function Name:")[1].split()[0]
        elif "ScratchSize" in line and current and any(k in current for k in kernels):
            size = int(line.split("ScratchSize [bytes/lane]:")[1].split()[0])
            if size != 0:
                raise RuntimeError(f"{current} uses {size} bytes of scratch per lane; its "
                                   "explicit vmcnt waits assume it uses none")


def _compile(src: Path, obj: Path) -> None:
    cmd = [HIPCC, *COMMON_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature;
    # that is expected and harmless, so only real failures are reported.
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed on {src.name}")
    _check_no_scratch(src, res.stderr)


def _link(objs, out: Path) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *[str(o) for o in objs]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"link of {out.name} failed")
    os.replace(tmp, out)


def build(verbose: bool = False) -> Path:
    """Compile every source and link libvapi_kv.so (and the benchmark's
    libvapi_probe.so). Always rebuilds."""
    OBJ_DIR.mkdir(exist_ok=True)
    jobs = [(CSRC / n, OBJ_DIR / (Path(n).stem + ".o")) for n in SOURCES + PROBE_SOURCES]
    with ThreadPoolExecutor(max_workers=min(len(jobs), 4)) as ex:
        list(ex.map(lambda j: _compile(*j), jobs))
    _link([o for s, o in jobs if s.name in SOURCES], LIB)
    _link([o for s, o in jobs if s.name in PROBE_SOURCES], PROBE_LIB)
    if verbose:
        print(f"built {LIB} and {PROBE_LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)

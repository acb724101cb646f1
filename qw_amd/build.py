"""Build libqwattn.so (gfx950) in-tree with hipcc.

    python -m qw_amd.build        # or qw_amd.build.build() from Python

Every HIP source under qw_amd/csrc is compiled for gfx950 only and linked
into qw_amd/libqwattn.so. Packed-fp32 VALU ops are disabled
(-target-feature -packed-fp32-ops) and no fast-math flag is used: the
quantizer relies on IEEE division and round-half-even.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libqwattn.so")
BUILD_DIR = os.path.join(HERE, "_build")
ARCH = "gfx950"

SOURCES = ["kv_cache.hip", "attend_decode.hip", "attend_block.hip", "dlsa.hip", "dlsa_typed.hip",
           "sdpa_general.hip", "dlsa_select.hip", "rope.hip", "turbo4.hip", "abi.hip"]
# The measurement library (read-floor and copy kernels), loaded by bench.py only.
CEIL_SOURCES = ["ceiling.hip"]
CEIL_OUT = os.path.join(HERE, "libqwceil.so")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm required to build libqwattn.so)")
    return path


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", os.path.join(ROOT, "include"), "-I", CSRC,
           "-c", os.path.join(CSRC, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr}")
    if proc.stderr.strip():
        # Warnings are surfaced, not hidden.
        sys.stderr.write(proc.stderr)
    return obj


def _link(objs, out: str) -> None:
    tmp = out + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, out)


def build(verbose: bool = False) -> str:
    """Compile every source and link libqwattn.so (and the measurement library
    libqwceil.so); always rebuilds."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = SOURCES + CEIL_SOURCES
    jobs = min(len(srcs), max(1, (os.cpu_count() or 2)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = dict(zip(srcs, ex.map(_compile, srcs)))
    _link([objs[s] for s in SOURCES], OUT)
    _link([objs[s] for s in CEIL_SOURCES], CEIL_OUT)
    if verbose:
        print(f"built {OUT} and {CEIL_OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)

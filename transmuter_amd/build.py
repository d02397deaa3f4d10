"""Builds libtmhip.so, the gfx950 HIP library of the quantized-weight operators, in-tree.

    python -m transmuter_amd.build          # or: python transmuter_amd/build.py

Each csrc/*.hip file compiles to an object under transmuter_amd/_build/ (in parallel), and the
objects link into transmuter_amd/libtmhip.so. The code targets gfx950 only. Packed f32 vector
instructions are disabled (-packed-fp32-ops); the warning the host pass prints about that
feature is expected.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libtmhip.so")
ARCH = "gfx950"

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc was not found; the HIP library cannot be built")
    return path


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


# Per-file flags. The decode GEMV's kernels (and the gather, DequantizeLinear and MatMulInteger
# kernels) take their leading arguments preloaded into SGPRs at wave launch (gfx950 kernarg
# preloading), so a wavefront's first loads do not wait on a kernel-argument fetch (0.38 us of a
# 2.8 us launch at the Qwen3-0.6B projection shapes).
PRELOAD = ["-mllvm", "-amdgpu-kernarg-preload-count=8"]
EXTRA = {"tmh_gemv.hip": PRELOAD, "tmh_bench.hip": PRELOAD, "tmh_quant_ops.hip": PRELOAD}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [hipcc(), *COMMON, *EXTRA.get(os.path.basename(src), []), "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> str:
    """Compiles every csrc/*.hip for gfx950 and links libtmhip.so. Returns the library path."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"linking libtmhip.so failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build()

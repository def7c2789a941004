"""Build libarm_ai_amd.so (the HIP kernels + the extern "C" boundary) for gfx950.

Run ``python -m arm_ai_amd.build`` (or ``__graft_entry__.build()``).  Every
``csrc/*.hip`` file is compiled with hipcc into ``_build/``, then linked into
``arm_ai_amd/libarm_ai_amd.so`` in the source tree, next to the loader.  The
measurement aids in ``bench_aids/`` (read-only kernels bench.py times beside
the matvec) go into a separate ``arm_ai_amd/libaq_bench.so``, so the product
library exports only the ABI of include/aq.h.

Flags: IEEE f32 arithmetic (no fast-math, no FMA contraction, so the
activation quantizers divide and round exactly as the reference's Rust code
does) and packed-FP32 instructions disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libarm_ai_amd.so")
BENCH_AIDS = os.path.join(HERE, "bench_aids")
BENCH_LIB = os.path.join(HERE, "libaq_bench.so")
ARCH = os.environ.get("ARM_AI_AMD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm is required to build libarm_ai_amd.so)")


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.relpath(src, HERE).replace(os.sep, "_") + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def _link(objs: list[str], lib: str) -> None:
    tmp = lib + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {lib} failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    aids = sorted(glob.glob(os.path.join(BENCH_AIDS, "*.hip")))
    workers = min(len(srcs) + len(aids), max(1, (os.cpu_count() or 2) // 2), 8)
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(_compile, srcs + aids))
    _link(objs[:len(srcs)], LIB)
    _link(objs[len(srcs):], BENCH_LIB)
    if verbose:
        print(f"built {LIB} and {BENCH_LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

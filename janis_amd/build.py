"""Builds libjanis_hip.so in-tree for gfx950 with hipcc.

    python -m janis_amd.build

Every HIP source under janis_amd/csrc/ is compiled separately (in parallel)
and linked into janis_amd/libjanis_hip.so, which exports only the C ABI
declared in include/janis_hip.h; bench_kernels.hip (bench.py's plain-read and
copy kernels) becomes janis_amd/libjanis_bench.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libjanis_hip.so")
SOURCES = ["runtime.hip", "qmv.hip", "qmm.hip", "gather.hip", "dequant.hip", "decode.hip", "ops.hip"]
# bench.py's measurement kernels (plain read, copy): a library of their own,
# outside the backend's C ABI
BENCH_SOURCE = "bench_kernels.hip"
BENCH_LIB = os.path.join(HERE, "libjanis_bench.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CFLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # keep the compiler from forming packed fp32 instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    "-fvisibility=hidden",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def _link(objs, out, extra=()) -> None:
    tmp = out + ".tmp"
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", tmp, *objs, *extra]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)


def build(verbose: bool = False) -> str:
    """Compile and link both libraries; always rebuilds. Returns the backend's path."""
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES) + 1, os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES + [BENCH_SOURCE]))
    _link(objs[:-1], LIB, ["-Wl,--version-script=" + os.path.join(CSRC, "exports.map")])
    _link(objs[-1:], BENCH_LIB)
    if verbose:
        print("built", LIB, "and", BENCH_LIB)
    return LIB


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

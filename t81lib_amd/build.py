"""Builds libt81_hip.so in-tree with hipcc for gfx950.

``python -m t81lib_amd.build`` (or ``__graft_entry__.build()``) compiles the
library sources of ``csrc/`` into ``t81lib_amd/libt81_hip.so``, and the
measurement kernels bench.py uses (``csrc/floors.hip``, not part of the t81lib
path) into ``t81lib_amd/libt81_floors.so``.  The libraries travel with the
source tree; nothing is installed.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libt81_hip.so")
FLOORS_LIB = os.path.join(HERE, "libt81_floors.so")
ARCH = "gfx950"

SOURCES = ["abi.hip", "pack.hip", "gemv.hip", "gemv_strip.hip", "gemm.hip", "gemm_i8.hip",
           "limb.hip", "elementwise.hip", "tq.hip", "tq_row.hip", "gemv_tq2.hip", "transpose.hip",
           "spmm.hip", "noalloc.hip"]

# -packed-fp32-ops: no v_pk_*_f32 from the compiler (they are never written by hand either).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libt81_hip.so")
    return path


def build(verbose: bool = False) -> str:
    """Compiles the libraries (always; it is the build check) and returns the path of
    libt81_hip.so.  Each source compiles to its own object in parallel, then one shared
    link per library."""
    from concurrent.futures import ThreadPoolExecutor

    objdir = os.path.join(HERE, "_obj")
    os.makedirs(objdir, exist_ok=True)
    jobs = []
    for src in SOURCES + ["floors.hip"]:
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        jobs.append((obj, [hipcc(), *HIPCC_FLAGS, "-c", "-o", obj, os.path.join(CSRC, src)]))

    def run(cmd):
        if verbose:
            print(" ".join(cmd), flush=True)
        return subprocess.run(cmd, capture_output=True, text=True)

    workers = max(1, min(len(jobs), os.cpu_count() or 1))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        results = list(pool.map(run, [cmd for _, cmd in jobs]))
    for (obj, _), proc in zip(jobs, results):
        if proc.returncode != 0:
            sys.stderr.write(proc.stdout + proc.stderr)
            raise RuntimeError(f"hipcc failed compiling {os.path.basename(obj)}")
    objs = {os.path.basename(obj): obj for obj, _ in jobs}
    floors_obj = objs.pop("floors.o")
    for lib, members in ((LIB, list(objs.values())), (FLOORS_LIB, [floors_obj])):
        tmp = lib + ".tmp"
        proc = run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *members])
        if proc.returncode != 0:
            sys.stderr.write(proc.stdout + proc.stderr)
            raise RuntimeError(f"hipcc failed linking {os.path.basename(lib)}")
        os.replace(tmp, lib)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))

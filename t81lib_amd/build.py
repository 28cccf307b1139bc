"""Builds libt81_hip.so in-tree with hipcc for gfx950.

``python -m t81lib_amd.build`` (or ``__graft_entry__.build()``) compiles every
``csrc/*.hip`` into ``t81lib_amd/libt81_hip.so``.  The library travels with the
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
ARCH = "gfx950"

SOURCES = ["abi.hip", "pack.hip", "gemv.hip", "gemm.hip", "limb.hip", "elementwise.hip"]

# -packed-fp32-ops: no v_pk_*_f32 from the compiler (they are never written by hand either).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
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
    """Compiles the library (always; it is the build check) and returns its path."""
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, "-o", tmp, *srcs]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError("hipcc failed building libt81_hip.so")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))

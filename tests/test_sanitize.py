"""Host AddressSanitizer + UndefinedBehaviorSanitizer runs (CPU only).

* The ABI's host side -- every entry point's argument checks, error text and device
  check -- built with host-only sanitizers and driven by ``tests/sanitize/abi_check.cpp``
  with rejected and extreme arguments (INT64_MIN / INT64_MAX sizes, so unguarded size
  arithmetic would overflow and abort).
* The oracle's C restatement built with ASan + UBSan, under its own tests
  (``test_oracle.py``, ``test_gguf_oracle.py``) in a child process with the gcc ASan
  runtime preloaded.

Both builds abort at the first report, so a passing run means no report.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = os.path.join(ROOT, "tests", "sanitize")
OUT = os.path.join(SAN, "_build")
OBJDIR = os.path.join(ROOT, "t81lib_amd", "_obj")


def _make(target: str) -> None:
    proc = subprocess.run(["make", "-s", "-C", SAN, target], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stdout + proc.stderr


def _asan_env() -> dict:
    env = dict(os.environ)
    # leak checking off: the HIP runtime keeps process-lifetime allocations
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1:abort_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    return env


def test_abi_host_checks_under_sanitizers():
    if not os.path.exists(os.path.join(OBJDIR, "gemm.o")):
        pytest.skip("library objects not built (run __graft_entry__.build() first)")
    if shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc not available")
    _make(os.path.join(OUT, "abi_check"))
    proc = subprocess.run([os.path.join(OUT, "abi_check")], capture_output=True, text=True,
                          env=_asan_env(), timeout=300)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert ", 0 failures" in proc.stdout, proc.stdout


def test_oracle_under_sanitizers():
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    _make(os.path.join(OUT, "liboracle_san.so"))
    runtime = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True,
                             text=True).stdout.strip()
    if not os.path.isabs(runtime) or not os.path.exists(runtime):
        pytest.skip("gcc's ASan runtime not found")
    env = _asan_env()
    env["LD_PRELOAD"] = runtime
    env["T81_ORACLE_LIB"] = os.path.join(OUT, "liboracle_san.so")
    proc = subprocess.run(
        [sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
         os.path.join(ROOT, "tests", "test_oracle.py"),
         os.path.join(ROOT, "tests", "test_gguf_oracle.py")],
        capture_output=True, text=True, env=env, cwd=ROOT, timeout=600)
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-4000:]
    assert " passed" in proc.stdout and "AddressSanitizer" not in proc.stderr

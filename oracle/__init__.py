"""CPU checkers for the packed-ternary path -- TEST INFRASTRUCTURE ONLY.

``oracle`` wraps two shared libraries built by ``oracle/Makefile``:

* ``liboracle.so`` -- the C restatement of the reference algorithm
  (``oracle/t81_oracle.c``; every function cites the reference lines it
  restates);
* ``_ref/libt81ref_*.so`` -- the reference's own ``gemm_cpu.cpp`` and limb
  headers compiled from ``/root/reference`` (present only where that tree
  was available at build time), reached through ``oracle/ref_driver.cpp``.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package.  The product package ``t81lib_amd``
never imports it and has no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# T81_ORACLE_LIB selects another build of the same sources (tests/sanitize builds one
# with AddressSanitizer + UndefinedBehaviorSanitizer and runs the oracle tests on it).
_ORACLE_SO = os.environ.get("T81_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")

TRITS = 48
TRYTES = 16

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i8p = ctypes.POINTER(ctypes.c_int8)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)


def build(reference: bool = True) -> None:
    """Runs oracle/Makefile (the reference builds only when its tree exists; the plugin
    check also needs libt81_hip.so, so build that first)."""
    targets = ["oracle"]
    if reference and os.path.isdir("/root/reference/src/linalg"):
        targets.append("ref")
        if os.path.exists(os.path.join(os.path.dirname(HERE), "t81lib_amd", "libt81_hip.so")):
            targets.append("plugin")
    subprocess.run(["make", "-s", "-C", HERE, *targets], check=True)


PLUGIN_CHECK = os.path.join(HERE, "_ref", "plugin_check")


def _ptr(a: np.ndarray, typ):
    return a.ctypes.data_as(typ)


def _load_oracle() -> ctypes.CDLL:
    if not os.path.exists(_ORACLE_SO):
        build(reference=False)
    lib = ctypes.CDLL(_ORACLE_SO)
    lib.orc_quantize_trit.restype = ctypes.c_int8
    lib.orc_quantize_trit.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_int]
    lib.orc_torch_threshold.restype = ctypes.c_float
    lib.orc_torch_threshold.argtypes = [ctypes.c_double]
    for name in ("orc_where", "orc_lerp"):
        getattr(lib, name).argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_int64]
    lib.orc_clamp.argtypes = [_f32p, _f32p, ctypes.c_int64, ctypes.c_float, ctypes.c_float]
    lib.orc_addcmul.argtypes = [_f32p, _f32p, _f32p, ctypes.c_float, _f32p, ctypes.c_int64]
    lib.orc_tryte_of.restype = ctypes.c_uint8
    lib.orc_tryte_of.argtypes = [ctypes.c_int] * 3
    lib.orc_trits_of.argtypes = [ctypes.c_uint8, _i8p]
    lib.orc_pack_rows.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_float,
                                  ctypes.c_int, _u8p]
    lib.orc_pack_trits_rows.argtypes = [_i8p, ctypes.c_int64, ctypes.c_int64, _u8p]
    lib.orc_pack_cols.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_float,
                                  ctypes.c_int, _u8p]
    lib.orc_unpack.restype = ctypes.c_int
    lib.orc_unpack.argtypes = [_u8p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _i8p]
    lib.orc_mul_wide.argtypes = [_u8p, _u8p, _u8p, _u8p]
    lib.orc_tryte_table.argtypes = [_f64p]
    lib.orc_limb_to_double.restype = ctypes.c_double
    lib.orc_limb_to_double.argtypes = [_u8p]
    lib.orc_multiply_to_double.restype = ctypes.c_double
    lib.orc_multiply_to_double.argtypes = [_u8p, _u8p]
    lib.orc_gemm_limb.restype = ctypes.c_int
    lib.orc_gemm_limb.argtypes = [_u8p, _u8p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_float, ctypes.c_float]
    lib.orc_trit_matmul_f64.argtypes = [_f64p, ctypes.c_int64, ctypes.c_int64, _u8p,
                                        ctypes.c_int64, _i8p, _f64p]
    lib.orc_trit_matmul_abs_f64.argtypes = lib.orc_trit_matmul_f64.argtypes
    lib.orc_trit_matmul_i64.argtypes = [_i8p, ctypes.c_int64, ctypes.c_int64, _u8p,
                                        ctypes.c_int64, _i8p, _i64p]
    lib.orc_spmm_simple.restype = ctypes.c_int
    lib.orc_spmm_simple.argtypes = [_i64p, _i32p, _i32p, ctypes.c_int64, ctypes.c_int,
                                    ctypes.c_int, _f32p, _f32p, ctypes.c_int, ctypes.c_float,
                                    ctypes.c_float]
    lib.orc_f32_to_f16_bits.restype = ctypes.c_uint16
    lib.orc_f32_to_f16_bits.argtypes = [ctypes.c_float]
    lib.orc_f16_bits_to_f32.restype = ctypes.c_float
    lib.orc_f16_bits_to_f32.argtypes = [ctypes.c_uint16]
    lib.orc_tq_block_bytes.restype = ctypes.c_int
    lib.orc_tq_block_bytes.argtypes = [ctypes.c_int]
    lib.orc_tq_quantize.restype = ctypes.c_int
    lib.orc_tq_quantize.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_float,
                                    ctypes.c_int, _u8p]
    lib.orc_tq_dequantize.restype = ctypes.c_int
    lib.orc_tq_dequantize.argtypes = [_u8p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, _f32p]
    lib.orc_tq2_matmul_f64.argtypes = [_f64p, ctypes.c_int64, ctypes.c_int64, _u8p,
                                       ctypes.c_int64, _f64p, _f64p]
    lib.orc_tq1r_scale.restype = ctypes.c_float
    lib.orc_tq1r_scale.argtypes = [_f32p, ctypes.c_int64]
    lib.orc_tq1r_quantize_row.restype = ctypes.c_float
    lib.orc_tq1r_quantize_row.argtypes = [_f32p, ctypes.c_int64, ctypes.c_float, ctypes.c_float,
                                          _u16p]
    lib.orc_tq1r_dequantize_row.argtypes = [_u16p, ctypes.c_int64, ctypes.c_float, _f32p]
    lib.orc_tq1r_dequant_tensor.restype = ctypes.c_int
    lib.orc_tq1r_dequant_tensor.argtypes = [_u8p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                            ctypes.c_int64, ctypes.c_int, _f32p]
    return lib


_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = _load_oracle()
    return _lib


# ------------------------------------------------------------------ codec --
def tryte_of(t0: int, t1: int, t2: int) -> int:
    return int(lib().orc_tryte_of(t0, t1, t2))


def trits_of(u: int) -> tuple[int, int, int]:
    out = np.zeros(3, np.int8)
    lib().orc_trits_of(u, _ptr(out, _i8p))
    return tuple(int(v) for v in out)


def quantize_trit(v: float, thr: float, mode: int = 0) -> int:
    return int(lib().orc_quantize_trit(v, thr, mode))


def torch_threshold(thr: float) -> float:
    return float(lib().orc_torch_threshold(thr))


def pack_rows(w: np.ndarray, thr: float, mode: int = 0) -> np.ndarray:
    """(rows, cols) float32 -> (rows, L, 16) uint8, reference pack_dense_matrix."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    L = (cols + TRITS - 1) // TRITS
    out = np.empty((rows, L, TRYTES), np.uint8)
    lib().orc_pack_rows(_ptr(w, _f32p), rows, cols, thr, mode, _ptr(out, _u8p))
    return out


def pack_trits_rows(t: np.ndarray) -> np.ndarray:
    t = np.ascontiguousarray(t, dtype=np.int8)
    rows, cols = t.shape
    L = (cols + TRITS - 1) // TRITS
    out = np.empty((rows, L, TRYTES), np.uint8)
    lib().orc_pack_trits_rows(_ptr(t, _i8p), rows, cols, _ptr(out, _u8p))
    return out


def pack_cols(x: np.ndarray, thr: float = 0.5, mode: int = 1) -> np.ndarray:
    """(tokens, K) float32 -> (L, tokens, 16) uint8, reference _pack_columnwise of x^T."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    tokens, k = x.shape
    L = (k + TRITS - 1) // TRITS
    out = np.empty((L, tokens, TRYTES), np.uint8)
    lib().orc_pack_cols(_ptr(x, _f32p), tokens, k, thr, mode, _ptr(out, _u8p))
    return out


def unpack(packed: np.ndarray, rows: int, cols: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    L = packed.shape[1]
    out = np.zeros((rows, cols), np.int8)
    rc = lib().orc_unpack(_ptr(packed, _u8p), rows, L, cols, _ptr(out, _i8p))
    if rc != 0:
        raise ValueError(f"unpack rejected input (code {rc})")
    return out


# ------------------------------------------------------------------- limb --
def mul_wide(a: np.ndarray, b: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    a = np.ascontiguousarray(a, np.uint8)
    b = np.ascontiguousarray(b, np.uint8)
    lo = np.empty(16, np.uint8)
    hi = np.empty(16, np.uint8)
    lib().orc_mul_wide(_ptr(a, _u8p), _ptr(b, _u8p), _ptr(lo, _u8p), _ptr(hi, _u8p))
    return lo, hi


def tryte_table() -> np.ndarray:
    out = np.empty(16 * 27, np.float64)
    lib().orc_tryte_table(_ptr(out, _f64p))
    return out.reshape(16, 27)


def limb_to_double(a: np.ndarray) -> float:
    a = np.ascontiguousarray(a, np.uint8)
    return float(lib().orc_limb_to_double(_ptr(a, _u8p)))


def multiply_to_double(a: np.ndarray, b: np.ndarray) -> float:
    a = np.ascontiguousarray(a, np.uint8)
    b = np.ascontiguousarray(b, np.uint8)
    return float(lib().orc_multiply_to_double(_ptr(a, _u8p), _ptr(b, _u8p)))


def gemm_limb(A: np.ndarray, B: np.ndarray, C: np.ndarray, M: int, N: int, K: int,
              alpha: float = 1.0, beta: float = 0.0) -> np.ndarray:
    """Reference gemm_ternary semantics; returns a new C (input C is not modified)."""
    A = np.ascontiguousarray(A, np.uint8)
    B = np.ascontiguousarray(B, np.uint8)
    out = np.array(C, dtype=np.float32, copy=True, order="C")
    rc = lib().orc_gemm_limb(_ptr(A, _u8p), _ptr(B, _u8p), _ptr(out, _f32p), M, N, K,
                             alpha, beta)
    if rc != 0:
        raise ValueError("gemm_ternary shape rejected")
    return out


# --------------------------------------------------------------- trit-dot --
def trit_matmul_f64(x: np.ndarray, w_packed: np.ndarray, K: int) -> np.ndarray:
    """out[m, n] = sum_k x[m, k] * T[n, k] in float64."""
    x = np.ascontiguousarray(x, np.float64)
    w_packed = np.ascontiguousarray(w_packed, np.uint8)
    M = x.shape[0]
    N = w_packed.shape[0]
    out = np.empty((M, N), np.float64)
    scratch = np.empty(max(K, 1), np.int8)
    lib().orc_trit_matmul_f64(_ptr(x, _f64p), M, K, _ptr(w_packed, _u8p), N,
                              _ptr(scratch, _i8p), _ptr(out, _f64p))
    return out


def trit_matmul_abs_f64(x: np.ndarray, w_packed: np.ndarray, K: int) -> np.ndarray:
    """out[m, n] = sum_k |x[m, k] * T[n, k]| -- the scale of the fp tolerances."""
    x = np.ascontiguousarray(x, np.float64)
    w_packed = np.ascontiguousarray(w_packed, np.uint8)
    M = x.shape[0]
    N = w_packed.shape[0]
    out = np.empty((M, N), np.float64)
    scratch = np.empty(max(K, 1), np.int8)
    lib().orc_trit_matmul_abs_f64(_ptr(x, _f64p), M, K, _ptr(w_packed, _u8p), N,
                                  _ptr(scratch, _i8p), _ptr(out, _f64p))
    return out


def trit_matmul_i64(x: np.ndarray, w_packed: np.ndarray, K: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.int8)
    w_packed = np.ascontiguousarray(w_packed, np.uint8)
    M = x.shape[0]
    N = w_packed.shape[0]
    out = np.empty((M, N), np.int64)
    scratch = np.empty(max(K, 1), np.int8)
    lib().orc_trit_matmul_i64(_ptr(x, _i8p), M, K, _ptr(w_packed, _u8p), N,
                              _ptr(scratch, _i8p), _ptr(out, _i64p))
    return out


# ----------------------------------------------------------- spmm_simple --
def _spmm(fn, values, rows_idx, cols_idx, rows, cols, B, C, N, alpha, beta):
    values = np.ascontiguousarray(values, np.int64)
    rows_idx = np.ascontiguousarray(rows_idx, np.int32)
    cols_idx = np.ascontiguousarray(cols_idx, np.int32)
    B = np.ascontiguousarray(B, np.float32)
    out = np.array(C, np.float32, copy=True)
    rc = fn(_ptr(values, _i64p), _ptr(rows_idx, _i32p), _ptr(cols_idx, _i32p), values.size,
            rows, cols, _ptr(B, _f32p), _ptr(out, _f32p), N, alpha, beta)
    return rc, out


def spmm_simple(values, rows_idx, cols_idx, rows: int, cols: int, B, C, N: int,
                alpha: float = 1.0, beta: float = 0.0):
    """(return code, C after the call): 0, -1 bad index (C partly updated), -2 bad dims."""
    return _spmm(lib().orc_spmm_simple, values, rows_idx, cols_idx, rows, cols, B, C, N,
                 alpha, beta)


# ------------------------------------------------------ GGUF TQ1_0 / TQ2_0 --
TQ1_0 = 34
TQ2_0 = 35
TQ_BLOCK = 256


def f32_to_f16_bits(v: float) -> int:
    return int(lib().orc_f32_to_f16_bits(float(v)))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().orc_f16_bits_to_f32(int(h)))


def tq_block_bytes(quant: int) -> int:
    return int(lib().orc_tq_block_bytes(quant))


def tq_quantize(w: np.ndarray, threshold: float, quant: int) -> np.ndarray:
    """(rows, cols) float32 -> (rows, blocks_per_row * block_bytes) uint8."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    nb = (cols + TQ_BLOCK - 1) // TQ_BLOCK
    out = np.zeros((rows, nb * tq_block_bytes(quant)), np.uint8)
    if lib().orc_tq_quantize(_ptr(w, _f32p), rows, cols, threshold, quant, _ptr(out, _u8p)):
        raise ValueError("unknown quant")
    return out


def tq_dequantize(packed: np.ndarray, rows: int, cols: int, quant: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, np.uint8)
    out = np.zeros((rows, cols), np.float32)
    if lib().orc_tq_dequantize(_ptr(packed, _u8p), rows, cols, quant, _ptr(out, _f32p)):
        raise ValueError("unknown quant")
    return out


def tq2_matmul_f64(x: np.ndarray, w_tq2: np.ndarray, K: int) -> tuple[np.ndarray, np.ndarray]:
    """(sum_k x[m,k] W[n,k], sum_k |x[m,k] W[n,k]|) in float64 over dequantized TQ2_0 rows."""
    x = np.ascontiguousarray(x, np.float64)
    w_tq2 = np.ascontiguousarray(w_tq2, np.uint8)
    M, N = x.shape[0], w_tq2.shape[0]
    out = np.empty((M, N), np.float64)
    scale = np.empty((M, N), np.float64)
    lib().orc_tq2_matmul_f64(_ptr(x, _f64p), M, K, _ptr(w_tq2, _u8p), N, _ptr(out, _f64p),
                             _ptr(scale, _f64p))
    return out, scale


# ------------------------------------- TQ1_0 row codec (gguf_quants.h) --
TQ1_TRITS_PER_BLOCK = 8
TQ1_BLOCK_ROWS = 32
TQ1R_ERRORS = {1: "buffer truncated while reading scale",
               2: "buffer truncated while skipping refinement bytes",
               3: "buffer truncated while reading quantized rows"}


def tq1r_words(n: int) -> int:
    return (int(n) + TQ1_TRITS_PER_BLOCK - 1) // TQ1_TRITS_PER_BLOCK


def tq1r_scale(v: np.ndarray) -> float:
    v = np.ascontiguousarray(v, np.float32).reshape(-1)
    return float(np.float32(lib().orc_tq1r_scale(_ptr(v, _f32p), v.size)))


def tq1r_quantize_row(v: np.ndarray, threshold: float = 0.45, scale: float = 0.0
                      ) -> tuple[float, np.ndarray]:
    """(scale used, ceil(n / 8) uint16 words) for one row."""
    v = np.ascontiguousarray(v, np.float32).reshape(-1)
    out = np.zeros(tq1r_words(v.size), np.uint16)
    used = lib().orc_tq1r_quantize_row(_ptr(v, _f32p), v.size, threshold, scale, _ptr(out, _u16p))
    return float(np.float32(used)), out


def tq1r_dequantize_row(words: np.ndarray, n: int, scale: float) -> np.ndarray:
    words = np.ascontiguousarray(words, np.uint16).reshape(-1)
    assert words.size >= tq1r_words(n)
    out = np.zeros(n, np.float32)
    lib().orc_tq1r_dequantize_row(_ptr(words, _u16p), n, scale, _ptr(out, _f32p))
    return out


def tq1r_dequant_tensor(buf, rows: int, cols: int, block_rows: int = TQ1_BLOCK_ROWS,
                        refinements: bool = False) -> tuple[int, np.ndarray]:
    """(0 or the failing check 1 / 2 / 3 of TQ1R_ERRORS, or -1 for negative sizes,
    rows x cols float32 as far as decoded)."""
    b = np.ascontiguousarray(np.frombuffer(bytes(buf), np.uint8))
    out = np.zeros((max(rows, 0), max(cols, 0)), np.float32)
    rc = lib().orc_tq1r_dequant_tensor(_ptr(b, _u8p) if b.size else None, b.size, rows, cols,
                                       block_rows, int(bool(refinements)), _ptr(out, _f32p))
    return int(rc), out


def tq1r_payload(values: np.ndarray, block_rows: int = TQ1_BLOCK_ROWS, refinements: bool = False,
                 threshold: float = 0.45) -> bytes:
    """The tensor payload dequant_tq1_0 / dequant_tq2_0 read, written with the row codec:
    per group of block_rows rows h = float16(max |v| of the group), 8 zero bytes when
    `refinements`, then each row's words from quantize_row_tq1_0 with the scale
    float(h)."""
    values = np.ascontiguousarray(values, np.float32)
    rows, cols = values.shape
    group = max(1, int(block_rows))
    parts = []
    for g0 in range(0, rows, group):
        blk = values[g0:g0 + group]
        h = f32_to_f16_bits(tq1r_scale(blk))
        parts.append(np.array([h], np.uint16).tobytes())
        if refinements:
            parts.append(bytes(8))
        s = f16_bits_to_f32(h)
        for r in range(blk.shape[0]):
            parts.append(tq1r_quantize_row(blk[r], threshold, s)[1].tobytes())
    return b"".join(parts)


# ------------------------------------------------ the compiled reference --
def _cpu_has_avx512f() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    return " avx512f" in line
    except OSError:
        pass
    return False


class Ref:
    """The reference's own CPU path (oracle/_ref), or None where it was not built."""

    def __init__(self, lib: ctypes.CDLL, variant: str):
        self.lib = lib
        self.variant = variant
        lib.t81ref_tryte_table.argtypes = [_f64p]
        for name in ("t81ref_mul_wide", "t81ref_mul_wide_scalar"):
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [_u8p, _u8p, _u8p, _u8p]
        lib.t81ref_limb_to_double.restype = ctypes.c_double
        lib.t81ref_limb_to_double.argtypes = [_u8p]
        lib.t81ref_multiply_to_double.restype = ctypes.c_double
        lib.t81ref_multiply_to_double.argtypes = [_u8p, _u8p]
        lib.t81ref_limb_from_value.restype = ctypes.c_int
        lib.t81ref_limb_from_value.argtypes = [ctypes.c_longlong, _u8p]
        lib.t81ref_limb_from_trits.restype = ctypes.c_int
        lib.t81ref_limb_from_trits.argtypes = [_i8p, _u8p]
        lib.t81ref_limb_min_max.argtypes = [_u8p, _u8p]
        lib.t81ref_random_limbs.argtypes = [ctypes.c_ulonglong, ctypes.c_int, _u8p]
        lib.t81ref_gemm_ternary.restype = ctypes.c_int
        lib.t81ref_gemm_ternary.argtypes = [_u8p, _u8p, _f32p, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_float, ctypes.c_float]
        lib.t81ref_gemm_ternary_rows.restype = ctypes.c_int
        lib.t81ref_gemm_ternary_rows.argtypes = [_u8p, _u8p, _f32p, ctypes.c_int, ctypes.c_int,
                                                 ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                 ctypes.c_float, ctypes.c_float]
        lib.t81ref_simd_path.restype = ctypes.c_char_p
        for name in ("t81ref_where", "t81ref_lerp"):
            getattr(lib, name).argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_longlong]
        lib.t81ref_clamp.argtypes = [_f32p, _f32p, ctypes.c_longlong, ctypes.c_float,
                                     ctypes.c_float]
        lib.t81ref_addcmul.argtypes = [_f32p, _f32p, _f32p, ctypes.c_float, _f32p,
                                       ctypes.c_longlong]
        lib.t81ref_tq1_compute_scale.restype = ctypes.c_float
        lib.t81ref_tq1_compute_scale.argtypes = [_f32p, ctypes.c_longlong]
        lib.t81ref_tq1_quantize_row.argtypes = [_f32p, ctypes.c_longlong, ctypes.c_float,
                                                ctypes.c_float, _u16p]
        lib.t81ref_tq1_dequantize_row.argtypes = [_u16p, ctypes.c_longlong, ctypes.c_float,
                                                  _f32p]
        lib.t81ref_tq1_half_to_float.restype = ctypes.c_float
        lib.t81ref_tq1_half_to_float.argtypes = [ctypes.c_uint16]

    def tq1_compute_scale(self, v) -> float:
        v = np.ascontiguousarray(v, np.float32).reshape(-1)
        return float(np.float32(self.lib.t81ref_tq1_compute_scale(_ptr(v, _f32p), v.size)))

    def tq1_quantize_row(self, v, threshold: float, scale: float) -> np.ndarray:
        """quantize_row_tq1_0 as it stands (the scale argument passed through)."""
        v = np.ascontiguousarray(v, np.float32).reshape(-1)
        out = np.zeros(tq1r_words(v.size), np.uint16)
        self.lib.t81ref_tq1_quantize_row(_ptr(v, _f32p), v.size, threshold, scale,
                                         _ptr(out, _u16p))
        return out

    def tq1_dequantize_row(self, words, n: int, scale: float) -> np.ndarray:
        words = np.ascontiguousarray(words, np.uint16).reshape(-1)
        out = np.zeros(n, np.float32)
        self.lib.t81ref_tq1_dequantize_row(_ptr(words, _u16p), n, scale, _ptr(out, _f32p))
        return out

    def tq1_half_to_float(self, bits: int) -> np.float32:
        return np.float32(self.lib.t81ref_tq1_half_to_float(int(bits)))

    def spmm_simple(self, values, rows_idx, cols_idx, rows: int, cols: int, B, C, N: int,
                    alpha: float = 1.0, beta: float = 0.0):
        """The reference's t81::sparse::spmm_simple: (0 or -1 if it threw, C after)."""
        fn = self.lib.t81ref_spmm_simple
        fn.restype = ctypes.c_int
        fn.argtypes = [_i64p, _i32p, _i32p, ctypes.c_longlong, ctypes.c_int, ctypes.c_int,
                       _f32p, _f32p, ctypes.c_int, ctypes.c_float, ctypes.c_float]
        return _spmm(fn, values, rows_idx, cols_idx, rows, cols, B, C, N, alpha, beta)

    def elementwise(self, op: str, a, b=None, c=None, p0: float = 0.0, p1: float = 0.0):
        """The reference's where / clamp / lerp / addcmul on Backend::CPU."""
        return _elementwise(self.lib, "t81ref_", op, a, b, c, p0, p1)

    def tryte_table(self) -> np.ndarray:
        out = np.empty(16 * 27, np.float64)
        self.lib.t81ref_tryte_table(_ptr(out, _f64p))
        return out.reshape(16, 27)

    def mul_wide(self, a, b, scalar: bool = False):
        a = np.ascontiguousarray(a, np.uint8)
        b = np.ascontiguousarray(b, np.uint8)
        lo = np.empty(16, np.uint8)
        hi = np.empty(16, np.uint8)
        fn = self.lib.t81ref_mul_wide_scalar if scalar else self.lib.t81ref_mul_wide
        if fn(_ptr(a, _u8p), _ptr(b, _u8p), _ptr(lo, _u8p), _ptr(hi, _u8p)) != 0:
            raise ValueError("reference mul_wide rejected input")
        return lo, hi

    def limb_to_double(self, a) -> float:
        a = np.ascontiguousarray(a, np.uint8)
        return float(self.lib.t81ref_limb_to_double(_ptr(a, _u8p)))

    def multiply_to_double(self, a, b) -> float:
        a = np.ascontiguousarray(a, np.uint8)
        b = np.ascontiguousarray(b, np.uint8)
        return float(self.lib.t81ref_multiply_to_double(_ptr(a, _u8p), _ptr(b, _u8p)))

    def limb_from_value(self, v: int) -> np.ndarray:
        out = np.empty(16, np.uint8)
        if self.lib.t81ref_limb_from_value(v, _ptr(out, _u8p)) != 0:
            raise ValueError("value out of range")
        return out

    def limb_from_trits(self, t) -> np.ndarray:
        t = np.ascontiguousarray(t, np.int8)
        out = np.empty(16, np.uint8)
        if self.lib.t81ref_limb_from_trits(_ptr(t, _i8p), _ptr(out, _u8p)) != 0:
            raise ValueError("invalid trits")
        return out

    def limb_min_max(self):
        lo = np.empty(16, np.uint8)
        hi = np.empty(16, np.uint8)
        self.lib.t81ref_limb_min_max(_ptr(lo, _u8p), _ptr(hi, _u8p))
        return lo, hi

    def random_limbs(self, seed: int, count: int) -> np.ndarray:
        out = np.empty((count, 16), np.uint8)
        self.lib.t81ref_random_limbs(seed, count, _ptr(out, _u8p))
        return out

    def gemm_ternary(self, A, B, C, M, N, K, alpha=1.0, beta=0.0) -> np.ndarray:
        A = np.ascontiguousarray(A, np.uint8)
        B = np.ascontiguousarray(B, np.uint8)
        out = np.array(C, dtype=np.float32, copy=True, order="C")
        rc = self.lib.t81ref_gemm_ternary(_ptr(A, _u8p), _ptr(B, _u8p), _ptr(out, _f32p),
                                          M, N, K, alpha, beta)
        if rc != 0:
            raise ValueError(f"reference gemm_ternary rejected the call ({rc})")
        return out

    def gemm_ternary_rows(self, A, B, C, M, N, K, r0, r1, alpha=1.0, beta=0.0) -> None:
        """In-place over rows [r0, r1) of C (used by the CPU baseline)."""
        rc = self.lib.t81ref_gemm_ternary_rows(_ptr(A, _u8p), _ptr(B, _u8p), _ptr(C, _f32p),
                                               M, N, K, r0, r1, alpha, beta)
        if rc != 0:
            raise ValueError(f"reference gemm_ternary rejected the call ({rc})")

    def simd_path(self) -> str:
        return self.lib.t81ref_simd_path().decode()


_ref_cache: dict = {}


def ref(variant: Optional[str] = None) -> Optional[Ref]:
    """Loads oracle/_ref/libt81ref_<variant>.so; variant defaults to avx512 when
    the host supports it (the C++ library build), else generic."""
    if variant is None:
        variant = "avx512" if _cpu_has_avx512f() else "generic"
    if variant == "avx512" and not _cpu_has_avx512f():
        return None
    if variant in _ref_cache:
        return _ref_cache[variant]
    path = os.path.join(REF_DIR, f"libt81ref_{variant}.so")
    if not os.path.exists(path):
        _ref_cache[variant] = None
        return None
    r = Ref(ctypes.CDLL(path), variant)
    _ref_cache[variant] = r
    return r


def _elementwise(lib, prefix: str, op: str, a, b=None, c=None, p0: float = 0.0, p1: float = 0.0):
    a = np.ascontiguousarray(a, np.float32)
    n = a.size
    out = np.empty_like(a)
    if op == "clamp":
        getattr(lib, prefix + "clamp")(_ptr(a, _f32p), _ptr(out, _f32p), n, p0, p1)
        return out
    b = np.ascontiguousarray(b, np.float32)
    c = np.ascontiguousarray(c, np.float32)
    if op == "addcmul":
        getattr(lib, prefix + "addcmul")(_ptr(a, _f32p), _ptr(b, _f32p), _ptr(c, _f32p), p0,
                                         _ptr(out, _f32p), n)
    else:
        getattr(lib, prefix + op)(_ptr(a, _f32p), _ptr(b, _f32p), _ptr(c, _f32p),
                                  _ptr(out, _f32p), n)
    return out


def elementwise(op: str, a, b=None, c=None, p0: float = 0.0, p1: float = 0.0) -> np.ndarray:
    """Oracle where (a=cond, b=x, c=y) / clamp (a, p0=lo, p1=hi) / lerp (a=start, b=end,
    c=weight) / addcmul (a=input, b=t1, c=t2, p0=value) over float32 arrays."""
    return _elementwise(lib(), "orc_", op, a, b, c, p0, p1)

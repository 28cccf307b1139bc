"""Loads libt81_hip.so and exposes its C ABI (include/t81_hip.h) to Python.

There is no CPU fallback: if the library is missing, or no gfx950 device is
present, every compute call raises.  Return codes map to the exception types
the reference's pybind11 binding raises (ValueError for argument errors,
RuntimeError for device errors, python/bindings.cpp:779-793).
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libt81_hip.so")

OK = 0
EINVAL_SHAPE = -1
EINVAL_K48 = -2
EINVAL_THRESHOLD = -3
EINVAL_DTYPE = -4
EINVAL_POINTER = -5
EHIP = -6
ENODEV = -7
EINVAL_INDEX = -8

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_I8 = 2
DTYPE_F16 = 3

THR_CPP = 0
THR_TORCH = 1

# every symbol include/t81_hip.h declares
EXPORTS = (
    "t81_hip_available",
    "t81_hip_last_error",
    "t81_hip_quantize_pack",
    "t81_hip_quantize",
    "t81_hip_pack_cols",
    "t81_hip_unpack",
    "t81_hip_validate_packed",
    "t81_hip_ternary_matmul",
    "t81_hip_ternary_matmul_kernel",
    "t81_hip_ternary_matmul_ws",
    "t81_hip_ternary_matmul_workspace_size",
    "t81_hip_ternary_matmul_noalloc",
    "t81_hip_gemm_ternary_limb",
    "t81_hip_where",
    "t81_hip_clamp",
    "t81_hip_lerp",
    "t81_hip_addcmul",
    "t81_hip_matmul_input_reference",
    "t81_hip_transpose_packed",
    "t81_hip_tq_block_bytes",
    "t81_hip_tq_quantize",
    "t81_hip_tq_dequantize",
    "t81_hip_tq2_matmul",
    "t81_hip_tq1_quantize_rows",
    "t81_hip_tq1_dequantize_rows",
    "t81_hip_tq1_payload_bytes",
    "t81_hip_tq1_quantize_payload",
    "t81_hip_tq1_dequantize_payload",
    "t81_hip_spmm_plan_create",
    "t81_hip_spmm_plan_apply",
    "t81_hip_spmm_plan_info",
    "t81_hip_spmm_plan_destroy",
    "t81_hip_spmm_simple",
    "t81_hip_limb_tryte_table",
)

TQ1_0 = 34
TQ2_0 = 35

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_f = ctypes.c_float
_i = ctypes.c_int


class T81HipError(RuntimeError):
    """A device-side failure reported by libt81_hip (HIP error or no gfx950 device)."""


_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def _declare(lib: ctypes.CDLL) -> None:
    lib.t81_hip_available.restype = _i
    lib.t81_hip_available.argtypes = []
    lib.t81_hip_last_error.restype = ctypes.c_char_p
    lib.t81_hip_last_error.argtypes = []
    lib.t81_hip_quantize_pack.restype = _i
    lib.t81_hip_quantize_pack.argtypes = [_vp, _i, _vp, _i64, _i64, _f, _i, _vp]
    lib.t81_hip_quantize.restype = _i
    lib.t81_hip_quantize.argtypes = [_vp, _i, _vp, _i64, _f, _i, _vp]
    lib.t81_hip_pack_cols.restype = _i
    lib.t81_hip_pack_cols.argtypes = [_vp, _i, _vp, _i64, _i64, _f, _i, _vp]
    lib.t81_hip_unpack.restype = _i
    lib.t81_hip_unpack.argtypes = [_vp, _vp, _i64, _i64, _i64, _vp]
    lib.t81_hip_validate_packed.restype = _i
    lib.t81_hip_validate_packed.argtypes = [_vp, _i64, _vp, _vp]
    lib.t81_hip_ternary_matmul.restype = _i
    lib.t81_hip_ternary_matmul.argtypes = [_vp, _i, _vp, _vp, _i64, _i64, _i64, _f, _f, _vp, _vp]
    lib.t81_hip_ternary_matmul_kernel.restype = _i
    lib.t81_hip_ternary_matmul_kernel.argtypes = [_i, _vp, _i, _vp, _vp, _i64, _i64, _i64, _f,
                                                  _f, _vp, _vp]
    lib.t81_hip_ternary_matmul_ws.restype = _i
    lib.t81_hip_ternary_matmul_ws.argtypes = [_i, _vp, _i, _vp, _vp, _i64, _i64, _i64, _f, _f,
                                              _vp, _vp, _i64, _vp]
    lib.t81_hip_ternary_matmul_workspace_size.restype = _i64
    lib.t81_hip_ternary_matmul_workspace_size.argtypes = [_i64, _i64, _i64, _i]
    lib.t81_hip_ternary_matmul_noalloc.restype = _i
    lib.t81_hip_ternary_matmul_noalloc.argtypes = [_i, _vp, _i, _vp, _vp, _i64, _i64, _i64, _f,
                                                   _f, _vp, _vp]
    lib.t81_hip_gemm_ternary_limb.restype = _i
    lib.t81_hip_gemm_ternary_limb.argtypes = [_vp, _vp, _vp, _i, _i, _i, _f, _f, _vp]
    lib.t81_hip_where.restype = _i
    lib.t81_hip_where.argtypes = [_vp, _vp, _vp, _vp, _i64, _vp]
    lib.t81_hip_clamp.restype = _i
    lib.t81_hip_clamp.argtypes = [_vp, _vp, _i64, _f, _f, _vp]
    lib.t81_hip_lerp.restype = _i
    lib.t81_hip_lerp.argtypes = [_vp, _vp, _vp, _vp, _i64, _vp]
    lib.t81_hip_addcmul.restype = _i
    lib.t81_hip_addcmul.argtypes = [_vp, _vp, _vp, _f, _vp, _i64, _vp]
    lib.t81_hip_matmul_input_reference.restype = _i
    lib.t81_hip_matmul_input_reference.argtypes = [_vp, _vp, _i, _vp, _i64, _i64, _i64, _f, _f,
                                                   _f, _vp]
    lib.t81_hip_transpose_packed.restype = _i
    lib.t81_hip_transpose_packed.argtypes = [_vp, _vp, _i64, _i64, _vp]
    lib.t81_hip_tq_block_bytes.restype = _i
    lib.t81_hip_tq_block_bytes.argtypes = [_i]
    lib.t81_hip_tq_quantize.restype = _i
    lib.t81_hip_tq_quantize.argtypes = [_vp, _vp, _i64, _i64, _f, _i, _vp]
    lib.t81_hip_tq_dequantize.restype = _i
    lib.t81_hip_tq_dequantize.argtypes = [_vp, _vp, _i64, _i64, _i, _vp]
    lib.t81_hip_tq2_matmul.restype = _i
    lib.t81_hip_tq2_matmul.argtypes = [_vp, _i, _vp, _vp, _i64, _i64, _i64, _f, _f, _vp, _vp]
    lib.t81_hip_tq1_quantize_rows.restype = _i
    lib.t81_hip_tq1_quantize_rows.argtypes = [_vp, _i64, _i64, _f, _vp, _vp, _vp, _vp]
    lib.t81_hip_tq1_dequantize_rows.restype = _i
    lib.t81_hip_tq1_dequantize_rows.argtypes = [_vp, _i64, _i64, _vp, _vp, _vp]
    lib.t81_hip_tq1_payload_bytes.restype = _i64
    lib.t81_hip_tq1_payload_bytes.argtypes = [_i64, _i64, _i64, _i]
    lib.t81_hip_tq1_quantize_payload.restype = _i
    lib.t81_hip_tq1_quantize_payload.argtypes = [_vp, _i64, _i64, _i64, _i, _f, _vp, _vp]
    lib.t81_hip_tq1_dequantize_payload.restype = _i
    lib.t81_hip_tq1_dequantize_payload.argtypes = [_vp, _i64, _i64, _i64, _i64, _i, _vp, _vp]
    lib.t81_hip_spmm_plan_create.restype = _i
    lib.t81_hip_spmm_plan_create.argtypes = [_vp, _vp, _vp, _i64, _i, _i,
                                             ctypes.POINTER(ctypes.c_void_p),
                                             ctypes.POINTER(ctypes.c_int64), _vp]
    lib.t81_hip_spmm_plan_apply.restype = _i
    lib.t81_hip_spmm_plan_apply.argtypes = [_vp, _vp, _vp, _i, _f, _f, _vp]
    lib.t81_hip_spmm_plan_info.restype = _i
    lib.t81_hip_spmm_plan_info.argtypes = [_vp, ctypes.POINTER(ctypes.c_int),
                                           ctypes.POINTER(ctypes.c_int),
                                           ctypes.POINTER(ctypes.c_int64)]
    lib.t81_hip_spmm_plan_destroy.restype = None
    lib.t81_hip_spmm_plan_destroy.argtypes = [_vp]
    lib.t81_hip_spmm_simple.restype = _i
    lib.t81_hip_spmm_simple.argtypes = [_vp, _vp, _vp, _i64, _i, _i, _vp, _vp, _i, _f, _f, _vp]
    lib.t81_hip_limb_tryte_table.restype = None
    lib.t81_hip_limb_tryte_table.argtypes = [_vp]


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise ImportError(
                        f"{LIB_PATH} is missing: build it with `python -m t81lib_amd.build` "
                        "(there is no CPU fallback)")
                loaded = ctypes.CDLL(LIB_PATH)
                _declare(loaded)
                _lib = loaded
    return _lib


def last_error() -> str:
    msg = lib().t81_hip_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> None:
    """Raises the reference's exception type for a non-zero ABI return code."""
    if rc == OK:
        return
    msg = last_error() or f"libt81_hip error {rc}"
    if rc in (EINVAL_SHAPE, EINVAL_K48, EINVAL_THRESHOLD, EINVAL_DTYPE, EINVAL_POINTER,
              EINVAL_INDEX):
        raise ValueError(msg)
    raise T81HipError(msg)


def available() -> bool:
    """True when the library loads and the current device is a gfx950."""
    try:
        return bool(lib().t81_hip_available())
    except OSError:
        return False

"""CPU checks of libt81_hip.so: it loads, exports every declared symbol, and rejects bad
arguments with the reference's error text before touching a device."""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

from t81lib_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "t81_hip.h")


def declared_symbols() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(t81_hip_\w+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_symbols()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.EXPORTS)


def test_limb_table_bit_exact_with_reference(golden):
    """K4's constant-evaluated tryte table equals build_tryte_contributions as compiled
    from the reference (include/t81/linalg/gemm.hpp:28-41)."""
    buf = (ctypes.c_double * 432)()
    _lib.lib().t81_hip_limb_tryte_table(ctypes.cast(buf, ctypes.c_void_p))
    got = np.frombuffer(buf, dtype=np.float64).reshape(16, 27)
    np.testing.assert_array_equal(got.view(np.uint64), golden["table"].view(np.uint64))


def _call(rc):
    return rc, _lib.last_error()


def test_validation_codes_and_messages():
    lib = _lib.lib()
    rc, msg = _call(lib.t81_hip_quantize_pack(None, _lib.DTYPE_F32, None, 4, 4, 0.0,
                                              _lib.THR_CPP, None))
    assert rc == _lib.EINVAL_THRESHOLD and msg == "threshold must be between 0 (exclusive) and 1"
    rc, msg = _call(lib.t81_hip_quantize_pack(None, _lib.DTYPE_F32, None, 4, 4, 1.5,
                                              _lib.THR_CPP, None))
    assert rc == _lib.EINVAL_THRESHOLD
    rc, msg = _call(lib.t81_hip_quantize_pack(None, _lib.DTYPE_F32, None, -1, 4, 0.5,
                                              _lib.THR_CPP, None))
    assert rc == _lib.EINVAL_SHAPE
    rc, msg = _call(lib.t81_hip_quantize_pack(None, _lib.DTYPE_F32, None, 4, 4, 0.5,
                                              _lib.THR_CPP, None))
    assert rc == _lib.EINVAL_POINTER
    rc, msg = _call(lib.t81_hip_gemm_ternary_limb(None, None, None, 2, 3, 47, 1.0, 0.0, None))
    assert rc == _lib.EINVAL_K48 and msg == "gemm_ternary requires K divisible by 48"
    rc, msg = _call(lib.t81_hip_gemm_ternary_limb(None, None, None, -2, 3, 48, 1.0, 0.0, None))
    assert rc == _lib.EINVAL_SHAPE and msg == "gemm_ternary dimensions must be non-negative"
    # M == 0 is a no-op before any device check (gemm_gpu.hpp:188-190)
    assert lib.t81_hip_gemm_ternary_limb(None, None, None, 0, 3, 48, 1.0, 0.0, None) == 0
    rc, msg = _call(lib.t81_hip_ternary_matmul(None, _lib.DTYPE_I8, None, None, 1, 1, 48, 2.0,
                                               0.0, None, None))
    assert rc == _lib.EINVAL_DTYPE
    rc, msg = _call(lib.t81_hip_ternary_matmul(None, 9, None, None, 1, 1, 48, 1.0, 0.0, None,
                                               None))
    assert rc == _lib.EINVAL_DTYPE
    rc, msg = _call(lib.t81_hip_ternary_matmul_kernel(2, None, _lib.DTYPE_BF16, None, None, 17,
                                                      1, 48, 1.0, 0.0, None, None))
    assert rc == _lib.EINVAL_POINTER or rc == _lib.EINVAL_SHAPE
    rc, msg = _call(lib.t81_hip_unpack(None, None, 2, 1, 49, None))
    assert rc == _lib.EINVAL_SHAPE and msg == "cols exceeds packed trit capacity"


def test_python_check_maps_exception_types():
    with pytest.raises(ValueError, match="K divisible by 48"):
        _lib.check(_lib.lib().t81_hip_gemm_ternary_limb(None, None, None, 1, 1, 5, 1.0, 0.0, None))
    with pytest.raises(_lib.T81HipError):
        _lib.check(_lib.EHIP)

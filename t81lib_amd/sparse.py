"""Sparse ternary x dense products on the GPU (the reference's t81::sparse, simple.hpp).

``SparseTernaryMatrix`` holds a COO matrix -- (row, col, integer value) entries in a
significant list order -- in its device form (entries stably sorted by row), built once
and applied to any number of dense right-hand sides:

    A = SparseTernaryMatrix(values, row_indices, col_indices, rows, cols)
    C = A.matmul(B)                       # (rows, N) float32, B (cols, N) on the GPU
    A.matmul(B2, C, alpha=0.5, beta=1.0)  # C = 0.5 * A B2 + C, in place

Results are bit-identical to t81::sparse::spmm_simple (include/t81/sparse/simple.hpp:37-94):
every entry's contribution is rounded into C in list order, in double.
"""

from __future__ import annotations

import ctypes
from typing import Any, Optional

import numpy as np
import torch

from . import _lib

INT32_MIN, INT32_MAX = -2**31, 2**31 - 1


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def entry_arrays(values: Any, row_indices: Any, col_indices: Any,
                 device: torch.device) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Device int64 values and int32 indices, converted like the binding's arguments
    (std::vector<long long> / std::vector<int32_t>, python/bindings.cpp:890-892):
    non-integers and integers out of range raise TypeError; lengths must match."""
    out = []
    for obj, lo, hi, dt in ((values, -2**63, 2**63 - 1, torch.int64),
                            (row_indices, INT32_MIN, INT32_MAX, torch.int32),
                            (col_indices, INT32_MIN, INT32_MAX, torch.int32)):
        if isinstance(obj, torch.Tensor):
            if obj.dtype.is_floating_point or obj.dtype.is_complex or obj.dtype == torch.bool:
                raise TypeError("spmm_simple: entries must be integers")
            t = obj.reshape(-1)
            if t.numel() and dt == torch.int32 and t.dtype == torch.int64:
                if int(t.min()) < lo or int(t.max()) > hi:
                    raise TypeError("spmm_simple: index out of the int32 range")
            out.append(t.to(device=device, dtype=dt).contiguous())
            continue
        seq = list(obj) if not isinstance(obj, np.ndarray) else obj.reshape(-1)
        if isinstance(seq, np.ndarray):
            if seq.dtype.kind not in "iu":
                raise TypeError("spmm_simple: entries must be integers")
            if seq.size and (int(seq.min()) < lo or int(seq.max()) > hi):
                raise TypeError("spmm_simple: integer out of range")
            arr = seq.astype(np.int64 if dt == torch.int64 else np.int32)
        else:
            for x in seq:
                if isinstance(x, (bool, float)) or not hasattr(x, "__index__"):
                    raise TypeError("spmm_simple: entries must be integers")
            ints = [int(x.__index__()) for x in seq]
            if any(x < lo or x > hi for x in ints):
                raise TypeError("spmm_simple: integer out of range")
            arr = np.array(ints, dtype=np.int64 if dt == torch.int64 else np.int32)
        out.append(torch.from_numpy(arr).to(device))
    v, r, c = out
    if not (v.numel() == r.numel() == c.numel()):
        raise ValueError("Values and indices lengths must match")  # bindings.cpp:900-902
    return v, r, c


class SparseTernaryMatrix:
    """Device form of a COO ternary matrix (``SimpleSparseTernary``, simple.hpp:15-21)."""

    def __init__(self, values: Any, row_indices: Any, col_indices: Any, rows: int, cols: int):
        if rows < 0 or cols < 0:
            raise ValueError("Matrix dimensions must be non-negative")
        if not torch.cuda.is_available():
            raise _lib.T81HipError("t81lib_amd needs a gfx950 GPU; none is visible")
        self.device = torch.device("cuda", torch.cuda.current_device())
        v, r, c = entry_arrays(values, row_indices, col_indices, self.device)
        self.rows, self.cols = int(rows), int(cols)
        self._plan = ctypes.c_void_p()
        bad = ctypes.c_int64(-1)
        L = _lib.lib()
        rc = L.t81_hip_spmm_plan_create(v.data_ptr(), r.data_ptr(), c.data_ptr(), v.numel(),
                                        self.rows, self.cols, ctypes.byref(self._plan),
                                        ctypes.byref(bad), _stream())
        if rc != _lib.OK:
            msg = _lib.last_error()
            self.close()
            if rc == _lib.EINVAL_INDEX:
                raise ValueError(msg)  # simple.hpp:79-84
            _lib.check(rc)
        nnz = ctypes.c_int64()
        L.t81_hip_spmm_plan_info(self._plan, None, None, ctypes.byref(nnz))
        self.nnz = int(nnz.value)

    def matmul(self, B: torch.Tensor, C: Optional[torch.Tensor] = None, alpha: float = 1.0,
               beta: float = 0.0) -> torch.Tensor:
        """C = alpha * A B + beta * C with B (cols, N) float32 on the GPU; C (rows, N)
        float32 is written in place (a new one when omitted, which needs beta == 0)."""
        if self._plan is None or not self._plan.value:
            raise ValueError("matrix is closed")
        if B.ndim != 2 or B.shape[0] != self.cols or B.dtype != torch.float32 or not B.is_cuda:
            raise ValueError("B must be a (cols, N) float32 GPU tensor")
        B = B.contiguous()
        N = B.shape[1]
        if C is None:
            if beta != 0.0:
                raise ValueError("beta != 0 needs an input C")
            C = torch.empty((self.rows, N), dtype=torch.float32, device=B.device)
        elif (tuple(C.shape) != (self.rows, N) or C.dtype != torch.float32
              or not C.is_contiguous() or not C.is_cuda):
            raise ValueError("C must be a contiguous (rows, N) float32 GPU tensor")
        _lib.check(_lib.lib().t81_hip_spmm_plan_apply(self._plan, B.data_ptr(), C.data_ptr(), N,
                                                      alpha, beta, _stream()))
        return C

    def close(self) -> None:
        plan = getattr(self, "_plan", None)
        if plan is not None and plan.value:
            torch.cuda.current_stream().synchronize()
            _lib.lib().t81_hip_spmm_plan_destroy(plan)
        self._plan = None

    def __del__(self):  # pragma: no cover - interpreter shutdown order varies
        try:
            self.close()
        except Exception:
            pass

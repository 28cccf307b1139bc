"""The reference's ``t81lib`` extension-module surface for the packed path, on the GPU.

Same names, argument meanings, defaults and exception types as the pybind11
module (python/bindings.cpp:759-767 constants, :769-810 ``gemm_ternary``,
:405-517 quantize/pack, :519-638 and :961-995 the TQ1_0 row codec, :640-686 unpack,
:888-940 ``spmm_simple``).  Arguments may be NumPy arrays /
buffers (copied to the GPU, results copied back -- the host-span contract of
``rocm_gemm_ternary``, src/linalg/gemm_rocm.cpp:335-396) or GPU torch tensors
(used in place, no copies).  Every computation runs on the GPU; there is no
CPU path.
"""

from __future__ import annotations

from typing import Any

import numpy as np
import torch

from . import _lib, ops

TRITS_PER_LIMB = 48
TRYTES_PER_LIMB = 16
BYTES_PER_LIMB = 16
HAS_CUDA_BACKEND = False
HAS_METAL_BACKEND = False
TQ1_TRITS_PER_BLOCK = 8   # src/t81/core/gguf_quants.h:14
TQ1_BLOCK_ROWS = 32       # src/t81/core/gguf_quants.h:15


def _has_rocm() -> bool:
    return _lib.available()


def __getattr__(name: str) -> Any:
    if name == "HAS_ROCM_BACKEND":  # evaluated lazily: probing the device initialises HIP
        return _has_rocm()
    raise AttributeError(name)


def _device() -> torch.device:
    if not torch.cuda.is_available():
        raise _lib.T81HipError("t81lib_amd needs a gfx950 GPU; none is visible")
    return torch.device("cuda", torch.cuda.current_device())


def _as_device(obj: Any, dtype: torch.dtype) -> tuple[torch.Tensor, bool]:
    """(tensor on the GPU, was_host)."""
    if isinstance(obj, torch.Tensor):
        if obj.device.type == "cuda":
            return obj, False
        return obj.to(device=_device()), True
    arr = np.asarray(obj)
    return torch.from_numpy(np.ascontiguousarray(arr)).to(device=_device()), True


def _packed_bytes(obj: Any) -> tuple[torch.Tensor, bool]:
    """Packed limbs from a uint8 array/tensor, a V16 array, or any byte buffer."""
    if isinstance(obj, torch.Tensor):
        if obj.dtype != torch.uint8:
            raise ValueError("packed limbs must be uint8")
        t, host = _as_device(obj, torch.uint8)
        return t.contiguous().reshape(-1), host
    arr = np.asarray(memoryview(obj) if not isinstance(obj, np.ndarray) else obj)
    arr = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
    return torch.from_numpy(arr).to(device=_device()), True


def gemm_ternary(A: Any, B: Any, C: Any, M: int, N: int, K: int, alpha: float = 1.0,
                 beta: float = 0.0) -> None:
    """Packed-limb GEMM, reference semantics (limb-integer products, fp64 sums).

    C (M x N float32) is read and overwritten in place, like the reference.
    """
    if M < 0 or N < 0 or K < 0:
        raise ValueError("gemm_ternary dimensions must be non-negative")
    if K % TRITS_PER_LIMB != 0:
        raise ValueError("K must be divisible by the limb trit count")
    kl = K // TRITS_PER_LIMB
    a, _ = _packed_bytes(A)
    b, _ = _packed_bytes(B)
    if a.numel() != M * kl * BYTES_PER_LIMB:
        raise ValueError("A span size does not match (M, K / 48)")
    if b.numel() != kl * N * BYTES_PER_LIMB:
        raise ValueError("B span size does not match (K / 48, N)")
    if isinstance(C, torch.Tensor) and C.device.type == "cuda":
        if C.dtype != torch.float32 or tuple(C.shape) != (M, N) or not C.is_contiguous():
            raise ValueError("C tensor shape must match (M, N)")
        ops.gemm_limb(a, b, C, M, N, K, alpha, beta)
        return
    if isinstance(C, torch.Tensor):
        host = C
        if host.dtype != torch.float32 or host.numel() != M * N:
            raise ValueError("C tensor shape must match (M, N)")
        c = host.to(device=_device()).contiguous().reshape(M, N)
        ops.gemm_limb(a, b, c, M, N, K, alpha, beta)
        host.copy_(c.reshape(host.shape).cpu())
        return
    view = np.asarray(C if isinstance(C, np.ndarray) else memoryview(C)).reshape(-1)
    if view.dtype != np.float32 or view.size != M * N:
        raise ValueError("C tensor shape must match (M, N)")
    c = torch.from_numpy(np.ascontiguousarray(view).copy()).to(device=_device()).reshape(M, N)
    ops.gemm_limb(a, b, c, M, N, K, alpha, beta)
    view[...] = c.cpu().numpy().reshape(-1)


def _threshold_cpp(threshold: float) -> float:
    if threshold <= 0.0 or threshold > 1.0:
        raise ValueError("threshold must be between 0 (exclusive) and 1")
    return float(threshold)


def _return_like(result: torch.Tensor, was_host: bool):
    return result.cpu().numpy() if was_host else result


def quantize_to_trits(values: Any, threshold: float = 0.5):
    """Float array -> int8 trits in {-1, 0, 1} (python/bindings.cpp:416-445)."""
    thr = _threshold_cpp(threshold)
    t, host = _as_device(values, torch.float32)
    if t.ndim == 0:
        raise ValueError("expected at least one dimension for quantization")
    return _return_like(ops.quantize(t, thr, _lib.THR_CPP), host)


def dequantize_trits(trits: Any):
    """Trit tensor -> float32 (python/bindings.cpp:447-458)."""
    t, host = _as_device(trits, torch.int8)
    return _return_like(t.to(torch.int8).to(torch.float32), host)


def pack_dense_matrix(matrix: Any, threshold: float = 0.5):
    """2-D float array -> (rows, limbs, 16) uint8 packed limbs (python/bindings.cpp:460-517)."""
    thr = _threshold_cpp(threshold)
    t, host = _as_device(matrix, torch.float32)
    if t.ndim != 2:
        raise ValueError("pack_dense_matrix expects a 2D array")
    return _return_like(ops.quantize_pack(t, thr, _lib.THR_CPP), host)


def unpack_packed_limbs(packed: Any, rows: int, cols: int):
    """(rows, limbs, 16) uint8 -> (rows, cols) int8 trits (python/bindings.cpp:640-686)."""
    if rows < 0 or cols < 0:
        raise ValueError("rows and cols must be non-negative")
    t, host = _as_device(packed, torch.uint8)
    if t.ndim != 3:
        raise ValueError("packed limbs must be a 3D array")
    if t.shape[0] != rows:
        raise ValueError("row count mismatch")
    if t.shape[2] != BYTES_PER_LIMB:
        raise ValueError("packed limb innermost dimension must equal limb byte width")
    if cols > t.shape[1] * TRITS_PER_LIMB:
        raise ValueError("cols exceeds packed trit capacity")
    if ops.count_invalid_bytes(t):
        raise ValueError("limb bytes must encode canonical trytes")
    return _return_like(ops.unpack(t, rows, cols), host)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _tq1_words(cols: int) -> int:
    return (int(cols) + TQ1_TRITS_PER_BLOCK - 1) // TQ1_TRITS_PER_BLOCK


def _forcecast(obj: Any, np_dtype, t_dtype: torch.dtype) -> tuple[torch.Tensor, bool]:
    """The array as a contiguous GPU tensor of the given type, converted the way pybind11's
    forcecast converts (numpy's unsafe cast); (tensor, was_host)."""
    if isinstance(obj, torch.Tensor) and obj.device.type == "cuda":
        if obj.dtype != t_dtype:
            if t_dtype == torch.uint16:
                obj = (obj.to(torch.int64) & 0xFFFF).to(torch.int32).to(torch.uint16)
            else:
                obj = obj.to(t_dtype)
        return obj.contiguous(), False
    arr = obj.numpy() if isinstance(obj, torch.Tensor) else np.asarray(obj)
    arr = np.ascontiguousarray(arr.astype(np_dtype, copy=False))
    return torch.from_numpy(arr).to(device=_device()), True


def quantize_row_tq1_0(row: Any, threshold: float = 0.45, scale: float = 0.0):
    """One row of floats -> (scale, uint16 TQ1_0 words) (python/bindings.cpp:519-540 over
    quantize_row_tq1_0, src/t81/core/gguf_quants.h:116-144).  The returned scale is the
    argument when it is not <= 0 (a NaN argument is returned as given, while the words use
    the row's max |v|, as the binding does), else the row's max |v|."""
    t, host = _forcecast(row, np.float32, torch.float32)
    if t.ndim != 1:
        raise ValueError("quantize_row_tq1_0 requires a 1-D float array")
    n = t.numel()
    scale32 = float(np.float32(scale))
    threshold32 = float(np.float32(threshold))
    words = torch.empty(_tq1_words(n), dtype=torch.uint16, device=t.device)
    if n == 0:
        actual = 0.0 if scale32 <= 0.0 else scale32
        return actual, _return_like(words, host)
    s_in = torch.tensor([scale32], dtype=torch.float32, device=t.device)
    s_out = torch.empty(1, dtype=torch.float32, device=t.device)
    _lib.check(_lib.lib().t81_hip_tq1_quantize_rows(t.data_ptr(), 1, n, threshold32,
                                                     s_in.data_ptr(), s_out.data_ptr(),
                                                     words.data_ptr(), _stream()))
    actual = float(s_out.item()) if scale32 <= 0.0 else scale32
    return actual, _return_like(words, host)


def dequant_row_tq1_0(blocks: Any, cols: int, scale: float):
    """TQ1_0 words -> cols float32 values (python/bindings.cpp:542-559 over
    dequantize_row_tq1_0, src/t81/core/gguf_quants.h:146-168)."""
    if cols < 0:
        raise ValueError("cols must be non-negative")
    t, host = _forcecast(blocks, np.uint16, torch.uint16)
    need = _tq1_words(cols)
    if t.numel() < need:
        raise ValueError("packed buffer too small for the requested column count")
    out = torch.empty(int(cols), dtype=torch.float32, device=t.device)
    if cols > 0:
        s = torch.tensor([float(np.float32(scale))], dtype=torch.float32, device=t.device)
        _lib.check(_lib.lib().t81_hip_tq1_dequantize_rows(t.reshape(-1).data_ptr(), 1, cols,
                                                          s.data_ptr(), out.data_ptr(),
                                                          _stream()))
    return _return_like(out, host)


def _payload_bytes(buffer: Any) -> tuple[torch.Tensor, bool]:
    if isinstance(buffer, torch.Tensor):
        if buffer.element_size() != 1:
            raise ValueError("buffer must be observed as bytes")
        t, host = _as_device(buffer, buffer.dtype)
        return t.contiguous().reshape(-1).view(torch.uint8), host
    view = memoryview(buffer)
    if view.itemsize != 1:
        raise ValueError("buffer must be observed as bytes")
    arr = np.frombuffer(view.tobytes(), np.uint8)
    return torch.from_numpy(arr.copy()).to(device=_device()), True


def _dequant_tensor(buffer: Any, rows: int, cols: int, block_rows: int, refinements: bool):
    if rows < 0 or cols < 0:
        raise ValueError("rows and cols must be non-negative")
    data, host = _payload_bytes(buffer)
    out = torch.empty((int(rows), int(cols)), dtype=torch.float32, device=data.device)
    _lib.check(_lib.lib().t81_hip_tq1_dequantize_payload(
        data.data_ptr() if data.numel() else None, data.numel(), rows, cols, block_rows,
        int(refinements), out.data_ptr() if out.numel() else None, _stream()))
    return _return_like(out, host)


def dequant_tq1_0(buffer: Any, rows: int, cols: int, block_rows: int = TQ1_BLOCK_ROWS):
    """A whole TQ1_0 row-codec tensor payload -> (rows, cols) float32: per group of
    block_rows rows a float16 scale, then the rows' words (python/bindings.cpp:561-638,
    975-984)."""
    return _dequant_tensor(buffer, rows, cols, block_rows, False)


def dequant_tq2_0(buffer: Any, rows: int, cols: int, block_rows: int = TQ1_BLOCK_ROWS):
    """As dequant_tq1_0 with 8 reserved refinement bytes after each group's scale, skipped
    (python/bindings.cpp:986-995)."""
    return _dequant_tensor(buffer, rows, cols, block_rows, True)


def _float_span(obj: Any, count: int) -> tuple[torch.Tensor, Any]:
    """(GPU float32 tensor, host array to write back or None), with the buffer checks and
    messages of make_float_span (python/bindings.cpp:112-134), which the binding applies
    to B as well as C."""
    if isinstance(obj, torch.Tensor):
        if obj.device.type == "cuda":
            if obj.element_size() != 4:
                raise ValueError("C buffer must store float32 values")
            if not obj.is_contiguous():
                raise ValueError("C buffer must use C-style contiguous memory")
            if obj.numel() != count:
                raise ValueError("C buffer byte size mismatch")
            return obj.reshape(-1).view(torch.float32), None
        obj = obj.numpy()  # a host tensor: its own memory
    view = memoryview(obj)
    if view.readonly:
        raise ValueError("C buffer must be writable")
    if view.itemsize != 4:
        raise ValueError("C buffer must store float32 values")
    if not view.c_contiguous:
        raise ValueError("C buffer must use C-style contiguous memory")
    if view.nbytes != count * 4:
        raise ValueError("C buffer byte size mismatch")
    host = np.asarray(view).reshape(-1).view(np.float32)
    return torch.from_numpy(host.copy()).to(device=_device()), host


def spmm_simple(values: Any, row_indices: Any, col_indices: Any, rows: int, cols: int, B: Any,
                C: Any, N: int, alpha: float = 1.0, beta: float = 0.0) -> None:
    """COO sparse x dense multiply over ternary weights (python/bindings.cpp:888-940):
    C (rows x N) = alpha * A B + beta * C in place, B cols x N, entries applied in list
    order, bit-identical to t81::sparse::spmm_simple (include/t81/sparse/simple.hpp:37-94).
    An out-of-range index raises ValueError after updating C as the reference does
    (beta applied, the entries before it added)."""
    from .sparse import entry_arrays

    dev = _device()
    v, r, c = entry_arrays(values, row_indices, col_indices, dev)
    if rows < 0 or cols < 0:
        raise ValueError("Matrix dimensions must be non-negative")
    if N < 0:
        raise ValueError("Feature dimension N must be non-negative")
    b, _ = _float_span(B, cols * N)
    out, host = _float_span(C, rows * N)
    L = _lib.lib()
    rc = L.t81_hip_spmm_simple(v.data_ptr(), r.data_ptr(), c.data_ptr(), v.numel(), rows, cols,
                               b.data_ptr(), out.data_ptr(), N, alpha, beta,
                               torch.cuda.current_stream().cuda_stream)
    msg = _lib.last_error() if rc != _lib.OK else ""
    if host is not None and rc in (_lib.OK, _lib.EINVAL_INDEX):
        host[...] = out.cpu().numpy()
    if rc == _lib.EINVAL_INDEX:
        raise ValueError(msg)
    if rc != _lib.OK:
        _lib.check(rc)


__all__ = [
    "TRITS_PER_LIMB", "TRYTES_PER_LIMB", "BYTES_PER_LIMB", "HAS_CUDA_BACKEND",
    "HAS_METAL_BACKEND", "gemm_ternary", "quantize_to_trits", "dequantize_trits",
    "pack_dense_matrix", "unpack_packed_limbs", "spmm_simple", "TQ1_TRITS_PER_BLOCK",
    "TQ1_BLOCK_ROWS", "quantize_row_tq1_0", "dequant_row_tq1_0", "dequant_tq1_0",
    "dequant_tq2_0",
]

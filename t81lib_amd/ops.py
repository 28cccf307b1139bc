"""Device-tensor operations over libt81_hip.so (torch tensors in, torch tensors out).

All work is enqueued on ``torch.cuda.current_stream()``; inputs must already be
on the GPU (the wrappers in :mod:`t81lib_amd.t81lib` and
:mod:`t81lib_amd.tensor` move host data first).  Packed weights use the
reference's limb layout: ``(rows, L, 16)`` uint8, ``L = ceil(cols / 48)``.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib

TRITS_PER_LIMB = 48
TRYTES_PER_LIMB = 16
BYTES_PER_LIMB = 16

_FLOAT_CODES = {
    torch.float32: _lib.DTYPE_F32,
    torch.bfloat16: _lib.DTYPE_BF16,
    torch.float16: _lib.DTYPE_F16,
}
_MATMUL_CODES = {
    torch.float32: _lib.DTYPE_F32,
    torch.bfloat16: _lib.DTYPE_BF16,
    torch.int8: _lib.DTYPE_I8,
}


def limbs_for(cols: int) -> int:
    return (cols + TRITS_PER_LIMB - 1) // TRITS_PER_LIMB


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _require_cuda(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor")


def torch_threshold(threshold: float) -> float:
    """t81/torch/__init__.py:45: float(max(0.0, min(threshold, 0.9999)))."""
    return float(max(0.0, min(threshold, 0.9999)))


def quantize_pack(weight: torch.Tensor, threshold: float, thr_mode: int = _lib.THR_CPP,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """K1: (rows, cols) float -> (rows, L, 16) uint8 packed trits (bit-exact packer)."""
    _require_cuda(weight, "weight")
    if weight.ndim != 2:
        raise ValueError("pack_dense_matrix expects a 2D array")
    if weight.dtype not in _FLOAT_CODES:
        weight = weight.float()
    weight = weight.contiguous()
    rows, cols = weight.shape
    shape = (rows, limbs_for(cols), BYTES_PER_LIMB)
    if out is None:
        out = torch.empty(shape, dtype=torch.uint8, device=weight.device)
    elif tuple(out.shape) != shape or out.dtype != torch.uint8 or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous uint8 tensor of shape {shape}")
    _lib.check(_lib.lib().t81_hip_quantize_pack(weight.data_ptr(), _FLOAT_CODES[weight.dtype],
                                                out.data_ptr(), rows, cols, threshold, thr_mode,
                                                _stream()))
    return out


def quantize(values: torch.Tensor, threshold: float, thr_mode: int = _lib.THR_CPP) -> torch.Tensor:
    """Elementwise trits (int8) of a float tensor of any shape."""
    _require_cuda(values, "values")
    if values.dtype not in _FLOAT_CODES:
        values = values.float()
    values = values.contiguous()
    out = torch.empty(values.shape, dtype=torch.int8, device=values.device)
    _lib.check(_lib.lib().t81_hip_quantize(values.data_ptr(), _FLOAT_CODES[values.dtype],
                                           out.data_ptr(), values.numel(), threshold, thr_mode,
                                           _stream()))
    return out


def pack_cols(x: torch.Tensor, threshold: float = 0.5,
              thr_mode: int = _lib.THR_TORCH) -> torch.Tensor:
    """(tokens, K) float -> (L, tokens, 16) uint8: the column-wise packing of x^T."""
    _require_cuda(x, "x")
    if x.ndim != 2:
        raise ValueError("pack_cols expects a 2D tensor")
    if x.dtype not in _FLOAT_CODES:
        x = x.float()
    x = x.contiguous()
    tokens, k = x.shape
    out = torch.empty((limbs_for(k), tokens, BYTES_PER_LIMB), dtype=torch.uint8, device=x.device)
    _lib.check(_lib.lib().t81_hip_pack_cols(x.data_ptr(), _FLOAT_CODES[x.dtype], out.data_ptr(),
                                            tokens, k, threshold, thr_mode, _stream()))
    return out


def unpack(packed: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """(rows, L, 16) uint8 -> (rows, cols) int8 trits."""
    _require_cuda(packed, "packed")
    if packed.ndim != 3:
        raise ValueError("packed limbs must be a 3D array")
    if packed.shape[0] != rows:
        raise ValueError("row count mismatch")
    if packed.shape[2] != BYTES_PER_LIMB:
        raise ValueError("packed limb innermost dimension must equal limb byte width")
    packed = packed.contiguous()
    out = torch.empty((rows, cols), dtype=torch.int8, device=packed.device)
    _lib.check(_lib.lib().t81_hip_unpack(packed.data_ptr(), out.data_ptr(), rows,
                                         packed.shape[1], cols, _stream()))
    return out


def matmul_input_reference(w_packed: torch.Tensor, x: torch.Tensor, threshold: float = 0.5,
                           alpha: float = 1.0, beta: float = 0.0,
                           c: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The reference's literal matmul_input product in one kernel: x (tokens, K) quantized
    (torch form, threshold clamped as t81/torch/__init__.py:45) and packed column-wise
    inside the limb GEMM; returns C (rows, tokens) float32, bit-identical to
    pack_cols + gemm_limb."""
    _require_cuda(w_packed, "w_packed")
    _require_cuda(x, "x")
    if x.ndim != 2:
        raise ValueError("t81.trit linear helpers expect 2D activations")
    if x.dtype not in _FLOAT_CODES:
        x = x.float()
    x = x.contiguous()
    tokens, k = x.shape
    if w_packed.ndim != 3 or w_packed.shape[1] != limbs_for(k) or w_packed.dtype != torch.uint8:
        raise ValueError("packed weight limbs do not match K")
    w_packed = w_packed.contiguous()
    rows = w_packed.shape[0]
    if c is None:
        c = torch.zeros((rows, tokens), dtype=torch.float32, device=x.device)
    elif tuple(c.shape) != (rows, tokens) or c.dtype != torch.float32 or not c.is_contiguous():
        raise ValueError("C tensor shape must match (rows, tokens)")
    _lib.check(_lib.lib().t81_hip_matmul_input_reference(
        w_packed.data_ptr(), x.data_ptr(), _FLOAT_CODES[x.dtype], c.data_ptr(), rows, tokens, k,
        torch_threshold(threshold), alpha, beta, _stream()))
    return c


def transpose_packed(packed: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """(rows, L, 16) limbs of T -> (cols, ceil(rows / 48), 16) limbs of T^T."""
    _require_cuda(packed, "packed")
    if packed.dtype != torch.uint8 or packed.ndim != 3 or packed.shape[2] != BYTES_PER_LIMB:
        raise ValueError("packed weights must be a (N, L, 16) uint8 tensor")
    if packed.shape[0] != rows or packed.shape[1] != limbs_for(cols):
        raise ValueError("packed shape does not match rows / cols")
    packed = packed.contiguous()
    out = torch.empty((cols, limbs_for(rows), BYTES_PER_LIMB), dtype=torch.uint8,
                      device=packed.device)
    _lib.check(_lib.lib().t81_hip_transpose_packed(packed.data_ptr(), out.data_ptr(), rows, cols,
                                                   _stream()))
    return out


def count_invalid_bytes(packed: torch.Tensor) -> int:
    """Number of bytes > 26 (non-canonical trytes); synchronises the stream."""
    _require_cuda(packed, "packed")
    packed = packed.contiguous()
    bad = torch.empty(1, dtype=torch.int32, device=packed.device)
    _lib.check(_lib.lib().t81_hip_validate_packed(packed.data_ptr(), packed.numel(),
                                                  bad.data_ptr(), _stream()))
    return int(bad.item())


def ternary_matmul(x: torch.Tensor, w_packed: torch.Tensor, k: Optional[int] = None,
                   alpha: float = 1.0, beta: float = 0.0, c: Optional[torch.Tensor] = None,
                   bias: Optional[torch.Tensor] = None, kernel: Optional[int] = None
                   ) -> torch.Tensor:
    """K2/K3: C = alpha * X @ T^T + beta * C + bias over packed weights.

    x: (M, K) float32 / bfloat16 / int8 on the GPU; w_packed: (N, L, 16) uint8.
    Returns C (M, N): float32, or int32 (exact) for int8 activations.  When ``c``
    is given it is updated in place and returned.  ``kernel`` forces 2 (GEMV)
    or 3 (GEMM); by default M <= 16 runs the GEMV kernel.
    """
    _require_cuda(x, "x")
    _require_cuda(w_packed, "w_packed")
    if x.ndim != 2:
        raise ValueError("t81.trit linear helpers expect 2D activations")
    if x.dtype not in _MATMUL_CODES:
        x = x.float()
    x = x.contiguous()
    m, kx = x.shape
    k = kx if k is None else int(k)
    if k != kx:
        raise ValueError("rhs dimension does not match ternary weight width")
    if w_packed.ndim != 3 or w_packed.shape[2] != BYTES_PER_LIMB or w_packed.dtype != torch.uint8:
        raise ValueError("packed weights must be a (N, L, 16) uint8 tensor")
    if w_packed.shape[1] != limbs_for(k):
        raise ValueError("packed weight limbs do not match K")
    w_packed = w_packed.contiguous()
    n = w_packed.shape[0]
    out_dtype = torch.int32 if x.dtype == torch.int8 else torch.float32
    if c is None:
        if beta != 0.0:
            raise ValueError("beta != 0 needs an input C")
        c = torch.empty((m, n), dtype=out_dtype, device=x.device)
    else:
        _require_cuda(c, "C")
        if tuple(c.shape) != (m, n) or c.dtype != out_dtype or not c.is_contiguous():
            raise ValueError("C tensor shape must match (M, N)")
    bias_ptr = None
    if bias is not None:
        _require_cuda(bias, "bias")
        if bias.numel() != n:
            raise ValueError("bias must have N elements")
        bias = bias.float().contiguous()
        bias_ptr = bias.data_ptr()
    lib = _lib.lib()
    which = 0 if kernel is None else int(kernel)
    if which not in (0, 2, 3):
        raise ValueError("kernel must be 2 or 3")
    code = _MATMUL_CODES[x.dtype]
    # K3 with few output tiles, and K2 for 5..16 tokens, split K over a workspace from
    # torch's caching allocator (safe under graph capture); its size is 0 for every other
    # shape.
    ws_bytes = int(lib.t81_hip_ternary_matmul_workspace_size(m, n, k, code))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes > 0 else None
    rc = lib.t81_hip_ternary_matmul_ws(which, x.data_ptr(), code, w_packed.data_ptr(),
                                       c.data_ptr(), m, n, k, alpha, beta, bias_ptr,
                                       ws.data_ptr() if ws is not None else None, ws_bytes,
                                       _stream())
    _lib.check(rc)
    return c


def gemm_limb(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, m: int, n: int, k: int,
              alpha: float = 1.0, beta: float = 0.0) -> torch.Tensor:
    """K4: the reference's limb-integer gemm_ternary, C updated in place.

    a: M*K/48 limbs, b: K/48*N limbs (uint8, 16 bytes each), c: (M, N) float32.
    """
    for name, t in (("A", a), ("B", b), ("C", c)):
        _require_cuda(t, name)
    if m < 0 or n < 0 or k < 0:
        raise ValueError("gemm_ternary dimensions must be non-negative")
    if k % TRITS_PER_LIMB != 0:
        raise ValueError("K must be divisible by the limb trit count")
    kl = k // TRITS_PER_LIMB
    if a.dtype != torch.uint8 or a.numel() != m * kl * BYTES_PER_LIMB:
        raise ValueError("A span size does not match (M, K / 48)")
    if b.dtype != torch.uint8 or b.numel() != kl * n * BYTES_PER_LIMB:
        raise ValueError("B span size does not match (K / 48, N)")
    if c.dtype != torch.float32 or c.numel() != m * n or not c.is_contiguous():
        raise ValueError("C tensor shape must match (M, N)")
    a = a.contiguous()
    b = b.contiguous()
    _lib.check(_lib.lib().t81_hip_gemm_ternary_limb(a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n,
                                                    k, alpha, beta, _stream()))
    return c


def limb_tryte_table() -> "list[list[float]]":
    """The 16 x 27 table K4 converts limbs with (host-side, no device needed)."""
    import ctypes

    buf = (ctypes.c_double * (16 * 27))()
    _lib.lib().t81_hip_limb_tryte_table(ctypes.cast(buf, ctypes.c_void_p))
    return [[buf[p * 27 + u] for u in range(27)] for p in range(16)]


__all__ = [
    "quantize_pack", "quantize", "pack_cols", "unpack", "count_invalid_bytes", "ternary_matmul",
    "gemm_limb", "limb_tryte_table", "limbs_for", "torch_threshold",
]


# -- elementwise float32 ops of the backend contract (gemm_gpu.hpp:80-85, 233-249) --------

def _f32_operands(*tensors: torch.Tensor) -> list:
    n = tensors[0].numel()
    out = []
    for i, t in enumerate(tensors):
        _require_cuda(t, f"operand {i}")
        if t.dtype != torch.float32:
            raise ValueError("tensor metadata must describe float32 data")
        if t.numel() != n:
            raise ValueError("input shapes must match")
        out.append(t.contiguous())
    return out


def _f32_out(out: Optional[torch.Tensor], like: torch.Tensor) -> torch.Tensor:
    if out is None:
        return torch.empty_like(like)
    _require_cuda(out, "out")
    if out.dtype != torch.float32 or out.numel() != like.numel() or not out.is_contiguous():
        raise ValueError("out must be a contiguous float32 GPU tensor of the inputs' size")
    return out


def where(condition: torch.Tensor, x: torch.Tensor, y: torch.Tensor,
          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = condition != 0 ? x : y (cpu_where, src/linalg/gemm_dispatch.cpp:145-161)."""
    c, a, b = _f32_operands(condition, x, y)
    out = _f32_out(out, a)
    _lib.check(_lib.lib().t81_hip_where(c.data_ptr(), a.data_ptr(), b.data_ptr(),
                                        out.data_ptr(), a.numel(), _stream()))
    return out


def clamp(x: torch.Tensor, min_value: float, max_value: float,
          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """cpu_clamp, src/linalg/gemm_dispatch.cpp:163-177."""
    (a,) = _f32_operands(x)
    out = _f32_out(out, a)
    _lib.check(_lib.lib().t81_hip_clamp(a.data_ptr(), out.data_ptr(), a.numel(),
                                        float(min_value), float(max_value), _stream()))
    return out


def lerp(start: torch.Tensor, end: torch.Tensor, weight: torch.Tensor,
         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """start + weight * (end - start) (cpu_lerp, src/linalg/gemm_dispatch.cpp:179-194)."""
    s, e, w = _f32_operands(start, end, weight)
    out = _f32_out(out, s)
    _lib.check(_lib.lib().t81_hip_lerp(s.data_ptr(), e.data_ptr(), w.data_ptr(), out.data_ptr(),
                                       s.numel(), _stream()))
    return out


def addcmul(x: torch.Tensor, tensor1: torch.Tensor, tensor2: torch.Tensor, value: float,
            out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x + value * tensor1 * tensor2 (cpu_addcmul, src/linalg/gemm_dispatch.cpp:196-211)."""
    a, t1, t2 = _f32_operands(x, tensor1, tensor2)
    out = _f32_out(out, a)
    _lib.check(_lib.lib().t81_hip_addcmul(a.data_ptr(), t1.data_ptr(), t2.data_ptr(),
                                          float(value), out.data_ptr(), a.numel(), _stream()))
    return out

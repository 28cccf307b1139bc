"""GGUF ternary tensor codecs (TQ1_0, TQ2_0) on the GPU, and matmul straight from TQ2_0.

Mirrors the payload helpers of the reference's ``t81.gguf`` module
(t81/gguf.py:518-690, 1020-1069): the same block formats (llama.cpp's ggml
block_tq1_0 / block_tq2_0, 256 weights per block, ggml types 34 / 35), the same
threshold handling and the same bytes.  File reading and writing (the GGUF header,
metadata and tensor tables) stay with the reference; these functions produce and
consume the tensor payloads those files hold.

    payload = quantize_tensor(weight, "TQ2_0", threshold=0.45)   # uint8 (rows, bytes)
    weight_q = dequantize_tensor(payload, weight.shape, "TQ2_0")  # float32
    y = tq2_matmul(x, payload, k=weight.shape[1])                 # x @ weight_q.T
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import _lib

GGML_TYPE_TQ1_0 = _lib.TQ1_0  # t81/gguf.py:30
GGML_TYPE_TQ2_0 = _lib.TQ2_0  # t81/gguf.py:31
GGUF_QUANT_BLOCK_ROWS = 256   # t81/gguf.py:53
BLOCK_BYTES = {"TQ1_0": 54, "TQ2_0": 66}  # t81/gguf.py:1046-1051

_QUANTS = {"TQ1_0": GGML_TYPE_TQ1_0, "TQ2_0": GGML_TYPE_TQ2_0}


def _quant_code(quant: "str | int") -> int:
    if isinstance(quant, int) and quant in _QUANTS.values():
        return quant
    if isinstance(quant, str) and quant.upper() in _QUANTS:
        return _QUANTS[quant.upper()]
    raise ValueError(f"quant must be one of {sorted(_QUANTS)}")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def row_bytes(cols: int, quant: "str | int") -> int:
    code = _quant_code(quant)
    blocks = (int(cols) + GGUF_QUANT_BLOCK_ROWS - 1) // GGUF_QUANT_BLOCK_ROWS
    return blocks * (54 if code == GGML_TYPE_TQ1_0 else 66)


def quantize_tensor(tensor: torch.Tensor, quant: "str | int" = "TQ2_0",
                    threshold: float = 0.45) -> torch.Tensor:
    """2-D float tensor -> (rows, row_bytes) uint8 payload on the GPU.

    Same bytes as ``_quantize_tensor`` (t81/gguf.py:665-690): each row zero-padded to
    whole blocks, per block d = max |v|, trits of v / d (threshold clipped to [0, 1];
    0 selects round half away from zero), d stored as IEEE half.
    """
    code = _quant_code(quant)
    if tensor.ndim != 2:
        raise ValueError(f"Only 2D tensors supported, got shape {tuple(tensor.shape)}")
    if not tensor.is_cuda:
        tensor = tensor.to("cuda")
    src = tensor.to(torch.float32).contiguous()
    rows, cols = src.shape
    out = torch.empty((rows, row_bytes(cols, code)), dtype=torch.uint8, device=src.device)
    _lib.check(_lib.lib().t81_hip_tq_quantize(src.data_ptr(), out.data_ptr(), rows, cols,
                                              float(threshold), code, _stream()))
    return out


def dequantize_tensor(payload: torch.Tensor, shape: Sequence[int],
                      quant: "str | int" = "TQ2_0") -> torch.Tensor:
    """(rows, row_bytes) uint8 payload -> (rows, cols) float32 on the GPU
    (``_decode_quant_tensor``, t81/gguf.py:1020-1069)."""
    code = _quant_code(quant)
    rows, cols = int(shape[0]), int(shape[1]) if len(shape) > 1 else 1
    if not payload.is_cuda:
        payload = payload.to("cuda")
    payload = payload.reshape(-1).contiguous()
    if payload.dtype != torch.uint8:
        raise ValueError("payload must be uint8")
    if payload.numel() < rows * row_bytes(cols, code):
        raise ValueError("quantized tensor data truncated")
    out = torch.empty((rows, cols), dtype=torch.float32, device=payload.device)
    _lib.check(_lib.lib().t81_hip_tq_dequantize(payload.data_ptr(), out.data_ptr(), rows, cols,
                                                code, _stream()))
    return out


_X_CODES = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16,
            torch.int8: _lib.DTYPE_I8}


def tq2_matmul(x: torch.Tensor, w_tq2: torch.Tensor, k: int, alpha: float = 1.0,
               beta: float = 0.0, c: Optional[torch.Tensor] = None,
               bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """C = alpha * x @ W^T + beta * C + bias with W the TQ2_0 payload (N rows), read
    directly.  x: (M, K) float32 / bfloat16 / int8 on the GPU; C float32 (M, N)."""
    if x.ndim != 2 or x.shape[1] != k:
        raise ValueError("x must be (M, K)")
    if x.dtype not in _X_CODES:
        x = x.float()
    x = x.contiguous()
    m = x.shape[0]
    rb = row_bytes(k, GGML_TYPE_TQ2_0)
    if w_tq2.dtype != torch.uint8 or w_tq2.numel() % max(rb, 1) != 0:
        raise ValueError("w_tq2 must be a uint8 TQ2_0 payload of whole rows")
    w_tq2 = w_tq2.contiguous()
    # K = 0 rows hold no blocks: N then comes from C (or the bias)
    n = w_tq2.numel() // rb if rb else (c.shape[1] if c is not None else
                                         (bias.numel() if bias is not None else 0))
    if c is None:
        if beta != 0.0:
            raise ValueError("beta != 0 needs an input C")
        c = torch.empty((m, n), dtype=torch.float32, device=x.device)
    elif tuple(c.shape) != (m, n) or c.dtype != torch.float32 or not c.is_contiguous():
        raise ValueError("C tensor shape must match (M, N)")
    bias_ptr = None
    if bias is not None:
        if bias.numel() != n:
            raise ValueError("bias must have N elements")
        bias = bias.float().contiguous()
        bias_ptr = bias.data_ptr()
    _lib.check(_lib.lib().t81_hip_tq2_matmul(x.data_ptr(), _X_CODES[x.dtype], w_tq2.data_ptr(),
                                             c.data_ptr(), m, n, k, alpha, beta, bias_ptr,
                                             _stream()))
    return c


# ---- the reference's own TQ1_0 row codec (src/t81/core/gguf_quants.h), batched ----
TQ1_TRITS_PER_BLOCK = 8   # gguf_quants.h:14
TQ1_BLOCK_ROWS = 32       # gguf_quants.h:15


def _cuda_f32(t: torch.Tensor) -> torch.Tensor:
    if not t.is_cuda:
        t = t.to("cuda")
    return t.to(torch.float32).contiguous()


def quantize_rows_tq1_0(matrix: torch.Tensor, threshold: float = 0.45,
                        scales: Optional[torch.Tensor] = None
                        ) -> "tuple[torch.Tensor, torch.Tensor]":
    """(rows, cols) floats -> (scales float32 (rows,), words uint16 (rows, ceil(cols / 8))):
    quantize_row_tq1_0 (gguf_quants.h:116-144) on every row in one launch.  Row r uses
    scales[r] when given and > 0, else its max |v|; the scales used are returned."""
    src = _cuda_f32(matrix)
    if src.ndim != 2:
        raise ValueError("quantize_rows_tq1_0 expects a 2-D tensor")
    rows, cols = src.shape
    s_in = None
    if scales is not None:
        s_in = _cuda_f32(scales).reshape(-1)
        if s_in.numel() != rows:
            raise ValueError("scales must have one value per row")
    s_out = torch.zeros(rows, dtype=torch.float32, device=src.device)
    words = torch.empty((rows, (cols + 7) // 8), dtype=torch.uint16, device=src.device)
    _lib.check(_lib.lib().t81_hip_tq1_quantize_rows(
        src.data_ptr(), rows, cols, float(threshold),
        s_in.data_ptr() if s_in is not None else None, s_out.data_ptr(), words.data_ptr(),
        _stream()))
    return s_out, words


def dequant_rows_tq1_0(words: torch.Tensor, cols: int, scales: torch.Tensor) -> torch.Tensor:
    """(rows, ceil(cols / 8)) uint16 words and per-row scales -> (rows, cols) float32
    (dequantize_row_tq1_0, gguf_quants.h:146-168, on every row)."""
    if not words.is_cuda:
        words = words.to("cuda")
    if words.dtype not in (torch.uint16, torch.int16) or words.ndim != 2:
        raise ValueError("words must be a 2-D uint16 tensor")
    words = words.contiguous()
    rows = words.shape[0]
    if words.shape[1] < (cols + 7) // 8:
        raise ValueError("packed buffer too small for the requested column count")
    if words.shape[1] != (cols + 7) // 8:
        words = words[:, :(cols + 7) // 8].contiguous()
    s = _cuda_f32(scales).reshape(-1)
    if s.numel() != rows:
        raise ValueError("scales must have one value per row")
    out = torch.empty((rows, int(cols)), dtype=torch.float32, device=words.device)
    _lib.check(_lib.lib().t81_hip_tq1_dequantize_rows(words.data_ptr(), rows, cols, s.data_ptr(),
                                                      out.data_ptr(), _stream()))
    return out


def tq1_payload_bytes(rows: int, cols: int, block_rows: int = TQ1_BLOCK_ROWS,
                      refinements: bool = False) -> int:
    n = int(_lib.lib().t81_hip_tq1_payload_bytes(rows, cols, block_rows, int(refinements)))
    if n < 0:
        _lib.check(n)
    return n


def quantize_tq1_0_payload(matrix: torch.Tensor, block_rows: int = TQ1_BLOCK_ROWS,
                           refinements: bool = False, threshold: float = 0.45) -> torch.Tensor:
    """(rows, cols) floats -> the uint8 payload t81lib.dequant_tq1_0 (refinements False) or
    dequant_tq2_0 (True) reads: per group of block_rows rows a float16 scale
    h = half(max |v|), 8 zero bytes with refinements, then each row's words from
    quantize_row_tq1_0 with the scale float(h).  The reference has no writer for this
    payload; this one composes its row codec the way a caller of the binding would."""
    src = _cuda_f32(matrix)
    if src.ndim != 2:
        raise ValueError("quantize_tq1_0_payload expects a 2-D tensor")
    rows, cols = src.shape
    out = torch.empty(tq1_payload_bytes(rows, cols, block_rows, refinements), dtype=torch.uint8,
                      device=src.device)
    _lib.check(_lib.lib().t81_hip_tq1_quantize_payload(src.data_ptr(), rows, cols, block_rows,
                                                       int(refinements), float(threshold),
                                                       out.data_ptr(), _stream()))
    return out

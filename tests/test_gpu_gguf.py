"""GGUF TQ1_0 / TQ2_0 codecs and the TQ2_0 matmul on the GPU against the CPU oracle.

Codecs: bit-exact payload bytes and decoded floats (the formats are byte layouts;
the arithmetic is float32 with the reference's numpy roundings).  Matmul:
|y - ref| <= rtol * (|alpha| sum_k |x_k w_k| + |beta c| + |bias|) with rtol 1e-2
for bfloat16 and 1e-3 for float32 activations, exact-integer activations for int8
up to the float32 scale products (same 1e-3 bound).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import oracle
from t81lib_amd import gguf
from conftest import fp_tolerance_ok

pytestmark = pytest.mark.gpu

QUANTS = {"TQ1_0": oracle.TQ1_0, "TQ2_0": oracle.TQ2_0}


def announce(case: str) -> None:
    sys.__stderr__.write(f"[gpu case] {case}\n")
    sys.__stderr__.flush()


def weights(rows, cols, seed, specials=False):
    g = np.random.default_rng(seed)
    w = g.standard_normal((rows, cols)).astype(np.float32)
    if w.size:
        w[g.random(w.shape) < 0.01] *= 10.0
    if specials and w.size >= 8:
        flat = w.reshape(-1)
        flat[:6] = [np.inf, -np.inf, 0.0, -0.0, 7e4, -1e-30]
    return w


@pytest.mark.parametrize("quant", list(QUANTS))
@pytest.mark.parametrize("threshold", [0.45, 0.25, 0.0, 1.0, 3.0])
@pytest.mark.parametrize("shape", [(3, 4), (64, 128), (7, 600), (33, 1000), (5, 256), (1, 1),
                                   (2, 513), (0, 10), (4, 0), (6, 768), (3, 4096)])
def test_codecs_bit_exact(gpu, quant, threshold, shape):
    announce(f"tq codec {quant} thr={threshold} shape={shape}")
    rows, cols = shape
    w = weights(rows, cols, seed=rows * 131 + cols, specials=(threshold == 0.45))
    want = oracle.tq_quantize(w, threshold, QUANTS[quant])
    got = gguf.quantize_tensor(torch.from_numpy(w).to(gpu), quant, threshold).cpu().numpy()
    np.testing.assert_array_equal(got, want)
    dec_want = oracle.tq_dequantize(want, rows, cols, QUANTS[quant])
    dec_got = gguf.dequantize_tensor(torch.from_numpy(want).to(gpu), shape, quant).cpu().numpy()
    np.testing.assert_array_equal(dec_got.view(np.uint32), dec_want.view(np.uint32))


@pytest.mark.parametrize("cols", [1000, 1024])
@pytest.mark.parametrize("quant", list(QUANTS))
def test_dequantize_any_bytes(gpu, quant, cols):
    """Every byte value decodes (TQ2_0 digit 3 -> 2, TQ1_0 bytes >= 243 wrap) as the oracle
    (cols 1024: whole blocks, the float4 path)."""
    announce(f"tq dequant random bytes {quant} cols={cols}")
    rows = 17
    nbytes = gguf.row_bytes(cols, quant)
    g = np.random.default_rng(5)
    payload = g.integers(0, 256, (rows, nbytes), dtype=np.uint8)
    bb = 54 if quant == "TQ1_0" else 66
    blocks = payload.reshape(rows, -1, bb)
    blocks[..., -2:] = np.frombuffer(np.float16(0.75).tobytes(), np.uint8)  # finite scales
    want = oracle.tq_dequantize(payload, rows, cols, QUANTS[quant])
    got = gguf.dequantize_tensor(torch.from_numpy(payload).to(gpu), (rows, cols), quant)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("quant,thr,lo,hi,shape", [
    ("TQ1_0", 0.45, -1.0, 0.8, (3, 4)),     # tests/python/test_gguf.py:68-75
    ("TQ2_0", 0.25, -0.9, 0.9, (3, 4)),
    ("TQ2_0", 0.45, -0.9, 0.9, (3, 4)),     # test_roundtrip_gguf_tq2
    ("TQ1_0", 0.45, -5.0, 5.0, (64, 128)),  # test_roundtrip_large_linear
])
def test_reference_roundtrip_cases(gpu, quant, thr, lo, hi, shape):
    announce(f"tq reference case {quant} {shape}")
    w = torch.linspace(lo, hi, shape[0] * shape[1], dtype=torch.float32).reshape(shape)
    payload = gguf.quantize_tensor(w.to(gpu), quant, thr)
    decoded = gguf.dequantize_tensor(payload, shape, quant).cpu()
    assert decoded.shape == shape and torch.isfinite(decoded).all()
    want = oracle.tq_dequantize(oracle.tq_quantize(w.numpy(), thr, QUANTS[quant]), *shape,
                                QUANTS[quant])
    np.testing.assert_array_equal(decoded.numpy(), want)


MATMUL = [  # M, N, K
    (1, 300, 4096), (1, 17, 256), (2, 64, 1000), (3, 31, 4100), (4, 129, 14336),
    (5, 40, 3072), (9, 33, 512), (16, 70, 2048), (1, 5, 300), (4, 1000, 4096), (1, 8, 100000),
]


@pytest.mark.parametrize("M,N,K", MATMUL)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.int8])
def test_tq2_matmul_vs_oracle(gpu, M, N, K, dtype):
    announce(f"tq2 matmul {dtype} M={M} N={N} K={K}")
    g = torch.Generator("cpu").manual_seed(M * 7919 + N * 31 + K)
    w = torch.randn((N, K), generator=g)
    payload = oracle.tq_quantize(w.numpy(), 0.45, oracle.TQ2_0)
    if dtype == torch.int8:
        x = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    else:
        x = torch.randn((M, K), generator=g).to(dtype)
    c0 = torch.randn((M, N), generator=g)
    bias = torch.randn((N,), generator=g)
    xd = x.to(torch.float64).numpy()
    acc, scale_acc = oracle.tq2_matmul_f64(xd, payload, K)
    wg = torch.from_numpy(payload).to(gpu)
    rtol = 1e-2 if dtype == torch.bfloat16 else 1e-3
    for alpha, beta, use_bias in ((1.0, 0.0, False), (0.5, 1.0, True), (-2.0, 0.25, False)):
        c = c0.clone().to(gpu)
        out = gguf.tq2_matmul(x.to(gpu), wg, K, alpha=alpha, beta=beta,
                              c=c if beta != 0.0 else None,
                              bias=bias.to(gpu) if use_bias else None).cpu().numpy()
        cc = c0.to(torch.float64).numpy()
        ref = alpha * acc + (beta * cc if beta != 0 else 0)
        scale = abs(alpha) * scale_acc + (abs(beta) * np.abs(cc) if beta != 0 else 0)
        if use_bias:
            ref = ref + bias.to(torch.float64).numpy()
            scale = scale + np.abs(bias.to(torch.float64).numpy())
        ok, worst, nbad = fp_tolerance_ok(out, ref, scale, rtol)
        assert ok, f"alpha={alpha} beta={beta}: {nbad} outside, worst rel {worst:.3g}"


def test_tq2_matmul_zero_k_and_empty(gpu):
    announce("tq2 matmul K=0 and empty shapes")
    c = torch.randn((3, 5), device=gpu)
    bias = torch.randn((5,), device=gpu)
    want = (0.5 * c + bias).cpu()
    out = gguf.tq2_matmul(torch.empty((3, 0), device=gpu), torch.empty((0,), dtype=torch.uint8,
                          device=gpu), 0, beta=0.5, c=c, bias=bias)
    # no blocks: N is taken from C, the payload is empty
    torch.testing.assert_close(out.cpu(), want, rtol=0, atol=0)


def test_argument_errors(gpu):
    announce("tq argument errors")
    w = torch.randn((4, 300), device=gpu)
    with pytest.raises(ValueError, match="quant must be one of"):
        gguf.quantize_tensor(w, "INVALID")
    with pytest.raises(ValueError):
        gguf.quantize_tensor(torch.randn(3, device=gpu), "TQ2_0")
    payload = gguf.quantize_tensor(w, "TQ2_0")
    with pytest.raises(ValueError, match="truncated"):
        gguf.dequantize_tensor(payload[:2], (4, 300), "TQ2_0")
    x = torch.randn((1, 300), device=gpu)
    with pytest.raises(ValueError, match="misaligned"):
        flat = torch.empty(payload.numel() + 2, dtype=torch.uint8, device=gpu)
        flat[2:] = payload.reshape(-1)
        gguf.tq2_matmul(x, flat[2:], 300)

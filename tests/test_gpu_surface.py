"""The reference's Python surface on the GPU path: t81lib.gemm_ternary, TernaryTensor,
t8.nn.Linear -- the reference's own tests re-run here, plus value checks they lack."""

from __future__ import annotations

import array
import sys
import warnings

import numpy as np
import pytest
import torch

from t81lib_amd import nn as t8nn, ops, t81lib
from t81lib_amd.tensor import TernaryTensor, trit
from conftest import accum_rtol, fp_tolerance_ok

pytestmark = pytest.mark.gpu


def announce(case: str) -> None:
    sys.__stderr__.write(f"[gpu case] {case}\n")
    sys.__stderr__.flush()


def test_reference_binding_known_answers(gpu):
    """tests/python/test_bindings.py:16-38 with the same buffers (memoryview + array.array)."""
    announce("surface gemm_ternary known answers")
    M, N, K = 2, 3, 48
    a = memoryview(bytearray(bytes([13] * 16) * M))
    b = memoryview(bytearray(bytes([13] * 16) * N))
    c = array.array("f", [0.0] * (M * N))
    t81lib.gemm_ternary(a, b, c, M, N, K)
    assert all(abs(v) <= 1e-6 for v in c)
    c = array.array("f", [2.0] * (M * N))
    t81lib.gemm_ternary(a, b, c, M, N, K, alpha=0.0, beta=0.5)
    assert all(abs(v - 1.0) <= 1e-6 for v in c)
    assert t81lib.HAS_ROCM_BACKEND


def test_gemm_ternary_device_tensors_in_place(gpu, golden):
    announce("surface gemm_ternary device tensors")
    i = list(golden["g_names"]).index("low5")
    M, N, K = (int(v) for v in golden[f"g{i}_shape"])
    al, be = (float(v) for v in golden[f"g{i}_ab"])
    c = torch.from_numpy(golden[f"g{i}_C"].copy()).to(gpu)
    t81lib.gemm_ternary(torch.from_numpy(golden[f"g{i}_A"]).to(gpu),
                        torch.from_numpy(golden[f"g{i}_B"]).to(gpu), c, M, N, K, al, be)
    np.testing.assert_array_equal(c.cpu().numpy().view(np.uint32),
                                  golden[f"g{i}_out"].view(np.uint32))


def test_reference_torch_tests(gpu):
    """tests/python/test_torch_ternary.py:17-42: shapes, device round trip, move warning."""
    announce("surface TernaryTensor reference tests")
    weight = torch.linspace(-1.0, 1.0, steps=48, dtype=torch.float32).reshape(3, 16)
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always", RuntimeWarning)
        ternary = TernaryTensor.from_float(weight, threshold=0.45)
    assert any("moving tensor" in str(item.message) for item in caught)
    assert ternary.dtype is trit
    rhs = torch.randn(16, 4, dtype=torch.float32)
    out = torch.matmul(ternary, rhs)
    assert out.shape == (3, 4) and out.device.type == "cpu"
    rhs_gpu = rhs.to(gpu)
    out_gpu = torch.matmul(ternary, rhs_gpu)
    assert out_gpu.device == rhs_gpu.device
    # values: T @ rhs with T the 0.45-thresholded linspace
    t = torch.where(weight >= 0.45, 1.0, torch.where(weight <= -0.45, -1.0, 0.0))
    torch.testing.assert_close(out_gpu.cpu(), t @ rhs, rtol=1e-4, atol=1e-4)


def test_matmul_input_and_backward(gpu, orc):
    announce("surface matmul_input + backward")
    g = torch.Generator("cpu").manual_seed(1)
    w = torch.randn(70, 200, generator=g)
    t = TernaryTensor.from_float(w.to(gpu), threshold=0.45)
    x = torch.randn(5, 200, generator=g).to(gpu).requires_grad_(True)
    y = t.matmul_input(x)
    trits = torch.from_numpy(orc.unpack(orc.pack_rows(w.numpy(), np.float32(0.45), 1),
                                        70, 200)).float()
    torch.testing.assert_close(y.detach().cpu(), x.detach().cpu() @ trits.T, rtol=1e-4,
                               atol=1e-4)
    y.sum().backward()
    torch.testing.assert_close(x.grad.cpu(), trits.sum(0).expand(5, 200), rtol=0, atol=0)
    np.testing.assert_array_equal(t.trits().cpu().numpy(), trits.numpy().astype(np.int8))


def test_reference_limb_semantics_matches_oracle(gpu, orc):
    """semantics='reference_limb' reproduces the literal reference matmul_input."""
    announce("surface reference_limb")
    g = torch.Generator("cpu").manual_seed(2)
    w = torch.randn(40, 100, generator=g) * 0.3
    x = torch.randn(6, 100, generator=g) * 0.3
    t = TernaryTensor.from_float(w.to(gpu), threshold=0.45, semantics="reference_limb")
    y = t.matmul_input(x.to(gpu)).cpu().numpy()          # (tokens, rows)
    wp = orc.pack_rows(w.numpy(), np.float32(orc.torch_threshold(0.45)), 1)
    xp = orc.pack_cols(x.numpy(), np.float32(orc.torch_threshold(0.5)), 1)
    want = orc.gemm_limb(wp, xp, np.zeros((40, 6), np.float32), 40, 6, wp.shape[1] * 48)
    np.testing.assert_array_equal(y.T.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("tokens", [1, 4, 33])
def test_linear_eval_vs_oracle(gpu, orc, tokens):
    announce(f"surface Linear eval tokens={tokens}")
    torch.manual_seed(tokens)
    layer = t8nn.Linear(300, 130).to(gpu)
    with torch.no_grad():
        layer.weight.mul_(50.0)  # N(0,1)-ish weights so that ~1/3 of the trits are zero
    layer.eval()
    x = torch.randn(2, tokens, 300, device=gpu, dtype=torch.bfloat16)
    with torch.no_grad():
        y = layer(x)
    assert y.shape == (2, tokens, 130)
    wp = orc.pack_rows(layer.weight.detach().cpu().numpy(),
                       np.float32(orc.torch_threshold(0.45)), 1)
    xf = x.reshape(-1, 300).double().cpu().numpy()
    b = layer.bias.detach().double().cpu().numpy()
    ref = orc.trit_matmul_f64(xf, wp, 300) + b
    scale = orc.trit_matmul_abs_f64(xf, wp, 300) + np.abs(b)
    ok, worst, nbad = fp_tolerance_ok(y.reshape(-1, 130).float().cpu().numpy(), ref, scale,
                                      accum_rtol(300, torch.bfloat16))
    assert ok, f"{nbad} outside, worst {worst:.3g}"
    assert layer.ternary_weight is not None
    layer.train()
    assert layer.ternary_weight is None


@pytest.mark.parametrize("rows,cols", [(70, 200), (1, 1), (48, 48), (49, 97), (300, 1000),
                                       (1000, 300), (96, 192), (5, 4097), (2500, 1300)])
def test_transpose_packed_bit_exact(gpu, orc, rows, cols):
    """T^T limbs equal the oracle's pack of the transposed unpacked trits (zero-padded).
    (2500 x 1300: 14 x 7 = 98 tiles, so the eight XCDs' shares of the tile order differ
    in size.)"""
    announce(f"transpose_packed {rows}x{cols}")
    g = torch.Generator("cpu").manual_seed(rows * 1000 + cols)
    w = torch.randn(rows, cols, generator=g)
    packed = orc.pack_rows(w.numpy(), np.float32(0.45), 0)
    trits = orc.unpack(packed, rows, cols)
    want = orc.pack_trits_rows(np.ascontiguousarray(trits.T))
    got = ops.transpose_packed(torch.from_numpy(packed).to(gpu), rows, cols).cpu().numpy()
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("rows,cols,tokens", [(70, 200, 5), (300, 1000, 64), (1024, 512, 512),
                                              (4096, 1000, 33)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_grad_input_vs_oracle(gpu, orc, rows, cols, tokens, dtype):
    """grad_rhs = T^T @ grad_output (t81/torch/__init__.py:291-304) through the transposed
    limbs and the forward GEMM, within the float32 summation bound of sum |t g| (K = rows)."""
    announce(f"grad_input {rows}x{cols} tokens={tokens} {dtype}")
    g = torch.Generator("cpu").manual_seed(rows + cols + tokens)
    w = torch.randn(rows, cols, generator=g)
    t = TernaryTensor.from_float(w.to(gpu), threshold=0.45)
    grad = torch.randn(rows, tokens, generator=g).to(dtype)
    got = t.grad_input(grad.to(gpu)).cpu().numpy()                       # (cols, tokens)
    trits = t.trits().cpu().numpy().astype(np.float64)                  # (rows, cols)
    gd = grad.to(torch.float64).numpy()
    want = trits.T @ gd
    scale = np.abs(trits.T) @ np.abs(gd)
    ok, worst, nbad = fp_tolerance_ok(got, want, scale, accum_rtol(rows, dtype))
    assert ok, f"{nbad} outside, worst rel {worst:.3g}"
    # the cache follows the weights
    t.update_from_float((-w).to(gpu))
    np.testing.assert_array_equal(t.transposed_packed().cpu().numpy(),
                                  ops.transpose_packed(t.packed, rows, cols).cpu().numpy())

"""K1 quantize+pack and the codec kernels on the GPU, bit-exact against the oracle."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from t81lib_amd import _lib, ops, t81lib

pytestmark = pytest.mark.gpu


def announce(case: str) -> None:
    sys.__stderr__.write(f"[gpu case] {case}\n")
    sys.__stderr__.flush()


def weights(rows, cols, seed, scale=0.02, outliers=True):
    g = torch.Generator("cpu").manual_seed(seed)
    w = torch.randn((rows, cols), generator=g, dtype=torch.float32) * scale
    if outliers:
        mask = torch.rand((rows, cols), generator=g) < 0.01
        w[mask] *= 10
    return w


@pytest.mark.parametrize("rows,cols", [(3072, 3072), (8192, 3072)])
def test_pack_config2_bit_exact(gpu, orc, rows, cols):
    announce(f"K1 config2 {rows}x{cols}")
    w = weights(rows, cols, 0)
    got = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    torch.cuda.synchronize()
    want = orc.pack_rows(w.numpy(), 0.45, 0)
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    # effective weights W/0.02 (~34.7% zeros) through the torch form
    weff = w / 0.02
    got = ops.quantize_pack(weff.to(gpu), ops.torch_threshold(0.45), _lib.THR_TORCH)
    want = orc.pack_rows(weff.numpy(), np.float32(orc.torch_threshold(0.45)), 1)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("cols", [1, 2, 12, 47, 48, 49, 95, 97, 1000, 4097])
@pytest.mark.parametrize("aligned", [True, False])
def test_pack_ragged_shapes(gpu, orc, cols, aligned):
    announce(f"K1 ragged cols={cols} aligned={aligned}")
    w = weights(37, cols, cols, scale=1.0, outliers=False)
    src = w.to(gpu)
    if not aligned:  # an offset view breaks 16-byte alignment of the rows
        big = torch.empty(37 * cols + 1, dtype=torch.float32, device=gpu)
        big[1:] = src.reshape(-1)
        src = big[1:].view(37, cols)
    got = ops.quantize_pack(src, 0.5, _lib.THR_CPP)
    np.testing.assert_array_equal(got.cpu().numpy(), orc.pack_rows(w.numpy(), 0.5, 0))


@pytest.mark.parametrize("thr", [1e-6, 0.3, 0.45, 0.5, 0.9999, 1.0])
def test_pack_thresholds_and_special_values(gpu, orc, thr):
    announce(f"K1 thresholds thr={thr}")
    t32 = np.float32(thr)
    specials = np.array([t32, np.nextafter(t32, 2), np.nextafter(t32, -2), -t32,
                         np.nextafter(-t32, 2), np.nextafter(-t32, -2), 0.0, -0.0, 1.0, -1.0,
                         1.5, -1.5, np.inf, -np.inf, np.nan, 1e-30, -1e-30, 3e38], np.float32)
    w = np.resize(specials, (5, 150)).astype(np.float32)
    for mode in (_lib.THR_CPP, _lib.THR_TORCH):
        th = thr if mode == _lib.THR_CPP else orc.torch_threshold(thr)
        got = ops.quantize_pack(torch.from_numpy(w).to(gpu), th, mode)
        np.testing.assert_array_equal(got.cpu().numpy(), orc.pack_rows(w, th, mode),
                                      err_msg=f"mode={mode}")


def test_pack_torch_form_threshold_zero(gpu, orc):
    """torch form at threshold 0: zeros become -1 ('-1 wins', t81/torch/__init__.py:48-49)."""
    announce("K1 torch form thr=0")
    w = np.array([[0.0, -0.0, 1e-9, -1e-9, 0.7] * 10], np.float32)
    got = ops.quantize_pack(torch.from_numpy(w).to(gpu), 0.0, _lib.THR_TORCH)
    np.testing.assert_array_equal(got.cpu().numpy(), orc.pack_rows(w, 0.0, 1))
    assert orc.unpack(orc.pack_rows(w, 0.0, 1), 1, 50)[0, 0] == -1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_pack_half_inputs_match_float32_pack(gpu, orc, dtype):
    announce(f"K1 {dtype}")
    w = weights(64, 300, 4, scale=1.0, outliers=False).to(dtype)
    got = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    np.testing.assert_array_equal(got.cpu().numpy(), orc.pack_rows(w.float().numpy(), 0.45, 0))


def test_pack_empty(gpu):
    announce("K1 empty")
    assert ops.quantize_pack(torch.zeros((0, 5), device=gpu), 0.5).shape == (0, 1, 16)
    assert ops.quantize_pack(torch.zeros((4, 0), device=gpu), 0.5).shape == (4, 0, 16)


def test_quantize_unpack_pack_cols_validate(gpu, orc):
    announce("codec kernels")
    w = weights(33, 211, 7, scale=1.0, outliers=False)
    wg = w.to(gpu)
    q = ops.quantize(wg, 0.45, _lib.THR_CPP).cpu().numpy()
    want_t = orc.unpack(orc.pack_rows(w.numpy(), 0.45, 0), 33, 211)
    np.testing.assert_array_equal(q, want_t)
    packed = ops.quantize_pack(wg, 0.45, _lib.THR_CPP)
    np.testing.assert_array_equal(ops.unpack(packed, 33, 211).cpu().numpy(), want_t)
    np.testing.assert_array_equal(ops.unpack(packed, 33, 100).cpu().numpy(), want_t[:, :100])
    cols = ops.pack_cols(wg, 0.5, _lib.THR_TORCH)
    np.testing.assert_array_equal(cols.cpu().numpy(), orc.pack_cols(w.numpy(), 0.5, 1))
    assert ops.count_invalid_bytes(packed) == 0
    bad = packed.clone()
    bad.view(-1)[[0, 5, 99]] = torch.tensor([27, 200, 255], dtype=torch.uint8, device=gpu)
    assert ops.count_invalid_bytes(bad) == 3


def test_reference_surface_pack_and_quantize(gpu, orc):
    announce("t81lib.pack_dense_matrix / quantize_to_trits / unpack_packed_limbs")
    w = weights(16, 100, 3, scale=1.0, outliers=False).numpy()
    packed = t81lib.pack_dense_matrix(w)            # default threshold 0.5, numpy in/out
    assert isinstance(packed, np.ndarray) and packed.dtype == np.uint8
    np.testing.assert_array_equal(packed, orc.pack_rows(w, 0.5, 0))
    t = t81lib.quantize_to_trits(w, 0.5)
    np.testing.assert_array_equal(t, orc.unpack(packed, 16, 100))
    np.testing.assert_array_equal(t81lib.unpack_packed_limbs(packed, 16, 100), t)
    np.testing.assert_array_equal(t81lib.dequantize_trits(t), t.astype(np.float32))
    bad = packed.copy()
    bad[0, 0, 0] = 27
    with pytest.raises(ValueError, match="canonical"):
        t81lib.unpack_packed_limbs(bad, 16, 100)

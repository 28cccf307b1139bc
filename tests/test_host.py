"""Host-side logic of the Python surface, on the CPU: argument checks that the reference
binding performs before computing, and the loud failure when no GPU is present."""

from __future__ import annotations

import array

import numpy as np
import pytest
import torch

from t81lib_amd import _lib, nn as t8nn, ops, t81lib
from t81lib_amd.tensor import TernaryTensor, trit


def test_constants_mirror_reference():
    assert (t81lib.TRITS_PER_LIMB, t81lib.TRYTES_PER_LIMB, t81lib.BYTES_PER_LIMB) == (48, 16, 16)
    assert ops.limbs_for(4096) == 86 and ops.limbs_for(14336) == 299 and ops.limbs_for(0) == 0
    assert ops.torch_threshold(2.0) == 0.9999 and ops.torch_threshold(-1.0) == 0.0
    assert repr(trit) == "t81.trit"


def test_reference_argument_errors_before_any_device_work():
    with pytest.raises(ValueError, match="between 0 \\(exclusive\\) and 1"):
        t81lib.pack_dense_matrix(np.zeros((2, 2), np.float32), threshold=0.0)
    with pytest.raises(ValueError, match="between 0 \\(exclusive\\) and 1"):
        t81lib.quantize_to_trits(np.zeros(3, np.float32), threshold=1.01)
    with pytest.raises(ValueError, match="K must be divisible"):
        t81lib.gemm_ternary(b"\x0d" * 16, b"\x0d" * 16, array.array("f", [0.0]), 1, 1, 47)
    with pytest.raises(ValueError, match="non-negative"):
        t81lib.gemm_ternary(b"", b"", array.array("f"), -1, 1, 48)
    with pytest.raises(ValueError, match="non-negative"):
        t81lib.unpack_packed_limbs(np.zeros((1, 1, 16), np.uint8), -1, 3)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU failure mode")
def test_no_gpu_fails_loudly_instead_of_falling_back():
    with pytest.raises((_lib.T81HipError, RuntimeError)):
        t81lib.pack_dense_matrix(np.zeros((2, 2), np.float32), 0.5)
    with pytest.raises((_lib.T81HipError, RuntimeError)):
        TernaryTensor.from_float(torch.zeros(3, 16), threshold=0.45)
    layer = t8nn.Linear(16, 3).eval()
    with pytest.raises((_lib.T81HipError, RuntimeError)):
        layer(torch.zeros(2, 16))


def test_ternary_tensor_metadata_and_guard():
    packed = torch.full((3, 1, 16), 13, dtype=torch.uint8)
    t = TernaryTensor(packed, (3, 16), k_actual=16, k_limbs=1, threshold=0.45)
    assert t.shape == (3, 16) and t.dtype is trit and t.ndim == 2
    assert t._threshold == pytest.approx(0.45)
    with pytest.raises(NotImplementedError):
        t + 1
    with pytest.raises(ValueError):
        TernaryTensor(packed, (3, 16), k_actual=16, k_limbs=1, semantics="bogus")


def test_linear_train_mode_is_quantization_aware():
    """Train mode (t81/nn/linear.py:43-45,72-99): F.linear with ternary(w/s)*s, straight-through
    gradient to the float weight."""
    torch.manual_seed(0)
    layer = t8nn.Linear(8, 4, threshold=0.45)
    x = torch.randn(3, 8)
    y = layer(x)
    s = layer.weight.detach().abs().amax()
    wq = layer.weight.detach() / s
    q = torch.where(wq.abs() >= 0.45, wq.sign(), torch.zeros_like(wq)) * s
    torch.testing.assert_close(y, torch.nn.functional.linear(x, q, layer.bias))
    y.sum().backward()
    assert layer.weight.grad is not None and layer.weight.grad.abs().sum() > 0
    assert layer.ternary_weight is None
    layer.eval()
    assert layer.ternary_weight is None  # packed lazily on the first eval forward


def test_module_to_trit_argument_handling():
    """model.to(dtype=trit) takes the trit marker out before torch's own Module.to (which
    would raise TypeError on it), converts only then, and needs the GPU (no CPU fallback);
    other .to calls pass through."""
    from t81lib_amd import tensor as tt

    assert tt._extract_dtype_arg((), {"dtype": trit}) is trit
    assert tt._extract_dtype_arg((trit,), {}) is trit
    assert tt._extract_dtype_arg(("cpu", torch.float16), {}) is torch.float16
    assert tt._extract_dtype_arg(("cpu",), {}) is None
    layer = torch.nn.Linear(4, 3)
    assert layer.to(torch.float64) is layer and layer.weight.dtype == torch.float64
    if not torch.cuda.is_available():
        with pytest.raises((_lib.T81HipError, RuntimeError)):
            layer.to(dtype=trit)
    # without a cache the patched forward is the original
    x = torch.randn(2, 4, dtype=torch.float64)
    torch.testing.assert_close(layer(x), torch.nn.functional.linear(x, layer.weight, layer.bias))

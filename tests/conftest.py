"""Shared test setup.

Markers: ``gpu`` tests need a gfx950 device and the built libt81_hip.so; they
compare the HIP path with the CPU oracle (oracle/) through the C ABI.
Everything else runs on the CPU: the oracle against the golden vectors of the
compiled reference, host-side validation, and the library's exports.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden", "ref_vectors.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built libt81_hip.so")


@pytest.fixture(scope="session")
def golden():
    return np.load(GOLDEN)


@pytest.fixture(scope="session")
def orc():
    import oracle

    if not os.path.exists(os.path.join(ROOT, "oracle", "liboracle.so")):
        oracle.build(reference=False)
    return oracle


@pytest.fixture(scope="session")
def gpu():
    """The torch CUDA device; fails (does not skip) when a gpu-marked test has no GPU,
    so a silent CPU pass is impossible."""
    import torch

    from t81lib_amd import _lib

    if not torch.cuda.is_available():
        pytest.fail("gpu-marked test run without a visible GPU")
    _lib.lib()
    if not _lib.available():
        pytest.fail(f"libt81_hip reports no gfx950 device: {_lib.last_error()}")
    return torch.device("cuda", 0)


U32 = 2.0 ** -24          # unit roundoff of float32
NORTH_STAR_RTOL = {"f32": 1e-3, "bf16": 1e-2}


def _dtype_name(dtype) -> str:
    s = str(dtype)
    if s in ("f32", "torch.float32"):
        return "f32"
    if s in ("bf16", "torch.bfloat16"):
        return "bf16"
    raise ValueError(f"no float tolerance for {dtype}")


def accum_rtol(k: int, dtype) -> float:
    """Tolerance of the trit-dot kernels, relative to sum_k |alpha x_k t_k| + |beta c| +
    |bias|.  A trit times a bf16 value is exact in float32, so the only error of a bf16
    product is float32 summation: n additions in any order lose at most (n - 1) u of the
    summed magnitudes (u = 2^-24); u is doubled for the matrix cores' internal rounding,
    and 16 more additions cover the split-K partial sums and the alpha / beta / bias
    epilogue.  float32 activations run as a hi + lo bf16 pair: twice the terms and a
    representation error |x - hi - lo| <= 2^-16 |x|.  The result is capped by the
    north-star elementwise tolerance (1e-2 bf16, 1e-3 float32), which only binds for
    float32 at very long K."""
    name = _dtype_name(dtype)
    terms = k if name == "bf16" else 2 * k
    bound = 2.0 * (terms + 16) * U32 + (0.0 if name == "bf16" else 2.0 ** -16)
    return min(bound, NORTH_STAR_RTOL[name])


def fixed_point_activations(M: int, K: int, amax: int, seed: int):
    """float32 activations x = a + b / 256 with integers |a| <= amax and |b| <= 127.

    Each x holds at most 11 significant bits, so the kernels' split x = hi + lo into two
    bfloat16 values is exact, every product x * t is a multiple of 2^-8, and as long as
    (256 amax + 127) K < 2^24 every partial sum, in any order, is a multiple of 2^-8
    below 2^16 in magnitude: float32 adds them without rounding.  A float32 kernel must
    then reproduce the integer oracle bit for bit.  Returns (a int8, b int8, x float32)."""
    assert (256 * amax + 127) * K < 2 ** 24, "activations too large for exact float32 sums"
    rng = np.random.default_rng(seed)
    a = rng.integers(-amax, amax + 1, (M, K), dtype=np.int64).astype(np.int8)
    b = rng.integers(-127, 128, (M, K), dtype=np.int64).astype(np.int8)
    x = (a.astype(np.float64) + b.astype(np.float64) / 256.0).astype(np.float32)
    return a, b, x


def fixed_point_acc256(orc, a, b, packed, K: int) -> np.ndarray:
    """256 * (x @ T^T) as int64 from the integer oracle, by linearity: 256 (a T) + b T."""
    return 256 * orc.trit_matmul_i64(a, packed, K) + orc.trit_matmul_i64(b, packed, K)


def _frac_bits(v: float) -> int:
    q = 0
    while v * 2.0 ** q != np.floor(v * 2.0 ** q):
        q += 1
        assert q <= 16, f"{v} is not a short binary fraction"
    return q


def fixed_point_expected(acc256, alpha: float, beta: float, c=None, bias=None) -> np.ndarray:
    """alpha * acc256 / 256 + beta * c + bias as float32, exactly.  c and bias hold
    integers; the terms share a grid of 2^-f and the asserted bound keeps every partial
    sum of them, in any order, on that grid within float32's 24 bits."""
    f = max(8 + _frac_bits(alpha), _frac_bits(beta))
    y = alpha * (acc256.astype(np.float64) / 256.0)
    mag = np.abs(y)
    if beta != 0.0:
        cd = np.asarray(c, np.float64)
        assert np.array_equal(cd, np.floor(cd)), "C must hold integers"
        y = y + beta * cd
        mag = mag + np.abs(beta * cd)
    if bias is not None:
        bd = np.asarray(bias, np.float64)
        assert np.array_equal(bd, np.floor(bd)), "bias must hold integers"
        y = y + bd
        mag = mag + np.abs(bd)
    assert float(mag.max(initial=0.0)) < 2.0 ** (24 - f), "epilogue would round in float32"
    out = y.astype(np.float32)
    assert np.array_equal(out.astype(np.float64), y)
    return out


def fp_tolerance_ok(got, ref, scale, rtol, atol=1e-6):
    """|got - ref| <= rtol * scale + atol elementwise, scale = sum_k |alpha x_k t_k| + |beta c| + |bias|
    (a relative tolerance on the terms that were summed, so cancellation in a sum does not
    demand more than the inputs carry)."""
    got = np.asarray(got, np.float64)
    err = np.abs(got - ref)
    bound = rtol * scale + atol
    bad = ~(err <= bound)
    return (not bad.any()), float((err / np.maximum(scale, 1e-30)).max(initial=0.0)), int(bad.sum())

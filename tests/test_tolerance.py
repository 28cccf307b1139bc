"""The float tolerance of the trit-dot tests is tight enough to catch a wrong kernel.

conftest.accum_rtol bounds only float32 summation error (the products of trits and
bfloat16 values are exact).  These CPU tests plant plausible kernel mistakes in the
oracle's output -- the tail limb of every row dropped, one middle limb dropped, one
trit's sign flipped -- and require the bound to reject each of them at the decode
shape K = 4096, while a float32 accumulation of the same products in a bad order
(sequential, the largest error of the usual orders) still passes.  The north-star
1e-2 bound of the previous tests let the dropped tail limb through on every output.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import accum_rtol, fp_tolerance_ok


def _problem(orc, M, N, K, seed):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((N, K)).astype(np.float32)
    packed = orc.pack_rows(w, np.float32(0.45), 0)
    # bfloat16 values: float32 with the low 16 bits cleared
    x = rng.standard_normal((M, K)).astype(np.float32)
    x = (x.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    return x.astype(np.float64), packed


def _fp32_sequential(x, trits):
    """sum_k x[m, k] t[n, k] accumulated left to right in float32."""
    prod = (x[:, None, :] * trits[None, :, :]).astype(np.float32)
    acc = np.zeros(prod.shape[:2], np.float32)
    for k in range(prod.shape[2]):
        acc = acc + prod[:, :, k]
    return acc.astype(np.float64)


@pytest.mark.parametrize("M", [1, 16])
def test_bound_rejects_planted_mistakes(orc, M):
    N, K = 512, 4096
    x, packed = _problem(orc, M, N, K, seed=M)
    ref = orc.trit_matmul_f64(x, packed, K)
    scale = orc.trit_matmul_abs_f64(x, packed, K)
    rtol = accum_rtol(K, "bf16")
    L = packed.shape[1]

    trits = orc.unpack(packed, N, K).astype(np.float64)
    ok, worst, _ = fp_tolerance_ok(_fp32_sequential(x, trits), ref, scale, rtol)
    assert ok, f"a correct float32 accumulation must pass (worst {worst:.3g}, bound {rtol:.3g})"

    mutants = {}
    tail = packed.copy()
    tail[:, L - 1, :] = 13                                    # last limb: all-zero trits
    mutants["tail limb dropped"] = tail
    mid = packed.copy()
    mid[:, L // 2, :] = 13
    mutants["middle limb dropped"] = mid
    flip = orc.unpack(packed, N, K).copy()
    pick = np.random.default_rng(7)
    for n in range(N):                                        # one random nonzero trit per row
        flip[n, pick.choice(np.flatnonzero(flip[n]))] *= -1
    mutants["one trit sign flipped"] = orc.pack_trits_rows(flip)
    for name, bad_packed in mutants.items():
        got = orc.trit_matmul_f64(x, bad_packed, K)
        ok, _, nbad = fp_tolerance_ok(got, ref, scale, rtol)
        assert not ok, f"{name} passes the bound"
        assert nbad >= 0.2 * got.size, f"{name}: only {nbad} of {got.size} outputs rejected"
    # the previous 1e-2 bound accepted the dropped tail limb everywhere
    ok, _, _ = fp_tolerance_ok(orc.trit_matmul_f64(x, tail, K), ref, scale, 1e-2)
    assert ok


def test_bound_values():
    """The bound is the float32 summation bound, capped by the north-star tolerances."""
    assert accum_rtol(4096, "bf16") == pytest.approx(2 * (4096 + 16) * 2.0 ** -24)
    assert accum_rtol(48, "f32") == pytest.approx(2 * (96 + 16) * 2.0 ** -24 + 2.0 ** -16)
    assert accum_rtol(10 ** 6, "bf16") == 1e-2 and accum_rtol(14336, "f32") == 1e-3


def _bf16_rne(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("K", [97, 4096, 14336])
def test_fixed_point_pin_rejects_dropped_lo_plane(orc, K):
    """The bit-exact float32 tests (tests/test_gpu_exact_f32.py) catch a kernel that drops
    the lo bfloat16 plane of float32 activations, which the summation-bound tolerance lets
    through at long K.  The correct hi + lo split reproduces the expected bits."""
    from conftest import fixed_point_acc256, fixed_point_activations, fixed_point_expected

    M, N = 4, 384
    amax = 7 if (256 * 7 + 127) * K < 2 ** 24 else 3
    a, b, x = fixed_point_activations(M, K, amax, seed=K)
    w = np.random.default_rng(K + 1).standard_normal((N, K)).astype(np.float32)
    packed = orc.pack_rows(w, np.float32(0.45), 0)
    want = fixed_point_expected(fixed_point_acc256(orc, a, b, packed, K), 0.5, 0.0)

    hi = _bf16_rne(x)
    lo = _bf16_rne(x - hi)
    assert np.array_equal(hi.astype(np.float64) + lo, x.astype(np.float64)), "split must be exact"
    split = 0.5 * (orc.trit_matmul_f64(hi.astype(np.float64), packed, K)
                   + orc.trit_matmul_f64(lo.astype(np.float64), packed, K))
    assert np.array_equal(split.astype(np.float32).view(np.uint32), want.view(np.uint32))

    dropped = (0.5 * orc.trit_matmul_f64(hi.astype(np.float64), packed, K)).astype(np.float32)
    differ = float((dropped.view(np.uint32) != want.view(np.uint32)).mean())
    assert differ > 0.95, f"lo plane dropped: only {differ:.1%} of outputs differ"
    if K >= 4096:
        # the summation-bound tolerance alone accepts this mutant on most outputs at long K
        scale = 0.5 * orc.trit_matmul_abs_f64(x.astype(np.float64), packed, K)
        _, _, nbad = fp_tolerance_ok(dropped, want.astype(np.float64), scale, accum_rtol(K, "f32"))
        assert nbad < 0.5 * dropped.size

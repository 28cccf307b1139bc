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

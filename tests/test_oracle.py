"""Pins the CPU oracle (oracle/t81_oracle.c) before anything is compared with it.

Each oracle function is checked against (a) the golden vectors the compiled
reference produced (tests/golden/ref_vectors.npz, made by make_golden.py),
(b) the compiled reference itself when oracle/_ref is built here, and (c) what
the mathematics fixes (closed forms, exact integer arithmetic, brute force),
chosen so that a dropped term, a wrong sign or index, or a transposed operand
fails at least one check.
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest

POW3 = [3 ** i for i in range(97)]


def limb_value(b) -> int:
    """Balanced-ternary integer of a 16-byte limb, from the closed form u = 13 + t0 + 3t1 + 9t2."""
    v = 0
    for j, u in enumerate(np.asarray(b, np.uint8)):
        v += (int(u) - 13) * 27 ** j
    return v


def balanced_trits(v: int, n: int) -> list[int]:
    out = []
    for _ in range(n):
        r = v % 3
        if r == 2:
            r = -1
        out.append(r)
        v = (v - r) // 3
    assert v == 0
    return out


# ------------------------------------------------------------------- a1, a2 --
def test_tryte_code_closed_form_and_bijection(orc):
    seen = set()
    for t0, t1, t2 in itertools.product((-1, 0, 1), repeat=3):
        u = orc.tryte_of(t0, t1, t2)
        assert u == 13 + t0 + 3 * t1 + 9 * t2
        assert orc.trits_of(u) == (t0, t1, t2)
        seen.add(u)
    assert seen == set(range(27))
    assert orc.tryte_of(0, 0, 0) == 13  # ZERO_TRYTE, limb.hpp:39


def test_limb_encoding_matches_reference_from_trits(orc, golden):
    # limb::from_trits (limb.hpp:145-158) as compiled from the reference
    trits = golden["ft_trits"]
    packed = orc.pack_trits_rows(trits)  # one 48-trit row = one limb
    np.testing.assert_array_equal(packed[:, 0, :], golden["ft_bytes"])


# ----------------------------------------------------------------------- a3 --
THR = np.float32(0.45)


@pytest.mark.parametrize("mode", [0, 1])
def test_quantize_boundaries(orc, mode):
    up = np.nextafter(THR, np.float32(2))
    dn = np.nextafter(THR, np.float32(-2))
    cases = {
        float(THR): 1, float(up): 1, float(dn): 0, -float(THR): -1, -float(up): -1,
        -float(dn): 0, 0.0: 0, -0.0: 0, 1.0: 1, -1.0: -1, 7.5: 1, -7.5: -1,
        math.inf: 1, -math.inf: -1, math.nan: 0,
    }
    for v, want in cases.items():
        assert orc.quantize_trit(v, float(THR), mode) == want, (v, mode)


def test_torch_form_threshold_and_compare_dtype(orc):
    """t81/torch/__init__.py:44-50 executed with torch itself on boundary values: the
    float32 compare (Python scalar promoted to the tensor dtype), the [0, 0.9999]
    clamp, and '-1 wins' at threshold 0 -- all must match the oracle's torch form."""
    torch = pytest.importorskip("torch")

    def torch_quantize(t, threshold):
        threshold = float(max(0.0, min(threshold, 0.9999)))
        clipped = t.clamp(-1.0, 1.0)
        trits = torch.zeros_like(clipped, dtype=torch.int8)
        trits[clipped >= threshold] = 1
        trits[clipped <= -threshold] = -1
        return trits

    for thr in (0.45, 0.5, 0.0, 1.0, 0.99995, 0.3, 1e-7):
        t32 = np.float32(orc.torch_threshold(thr))
        vals = np.array([t32, np.nextafter(t32, 2), np.nextafter(t32, -2), -t32,
                         np.nextafter(-t32, 2), np.nextafter(-t32, -2), 0.0, -0.0, 1.0, -1.0,
                         0.45, 0.44999999, 0.4500001, 2.0, -2.0, np.inf, -np.inf, np.nan],
                        np.float32)
        want = torch_quantize(torch.from_numpy(vals), thr).numpy()
        got = np.array([orc.quantize_trit(float(v), float(t32), 1) for v in vals], np.int8)
        np.testing.assert_array_equal(got, want, err_msg=f"thr={thr}")
    # float32 compare: 0.45f >= 0.45 (double) would be False
    assert orc.quantize_trit(float(np.float32(0.45)), orc.torch_threshold(0.45), 1) == 1


# ---------------------------------------------------------------- a4, a5, a6 --
def brute_pack_rows(w: np.ndarray, thr: float) -> np.ndarray:
    rows, cols = w.shape
    L = -(-cols // 48)
    out = np.zeros((rows, L, 16), np.uint8)
    for r in range(rows):
        for c_l in range(L):
            for j in range(16):
                u = 0
                for p in range(3):
                    c = 48 * c_l + 3 * j + p
                    t = 0
                    if c < cols:
                        v = np.float32(w[r, c])
                        t = 1 if v >= np.float32(thr) else (-1 if v <= -np.float32(thr) else 0)
                    u += (t + 1) * 3 ** p  # base-3 digit form of the tryte
                out[r, c_l, j] = u
    return out


@pytest.mark.parametrize("cols", [1, 47, 48, 49, 100])
def test_pack_rows_brute_force(orc, cols):
    rng = np.random.default_rng(cols)
    w = rng.standard_normal((3, cols)).astype(np.float32)
    np.testing.assert_array_equal(orc.pack_rows(w, 0.45), brute_pack_rows(w, 0.45))
    # padding: trits past cols are 0 -> byte 13 when the whole triple is padding
    L = -(-cols // 48)
    if cols % 48:
        full_pad_from = (cols + 2) // 3
        assert (orc.pack_rows(w, 0.45)[:, L - 1, full_pad_from - 16 * (L - 1):] == 13).all()


def test_pack_rows_config2_statistics(orc):
    """Config 2 recipe: N(0, 0.02) + 1% outliers x10 at 0.45 -> only outliers survive."""
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((64, 3072)) * 0.02).astype(np.float32)
    mask = rng.random(w.shape) < 0.01
    w[mask] *= 10
    p = orc.pack_rows(w, 0.45)
    t = orc.unpack(p, 64, 3072)
    np.testing.assert_array_equal(t, np.where(w >= np.float32(0.45), 1,
                                              np.where(w <= -np.float32(0.45), -1, 0)))
    assert t.any()


def test_pack_cols_is_transposed_row_pack(orc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((7, 130)).astype(np.float32)
    cols = orc.pack_cols(x, 0.5, 1)                 # (L, tokens, 16)
    rows = orc.pack_rows(x, 0.5, 1)                 # (tokens, L, 16)
    np.testing.assert_array_equal(cols, rows.transpose(1, 0, 2))


def test_unpack_round_trip_and_errors(orc):
    rng = np.random.default_rng(2)
    w = rng.standard_normal((5, 97)).astype(np.float32)
    p = orc.pack_rows(w, 0.5)
    t = orc.unpack(p, 5, 97)
    np.testing.assert_array_equal(t, np.where(w >= 0.5, 1, np.where(w <= -0.5, -1, 0)))
    with pytest.raises(ValueError):
        orc.unpack(p, 5, 3 * 48 + 1)   # cols beyond capacity
    bad = p.copy()
    bad[0, 0, 0] = 27
    with pytest.raises(ValueError):
        orc.unpack(bad, 5, 97)


# ------------------------------------------------------------------ a10, a11 --
def test_mul_wide_golden_and_exact(orc, golden):
    a, b = golden["mw_a"], golden["mw_b"]
    for i in range(len(a)):
        lo, hi = orc.mul_wide(a[i], b[i])
        np.testing.assert_array_equal(lo, golden["mw_lo"][i])
        np.testing.assert_array_equal(hi, golden["mw_hi"][i])
        if i % 7 == 0:  # exact integer identity: V(lo) + V(hi) * 3^48 == V(a) * V(b)
            assert limb_value(lo) + limb_value(hi) * 3 ** 48 == limb_value(a[i]) * limb_value(b[i])
            assert abs(limb_value(lo)) <= (3 ** 48 - 1) // 2


def test_tryte_table_and_limb_to_double(orc, golden):
    t = orc.tryte_table()
    np.testing.assert_array_equal(t.view(np.uint64), golden["table"].view(np.uint64))
    # exact where 27^p and its multiples fit in 53 bits
    for p in range(11):
        for u in range(27):
            assert t[p, u] == (u - 13) * 27 ** p
    a = golden["mw_a"][9]
    assert orc.limb_to_double(a) == float(sum(t[p, a[p]] for p in range(16)))  # sequential order


def test_multiply_to_double_golden(orc, golden):
    a, b, want = golden["mw_a"], golden["mw_b"], golden["mw_prod"]
    got = np.array([orc.multiply_to_double(a[i], b[i]) for i in range(len(a))])
    np.testing.assert_array_equal(got.view(np.uint64), want.view(np.uint64))


def test_gemm_limb_golden(orc, golden):
    for i, name in enumerate(golden["g_names"]):
        M, N, K = (int(v) for v in golden[f"g{i}_shape"])
        al, be = (float(v) for v in golden[f"g{i}_ab"])
        got = orc.gemm_limb(golden[f"g{i}_A"], golden[f"g{i}_B"], golden[f"g{i}_C"], M, N, K,
                            al, be)
        np.testing.assert_array_equal(got.view(np.uint32), golden[f"g{i}_out"].view(np.uint32),
                                      err_msg=str(name))


def test_gemm_limb_reference_known_answers(orc):
    """tests/python/test_bindings.py:16-38: zero limbs give 0; alpha=0, beta=0.5 on C=2 gives 1."""
    A = np.full((2, 1, 16), 13, np.uint8)
    B = np.full((1, 3, 16), 13, np.uint8)
    assert (orc.gemm_limb(A, B, np.zeros((2, 3), np.float32), 2, 3, 48) == 0).all()
    assert (orc.gemm_limb(A, B, np.full((2, 3), 2.0, np.float32), 2, 3, 48, 0.0, 0.5) == 1.0).all()
    with pytest.raises(ValueError):
        orc.gemm_limb(A, B, np.zeros((2, 3), np.float32), 2, 3, 47)


def test_gemm_limb_single_trit_limbs_reduce_to_integer_gemm(orc):
    """Limbs whose only nonzero trit is trit 0 have V in {-1, 0, 1}: the limb GEMM is then an
    exact integer GEMM of those values (a transposed operand or dropped term fails it)."""
    rng = np.random.default_rng(11)
    M, N, KL = 6, 5, 4
    ta = rng.integers(-1, 2, (M, KL))
    tb = rng.integers(-1, 2, (KL, N))
    A = np.full((M, KL, 16), 13, np.uint8)
    B = np.full((KL, N, 16), 13, np.uint8)
    A[..., 0] = 13 + ta
    B[..., 0] = 13 + tb
    C = rng.standard_normal((M, N)).astype(np.float32)
    got = orc.gemm_limb(A, B, C, M, N, KL * 48, 2.0, 0.5)
    want = (2.0 * (ta @ tb) + 0.5 * C.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(got, want)


@pytest.mark.skipif("not __import__('oracle').ref()", reason="oracle/_ref not built here")
def test_gemm_limb_matches_compiled_reference_live(orc):
    ref = orc.ref()
    rng = np.random.default_rng(3)
    for M, N, KL, nz in ((8, 8, 2, 16), (5, 11, 3, 4), (1, 17, 5, 7)):
        A = np.full((M, KL, 16), 13, np.uint8)
        B = np.full((KL, N, 16), 13, np.uint8)
        A[..., :nz] = rng.integers(0, 27, (M, KL, nz))
        B[..., :nz] = rng.integers(0, 27, (KL, N, nz))
        C = rng.standard_normal((M, N)).astype(np.float32)
        want = ref.gemm_ternary(A, B, C, M, N, KL * 48, 0.3, -1.5)
        got = orc.gemm_limb(A, B, C, M, N, KL * 48, 0.3, -1.5)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------ trit-dot oracle --
def test_trit_matmul_against_reference_embedding(orc, golden):
    """The compiled reference gemm_ternary on one-value-per-limb embeddings computes
    sum_k X[m,k] T[n,k] exactly; the trit-dot oracle must agree with it."""
    T, X = golden["emb_T"], golden["emb_X"]
    packed = orc.pack_trits_rows(T)
    got = orc.trit_matmul_i64(X, packed, T.shape[1])          # (M, N)
    np.testing.assert_array_equal(got.T.astype(np.float32), golden["emb_out"])


def test_trit_matmul_against_numpy(orc):
    rng = np.random.default_rng(9)
    M, N, K = 4, 9, 101
    T = rng.integers(-1, 2, (N, K)).astype(np.int8)
    X = rng.standard_normal((M, K))
    packed = orc.pack_trits_rows(T)
    np.testing.assert_allclose(orc.trit_matmul_f64(X, packed, K), X @ T.T.astype(np.float64),
                               rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(orc.trit_matmul_abs_f64(X, packed, K),
                               np.abs(X) @ np.abs(T.T).astype(np.float64), rtol=1e-12)
    Xi = rng.integers(-128, 128, (M, K)).astype(np.int8)
    np.testing.assert_array_equal(orc.trit_matmul_i64(Xi, packed, K),
                                  Xi.astype(np.int64) @ T.T.astype(np.int64))


def _same_or_both_nan(got: np.ndarray, want: np.ndarray) -> bool:
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    nan = np.isnan(want)
    return bool(np.array_equal(np.isnan(got), nan)
                and np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)))


EW_CASES = (("where", {}), ("clamp", dict(p0=-0.75, p1=1.25)), ("lerp", {}),
            ("addcmul", dict(p0=0.3)))


def test_elementwise_golden(orc, golden):
    """where / clamp / lerp / addcmul equal the reference's CPU loops bit for bit
    (src/linalg/gemm_dispatch.cpp:145-211, vectors from the compiled reference)."""
    a, b, c = golden["ew_a"], golden["ew_b"], golden["ew_c"]
    for op, kw in EW_CASES:
        got = orc.elementwise(op, a, b, c, **kw)
        assert _same_or_both_nan(got, golden["ew_" + op]), op


def test_elementwise_closed_forms(orc):
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    x = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    y = np.array([-1.0, -2.0, -3.0, -4.0], np.float32)
    cond = np.array([nan, -0.0, 0.0, 5.0], np.float32)
    # a NaN condition is "!= 0" (takes x); -0.0 and 0.0 take y
    np.testing.assert_array_equal(orc.elementwise("where", cond, x, y), [1.0, -2.0, -3.0, 4.0])
    v = np.array([nan, -inf, inf, -0.75, 1.25, 0.5, -0.0], np.float32)
    got = orc.elementwise("clamp", v, p0=-0.75, p1=1.25)
    assert np.isnan(got[0]) and list(got[1:]) == [-0.75, 1.25, -0.75, 1.25, 0.5, 0.0]
    s = np.array([1.5, -2.0, 1e30], np.float32)
    e = np.array([7.0, 3.0, -1e30], np.float32)
    np.testing.assert_array_equal(orc.elementwise("lerp", s, e, np.zeros(3, np.float32)), s)
    # separate roundings: 0.1f * 3.0f rounds before the add (an FMA would round once)
    t1 = np.array([0.1], np.float32)
    t2 = np.array([3.0], np.float32)
    want = np.float32(np.float32(np.float32(0.7) * t1[0]) * t2[0])
    got = orc.elementwise("addcmul", np.zeros(1, np.float32), t1, t2, p0=0.7)
    assert got[0] == want


@pytest.mark.skipif("not __import__('oracle').ref()", reason="oracle/_ref not built here")
def test_elementwise_matches_compiled_reference_live(orc):
    ref = orc.ref()
    rng = np.random.default_rng(12)
    a, b, c = (rng.standard_normal(1001).astype(np.float32) for _ in range(3))
    a[::5] = 0.0
    for op, kw in EW_CASES:
        assert _same_or_both_nan(orc.elementwise(op, a, b, c, **kw),
                                 ref.elementwise(op, a, b, c, **kw)), op


def _spmm_case(z, i):
    rows, cols, N = (int(d) for d in z[f"sp{i}_dims"])
    alpha, beta = (float(a) for a in z[f"sp{i}_ab"])
    return (z[f"sp{i}_values"], z[f"sp{i}_rows"], z[f"sp{i}_cols"], rows, cols, z[f"sp{i}_B"],
            z[f"sp{i}_C"], N, alpha, beta)


def test_spmm_golden(orc, golden):
    """spmm_simple equals the compiled reference (include/t81/sparse/simple.hpp:37-94) bit
    for bit on every fixture case, NaN payloads and the state of C on a throw included."""
    for i, name in enumerate(golden["sp_names"]):
        rc, out = orc.spmm_simple(*_spmm_case(golden, i))
        assert rc == int(golden[f"sp{i}_rc"]), name
        np.testing.assert_array_equal(out.view(np.uint32), golden[f"sp{i}_out"].view(np.uint32),
                                      err_msg=str(name))


def test_spmm_closed_forms(orc):
    f32 = np.float32
    # list order with a float rounding after every entry: 1e8 + 1 rounds back to 1e8,
    # so the entries (1e8, 1, -1e8) give 0 while an exact or reordered sum gives 1
    B = np.array([[1e8], [1.0]], f32)
    rc, out = orc.spmm_simple([1, 1, -1], [0, 0, 0], [0, 1, 0], 1, 2, B, np.zeros((1, 1), f32), 1)
    assert rc == 0 and out[0, 0] == 0.0
    rc, out = orc.spmm_simple([1, -1, 1], [0, 0, 0], [0, 0, 1], 1, 2, B, np.zeros((1, 1), f32), 1)
    assert out[0, 0] == 1.0
    # the integer value becomes a double once, to nearest even: 2^53 + 1 -> 2^53
    rc, out = orc.spmm_simple([2**53 + 1], [0], [0], 1, 1, np.ones((1, 1), f32),
                              np.zeros((1, 1), f32), 1)
    assert out[0, 0] == f32(2.0**53)
    # beta == 0 zero-fills (NaN gone); beta != 0 scales through double
    C = np.array([[np.nan, 3.0]], f32)
    rc, out = orc.spmm_simple([], [], [], 1, 1, np.zeros((1, 2), f32), C, 2, 1.0, 0.0)
    assert list(out[0]) == [0.0, 0.0]
    rc, out = orc.spmm_simple([], [], [], 1, 1, np.zeros((1, 2), f32), C, 2, 1.0, 0.1)
    assert np.isnan(out[0, 0]) and out[0, 1] == f32(np.float64(f32(3.0)) * np.float64(f32(0.1)))
    # a dense small case equals the exact float64 product when nothing rounds
    g = np.random.default_rng(3)
    vals = g.integers(-3, 4, 30)
    ri, ci = g.integers(0, 4, 30), g.integers(0, 5, 30)
    Bi = g.integers(-8, 9, (5, 6)).astype(f32)
    dense = np.zeros((4, 5))
    np.add.at(dense, (ri, ci), vals)
    rc, out = orc.spmm_simple(vals, ri, ci, 4, 5, Bi, np.zeros((4, 6), f32), 6)
    np.testing.assert_array_equal(out, (dense @ Bi.astype(np.float64)).astype(f32))
    # an out-of-range index stops at that entry (-1), entries before it applied
    rc, out = orc.spmm_simple([2, 5], [0, 3], [0, 0], 1, 1, np.ones((1, 1), f32),
                              np.zeros((1, 1), f32), 1)
    assert rc == -1 and out[0, 0] == 2.0


@pytest.mark.skipif("not __import__('oracle').ref()", reason="oracle/_ref not built here")
def test_spmm_matches_compiled_reference_live(orc):
    ref = orc.ref()
    g = np.random.default_rng(77)
    for rows, cols, N, nnz, alpha, beta in ((40, 30, 17, 900, 0.3, -2.0), (1, 1, 1, 50, 1.0, 0.0),
                                            (300, 200, 8, 5000, -1.7, 1.0)):
        vals = g.integers(-2**63, 2**63 - 1, nnz, dtype=np.int64, endpoint=True)
        vals[::3] = g.integers(-1, 2, vals[::3].size)
        ri = g.integers(0, rows, nnz).astype(np.int32)
        ci = g.integers(0, cols, nnz).astype(np.int32)
        B = (g.standard_normal((cols, N)) * 1e-17).astype(np.float32)
        C = g.standard_normal((rows, N)).astype(np.float32)
        got = orc.spmm_simple(vals, ri, ci, rows, cols, B, C, N, alpha, beta)
        want = ref.spmm_simple(vals, ri, ci, rows, cols, B, C, N, alpha, beta)
        assert got[0] == want[0]
        np.testing.assert_array_equal(got[1].view(np.uint32), want[1].view(np.uint32))

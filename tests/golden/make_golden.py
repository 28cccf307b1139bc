"""Writes tests/golden/ref_vectors.npz from the reference's own compiled CPU path.

Run in a container that has /root/reference (``make -C oracle ref`` builds
oracle/_ref/libt81ref_*.so from the reference sources).  The fixture holds
inputs and the outputs the reference code produced for them; it is data, not
source.  Vectors:

* ``table``                  16x27 tryte contributions (include/t81/linalg/gemm.hpp:28-41)
* ``mw_a``/``mw_b``/``mw_lo``/``mw_hi``/``mw_prod``
                             limb::mul_wide and multiply_to_double on the inputs of
                             tests/unit/test_limb_basic.cpp:68-116 (9 fixed limbs, all
                             pairs; 1000 random pairs, mt19937_64(0xdeadbeef))
* ``ft_trits``/``ft_bytes``  limb::from_trits on random trit vectors (the tryte code)
* ``g<i>_*``                 gemm_ternary_cpu_impl (src/linalg/gemm_cpu.cpp:8-71) cases
* ``emb_*``                  gemm_ternary on one-value-per-limb embeddings: small integers
                             as limbs, which turns the limb GEMM into an exact integer GEMM
                             (the cross-check of the trit-dot oracle)
* ``ew_*``                   where / clamp / lerp / addcmul on Backend::CPU
                             (src/linalg/gemm_dispatch.cpp:145-211) over float32 arrays
                             with NaN, +-inf, -0.0, denormals and zeros mixed in
* ``sp<i>_*``                t81::sparse::spmm_simple (include/t81/sparse/simple.hpp:37-94)
                             on limbs built from long long as its binding does: the
                             examples/ternary_sparse_preview.py shape, unsorted rows with
                             repeated entries, int64 values near +-2^63, NaN / inf /
                             denormal operands, beta == 0 over NaN, and out-of-range
                             indices (``_rc`` -1: C as the reference leaves it on throw)

and tests/golden/tq1_row_vectors.npz (``tq1_main``), the TQ1_0 row codec of
src/t81/core/gguf_quants.h compiled as it stands:

* ``q_*``   quantize_row_tq1_0 on ragged rows with NaN / +-inf / -0.0 / denormal values,
            values at +-threshold * scale and one ulp either side, thresholds outside
            [0, 0.9999] and NaN, supplied scales 0 / negative / NaN / inf / denormal; the
            returned scale follows the binding (python/bindings.cpp:531-539)
* ``d_*``   dequantize_row_tq1_0: the trits of every word 0 .. 65535 (the low 8 base-3
            digits of an out-of-range word), and 2048 words at scales 0, -0, +-1.5,
            +-inf, NaN, denormal, 3e38
* ``h_*``   half_to_float on all 65536 half patterns
* ``p_*``   tensor payloads (groups of block_rows rows: a half scale, 8 reserved bytes for
            the TQ2_0 variant, the rows' words) decoded row by row with the compiled
            dequantize_row_tq1_0 and half_to_float; the framing and its truncation checks
            follow python/bindings.cpp:561-638 (that file needs pybind11 and is not built
            here), ``p_rc`` naming the first failing check (1 scale, 2 reserved bytes,
            3 rows) of payloads cut short
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402


def spmm_cases():
    """(name, values, row_idx, col_idx, rows, cols, B, C, N, alpha, beta) for spmm_simple."""
    g = np.random.default_rng(2024)
    f32 = np.float32
    cases = []
    # examples/ternary_sparse_preview.py:8-40 (256 x 256, 3 % density, values in [-3, 3]
    # without 0), with 32 features instead of 128 to keep the fixture small
    nnz = int(256 * 256 * 0.03)
    v = g.integers(-3, 4, nnz).astype(np.int64)
    v[v == 0] = 1
    cases.append(("example", v, g.integers(0, 256, nnz).astype(np.int32),
                  g.integers(0, 256, nnz).astype(np.int32), 256, 256,
                  g.standard_normal((256, 32)).astype(f32), np.zeros((256, 32), f32), 32, 1.0, 0.0))
    # unsorted rows, many entries per row, int64 values whose double rounding matters
    rows, cols, N, nnz = 9, 7, 33, 400
    v = g.integers(-2**62, 2**62, nnz, dtype=np.int64)
    v[:6] = [2**63 - 1, -2**63, 2**53 + 1, -(2**53 + 1), 0, 1]
    v[6:40] = g.integers(-5, 6, 34)
    B = (g.standard_normal((cols, N)) * 1e-19).astype(f32)
    B.reshape(-1)[:8] = [np.inf, -np.inf, np.nan, -0.0, 1e-45, -3e-39, 3e38, 0.0]
    C = g.standard_normal((rows, N)).astype(f32)
    C.reshape(-1)[:4] = [np.nan, np.inf, -1e-40, -0.0]
    cases.append(("order_int64", v, g.integers(0, rows, nnz).astype(np.int32),
                  g.integers(0, cols, nnz).astype(np.int32), rows, cols, B, C, N, 0.7, -1.3))
    # beta == 0 replaces C (NaN included) by zeros before the entries
    cases.append(("beta0_nan", g.integers(-3, 4, 12).astype(np.int64),
                  g.integers(0, 5, 12).astype(np.int32), g.integers(0, 6, 12).astype(np.int32),
                  5, 6, g.standard_normal((6, 3)).astype(f32), np.full((5, 3), np.nan, f32), 3,
                  -2.5, 0.0))
    # alpha == 0 against an infinite B: 0 * inf = NaN in the touched rows
    Binf = np.ones((4, 2), f32)
    Binf[1, 0] = np.inf
    cases.append(("alpha0_inf", np.array([1, -1, 3], np.int64), np.array([0, 2, 2], np.int32),
                  np.array([1, 0, 1], np.int32), 3, 4, Binf, np.ones((3, 2), f32), 2, 0.0, 2.0))
    # out-of-range row at entry 7 and column at entry 0: C as left at the throw
    ri = g.integers(0, 6, 20).astype(np.int32)
    ci = g.integers(0, 5, 20).astype(np.int32)
    ri[7] = 6
    cases.append(("bad_row", g.integers(-4, 5, 20).astype(np.int64), ri, ci, 6, 5,
                  g.standard_normal((5, 4)).astype(f32), g.standard_normal((6, 4)).astype(f32), 4,
                  1.5, 0.5))
    ci2 = ci.copy()
    ci2[0] = -1
    cases.append(("bad_col", g.integers(-4, 5, 20).astype(np.int64), ri.copy(), ci2, 7, 5,
                  g.standard_normal((5, 4)).astype(f32), g.standard_normal((7, 4)).astype(f32), 4,
                  1.0, -0.25))
    cases.append(("empty", np.zeros(0, np.int64), np.zeros(0, np.int32), np.zeros(0, np.int32),
                  4, 3, g.standard_normal((3, 5)).astype(f32), g.standard_normal((4, 5)).astype(f32),
                  5, 1.0, 0.5))
    return cases


def main() -> None:
    oracle.build(reference=True)
    ref = oracle.ref("generic")
    if ref is None:
        raise SystemExit("oracle/_ref/libt81ref_generic.so is not built (needs /root/reference)")
    out: dict[str, np.ndarray] = {}
    out["table"] = ref.tryte_table()

    # test_limb_basic.cpp:68-78 fixed values, then its seeded random limbs
    lo_min, hi_max = ref.limb_min_max()
    fixed = [ref.limb_from_value(v) for v in (0, 1, -1, 42, -42, 1234, -1234)]
    fixed += [lo_min, hi_max]
    a_list, b_list = [], []
    for x in fixed:
        for y in fixed:
            a_list.append(x)
            b_list.append(y)
    rnd = ref.random_limbs(0xDEADBEEF, 2000)
    a_list += [rnd[2 * i] for i in range(1000)]
    b_list += [rnd[2 * i + 1] for i in range(1000)]
    mw_a = np.stack(a_list).astype(np.uint8)
    mw_b = np.stack(b_list).astype(np.uint8)
    lo = np.empty_like(mw_a)
    hi = np.empty_like(mw_a)
    prod = np.empty(len(mw_a), np.float64)
    for i in range(len(mw_a)):
        lo[i], hi[i] = ref.mul_wide(mw_a[i], mw_b[i])
        prod[i] = ref.multiply_to_double(mw_a[i], mw_b[i])
    out.update(mw_a=mw_a, mw_b=mw_b, mw_lo=lo, mw_hi=hi, mw_prod=prod)

    rng = np.random.default_rng(81)
    ft_trits = rng.integers(-1, 2, size=(256, 48), dtype=np.int8)
    ft_trits[0] = 0
    ft_trits[1] = 1
    ft_trits[2] = -1
    out["ft_trits"] = ft_trits
    out["ft_bytes"] = np.stack([ref.limb_from_trits(t) for t in ft_trits])

    cases = []
    # the two known-answer cases of tests/python/test_bindings.py:16-38
    cases.append(("zero", np.full((2, 1, 16), 13, np.uint8), np.full((1, 3, 16), 13, np.uint8),
                  np.zeros((2, 3), np.float32), 2, 3, 48, 1.0, 0.0))
    cases.append(("beta", np.full((2, 1, 16), 13, np.uint8), np.full((1, 3, 16), 13, np.uint8),
                  np.full((2, 3), 2.0, np.float32), 2, 3, 48, 0.0, 0.5))
    # full-range limbs: products overflow float32 -> +-inf (double sums stay finite)
    M, N, KL = 9, 13, 3
    cases.append(("full", rng.integers(0, 27, (M, KL, 16), dtype=np.uint8),
                  rng.integers(0, 27, (KL, N, 16), dtype=np.uint8),
                  rng.standard_normal((M, N)).astype(np.float32), M, N, KL * 48, 0.5, 1.0))
    # low trytes only: finite, rounding-sensitive outputs
    for nz, alpha, beta in ((3, 1.0, 0.0), (5, 0.37, -0.7), (8, -1.25, 2.0), (11, 3.0, 0.0)):
        A = np.full((M, KL, 16), 13, np.uint8)
        B = np.full((KL, N, 16), 13, np.uint8)
        A[..., :nz] = rng.integers(0, 27, (M, KL, nz))
        B[..., :nz] = rng.integers(0, 27, (KL, N, nz))
        cases.append((f"low{nz}", A, B, rng.standard_normal((M, N)).astype(np.float32), M, N,
                      KL * 48, alpha, beta))
    # NaN in C with beta = 0 still propagates (accum = C * beta, gemm_cpu.cpp:37-38)
    C = np.zeros((M, N), np.float32)
    C[0, 0] = np.nan
    A = np.full((M, 1, 16), 13, np.uint8)
    A[..., 0] = rng.integers(0, 27, (M, 1))
    B = np.full((1, N, 16), 13, np.uint8)
    B[..., 0] = rng.integers(0, 27, (1, N))
    cases.append(("nan", A, B, C, M, N, 48, 1.0, 0.0))
    for i, (name, A, B, C, M_, N_, K_, al, be) in enumerate(cases):
        out[f"g{i}_A"] = A
        out[f"g{i}_B"] = B
        out[f"g{i}_C"] = C
        out[f"g{i}_shape"] = np.array([M_, N_, K_], np.int64)
        out[f"g{i}_ab"] = np.array([al, be], np.float32)
        out[f"g{i}_out"] = ref.gemm_ternary(A, B, C, M_, N_, K_, al, be)
    out["g_names"] = np.array([c[0] for c in cases])

    # one value per limb: T (N x K) trits and X (M x K) int8 -> sum_k X[m,k] T[n,k]
    Mx, Nx, Kx = 5, 7, 37
    T = rng.integers(-1, 2, (Nx, Kx), dtype=np.int8)
    X = rng.integers(-128, 128, (Mx, Kx)).astype(np.int8)
    A = np.stack([[ref.limb_from_value(int(v)) for v in row] for row in T])          # (N, K)
    B = np.stack([[ref.limb_from_value(int(v)) for v in col] for col in X.T])        # (K, M)
    emb = ref.gemm_ternary(A, B, np.zeros((Nx, Mx), np.float32), Nx, Mx, Kx * 48)
    out.update(emb_T=T, emb_X=X, emb_out=emb)

    path = os.path.join(HERE, "ref_vectors.npz")
    # elementwise ops of the backend contract
    ew = np.random.default_rng(11)
    n = 257
    a, b, c = (ew.standard_normal(n).astype(np.float32) * 2 for _ in range(3))
    specials = np.array([np.nan, np.inf, -np.inf, -0.0, 0.0, 1e-45, 3e38, -3e38, 1.0, -1.0],
                        np.float32)
    for arr, shift in ((a, 0), (b, 3), (c, 7)):
        arr[: specials.size] = np.roll(specials, shift)
    a[20:60:3] = 0.0
    out.update(ew_a=a, ew_b=b, ew_c=c,
               ew_where=ref.elementwise("where", a, b, c),
               ew_clamp=ref.elementwise("clamp", a, p0=-0.75, p1=1.25),
               ew_lerp=ref.elementwise("lerp", a, b, c),
               ew_addcmul=ref.elementwise("addcmul", a, b, c, p0=0.3))
    for i, case in enumerate(spmm_cases()):
        name, values, ri, ci, rows, cols, B, C, N, al, be = case
        rc, res = ref.spmm_simple(values, ri, ci, rows, cols, B, C, N, al, be)
        out.update({f"sp{i}_values": values, f"sp{i}_rows": ri, f"sp{i}_cols": ci,
                    f"sp{i}_dims": np.array([rows, cols, N], np.int64),
                    f"sp{i}_ab": np.array([al, be], np.float32), f"sp{i}_B": B, f"sp{i}_C": C,
                    f"sp{i}_out": res, f"sp{i}_rc": np.array(rc, np.int64)})
    out["sp_names"] = np.array([c[0] for c in spmm_cases()])
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, SIMD path {ref.simd_path()})")


def tq1_quantize_cases():
    """(threshold, scale, values) for quantize_row_tq1_0."""
    g = np.random.default_rng(1081)
    f32 = np.float32
    cases = []
    for n in (1, 7, 8, 9, 15, 16, 17, 33, 100, 257, 1000):
        cases.append((0.45, 0.0, g.standard_normal(n).astype(f32)))
    v = g.standard_normal(64).astype(f32)
    for thr in (0.5, 0.0, -0.3, -0.0, 0.9999, 1.0, 1.5, np.nan, 1e-8, 0.45000002):
        cases.append((thr, 0.0, v))
    for sc in (-1.0, 2.5, np.nan, np.inf, 1e-40, 1e-30, 0.37):
        cases.append((0.45, sc, v))
    # values at +-threshold (scale 1) and one ulp either side
    t = f32(0.45)
    edge = np.array([t, -t, np.nextafter(t, f32(1)), np.nextafter(t, f32(0)),
                     -np.nextafter(t, f32(1)), -np.nextafter(t, f32(0)), 1.0, -1.0,
                     1.5, -7.0, 0.0, -0.0], f32)
    cases.append((0.45, 1.0, edge))
    cases.append((0.45, 0.0, np.concatenate([edge, np.array([1.0], f32)])))
    sp = np.array([np.nan, np.inf, -np.inf, -0.0, 0.0, 1e-45, -1e-40, 3e38, -3e38, 0.5, -0.5,
                   np.nan, 2.0, -2.0, 1e-38, 0.25, 0.75], f32)
    for sc in (0.0, 1.0, np.inf):
        cases.append((0.45, sc, sp))
    cases.append((0.45, 0.0, np.array([np.nan, np.nan, 0.0, -0.0], f32)))   # scale 0
    cases.append((0.45, 0.0, np.zeros(20, f32)))
    cases.append((0.45, 0.0, np.array([1e-42, -3e-43, 0.0, 1e-44, -1e-42], f32)))  # denormal max
    cases.append((0.3, 0.0, (g.standard_normal(333) * 1e-3).astype(f32)))
    return cases


def tq1_main() -> None:
    ref = oracle.ref("generic")
    if ref is None:
        raise SystemExit("oracle/_ref/libt81ref_generic.so is not built (needs /root/reference)")
    out: dict[str, np.ndarray] = {}
    # quantize: values concatenated, offsets per case
    qs = tq1_quantize_cases()
    vals, offs, woffs, words, thr, sc, ret = [], [0], [0], [], [], [], []
    for t, s_, v in qs:
        w = ref.tq1_quantize_row(v, t, s_)
        s32 = np.float32(s_)
        ret.append(s32 if not s32 <= 0 else np.float32(ref.tq1_compute_scale(v)))
        vals.append(v)
        offs.append(offs[-1] + v.size)
        words.append(w)
        woffs.append(woffs[-1] + w.size)
        thr.append(t)
        sc.append(s_)
    out.update(q_values=np.concatenate(vals), q_offsets=np.array(offs, np.int64),
               q_words=np.concatenate(words), q_word_offsets=np.array(woffs, np.int64),
               q_threshold=np.array(thr, np.float32), q_scale=np.array(sc, np.float32),
               q_returned_scale=np.array(ret, np.float32))
    # dequantize: the trits of every word (scale 1), and a sample of words at each scale
    all_words = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    out["d_trits"] = ref.tq1_dequantize_row(all_words, 8 * 65536, 1.0).astype(np.int8)
    sample = np.concatenate([np.arange(1024), np.random.default_rng(1083).integers(
        1024, 65536, 1024)]).astype(np.uint16)
    scales = np.array([0.0, -0.0, 1.5, -1.5, np.inf, -np.inf, np.nan, 1e-42, 3e38], np.float32)
    out["d_words"] = sample
    out["d_scales"] = scales
    out["d_values"] = np.stack([ref.tq1_dequantize_row(sample, 8 * sample.size, float(s_))
                                for s_ in scales])
    ragged = []
    for n in (0, 1, 5, 8, 13, 100):
        ragged.append(ref.tq1_dequantize_row(all_words[:64], n, 1.25))
    out["d_ragged"] = np.concatenate(ragged)
    out["h_values"] = np.array([ref.tq1_half_to_float(h) for h in range(65536)], np.float32)
    # tensor payloads written with the row codec, decoded with the compiled row decoder
    g = np.random.default_rng(1082)
    pay, poffs, pmeta, pvals, pvoffs = [], [0], [], [], [0]
    for rows, cols, block_rows, refine in ((5, 13, 32, 0), (70, 100, 32, 1), (33, 8, 7, 0),
                                           (9, 1, 1, 1), (4, 17, 0, 0), (6, 40, -5, 1),
                                           (3, 24, 1000, 0), (0, 10, 32, 0), (4, 0, 2, 1),
                                           (40, 16, 32, 0)):
        m = g.standard_normal((rows, cols)).astype(np.float32)
        if rows > 3 and cols:
            m[3] *= 1e-9                                  # a tiny row in a big group
        buf = bytearray(oracle.tq1r_payload(m, block_rows, bool(refine)))
        group = max(1, block_rows)
        stride = 2 + 8 * refine + 2 * ((cols + 7) // 8) * group
        if rows >= 9 and len(buf) > stride:              # crafted scales: NaN, inf, subnormal
            for gi, h in enumerate((0x7E01, 0xFC00, 0x0003)):
                if gi * stride + 1 < len(buf):
                    buf[gi * stride:gi * stride + 2] = np.array([h], np.uint16).tobytes()
        want = np.zeros((rows, cols), np.float32)
        wpr = (cols + 7) // 8
        for r in range(rows):
            gi, i = divmod(r, group)
            o = gi * stride
            h = int(np.frombuffer(bytes(buf[o:o + 2]), np.uint16)[0])
            ro = o + 2 + 8 * refine + i * 2 * wpr
            wr = np.frombuffer(bytes(buf[ro:ro + 2 * wpr]), np.uint16)
            want[r] = ref.tq1_dequantize_row(wr, cols, float(ref.tq1_half_to_float(h)))
        pay.append(np.frombuffer(bytes(buf), np.uint8))
        poffs.append(poffs[-1] + len(buf))
        pmeta.append((rows, cols, block_rows, refine))
        pvals.append(want.reshape(-1))
        pvoffs.append(pvoffs[-1] + want.size)
    out.update(p_bytes=np.concatenate(pay), p_offsets=np.array(poffs, np.int64),
               p_meta=np.array(pmeta, np.int64), p_values=np.concatenate(pvals),
               p_value_offsets=np.array(pvoffs, np.int64))
    # truncated payloads: (case index, length) -> the first failing check
    cuts = []
    for ci, (rows, cols, block_rows, refine) in enumerate(pmeta):
        full = poffs[ci + 1] - poffs[ci]
        for cut in sorted({0, 1, 2, 3, 9, 10, 11, full // 2, full - 1}):
            if 0 <= cut < full:
                rc, _ = oracle.tq1r_dequant_tensor(bytes(pay[ci][:cut]), rows, cols, block_rows,
                                                   bool(refine))
                cuts.append((ci, cut, rc))
    out["p_cuts"] = np.array(cuts, np.int64)
    path = os.path.join(HERE, "tq1_row_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "tq1":
        tq1_main()
    else:
        main()
        tq1_main()

/*
 * oracle/t81_oracle.c -- CPU restatement of t81lib's packed-ternary path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT.  This file is the checker the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py may load liboracle.so; the t81lib_amd package never does.
 *
 * Written from the reference's behaviour, not copied from it.  Each function
 * names the reference lines it restates.  How each one is pinned (golden
 * vectors from the compiled reference in oracle/_ref, closed forms, brute
 * force) is listed in tests/test_oracle.py; nothing here is "parity unpinned"
 * except the binding-level error strings, which are not restated here.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off: the fp64 sums below are
 * evaluated as separate multiply and add roundings, the contraction mode of
 * the reference's pybind11 build, which compiles gemm_cpu.cpp for plain
 * x86-64 without FMA: python/CMakeLists.txt:22-30).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define TRITS 48
#define TRYTES 16

/* ---------------------------------------------------------------- a1 ----
 * Tryte code.  include/t81/core/detail/lut.hpp:13-49 enumerates the 27
 * triples and stores tryte = 13 + t0 + 3*t1 + 9*t2; since 13 = 1 + 3 + 9 the
 * base-3 digits of the tryte are exactly t_i + 1. */
static inline uint8_t tryte_of(int t0, int t1, int t2) {
    return (uint8_t)(13 + t0 + 3 * t1 + 9 * t2);
}

static inline void trits_of(uint8_t u, int8_t *t) {
    t[0] = (int8_t)(u % 3) - 1;
    t[1] = (int8_t)((u / 3) % 3) - 1;
    t[2] = (int8_t)(u / 9) - 1;
}

uint8_t orc_tryte_of(int t0, int t1, int t2) { return tryte_of(t0, t1, t2); }

void orc_trits_of(uint8_t u, int8_t *out3) { trits_of(u, out3); }

/* ---------------------------------------------------------------- a3 ----
 * quantize_trit.
 *  mode 0: python/bindings.cpp:405-414 -- std::clamp(v,-1,1) (NaN passes
 *          through), then ">= thr -> +1, else <= -thr -> -1, else 0".
 *  mode 1: t81/torch/__init__.py:44-50 -- clamp, zero-init, "[c >= thr] = 1"
 *          then "[c <= -thr] = -1", so -1 wins when both hold.  The compares
 *          run in float32 (torch promotes the Python scalar to the tensor
 *          dtype); orc_torch_threshold gives that float32 threshold.
 */
static inline float clamp_pm1(float v) {
    /* std::clamp(v, lo, hi) == (v < lo) ? lo : (hi < v) ? hi : v */
    return (v < -1.0f) ? -1.0f : ((1.0f < v) ? 1.0f : v);
}

int8_t orc_quantize_trit(float v, float thr, int mode) {
    const float c = clamp_pm1(v);
    if (mode == 0) {
        if (c >= thr) return 1;
        if (c <= -thr) return -1;
        return 0;
    }
    int8_t t = 0;
    if (c >= thr) t = 1;
    if (c <= -thr) t = -1;
    return t;
}

/* t81/torch/__init__.py:45 -- float(max(0.0, min(threshold, 0.9999))) in
 * Python double arithmetic, then the float32 rounding the compare applies. */
float orc_torch_threshold(double thr) {
    const double lo = (0.9999 < thr) ? 0.9999 : thr; /* min(thr, 0.9999) */
    const double cl = (lo > 0.0) ? lo : 0.0;         /* max(0.0, lo)     */
    return (float)cl;
}

/* ---------------------------------------------------------------- a4 ----
 * Row-wise packer.  python/bindings.cpp:460-517 (pack_dense_matrix) and
 * t81/torch/__init__.py:68-80 (_pack_rowwise): out is (rows, L, 16) with
 * L = ceil(cols/48); byte j of limb l of row r holds the trits of columns
 * 48l+3j .. 48l+3j+2 (little-endian trytes, limb.hpp:145-158); columns past
 * `cols` are trit 0. */
void orc_pack_rows(const float *w, int64_t rows, int64_t cols, float thr, int mode,
                   uint8_t *out) {
    const int64_t L = (cols + TRITS - 1) / TRITS;
    for (int64_t r = 0; r < rows; ++r) {
        const float *src = w + r * cols;
        for (int64_t l = 0; l < L; ++l) {
            uint8_t *dst = out + (r * L + l) * TRYTES;
            for (int j = 0; j < TRYTES; ++j) {
                int t[3];
                for (int p = 0; p < 3; ++p) {
                    const int64_t c = l * TRITS + 3 * j + p;
                    t[p] = (c < cols) ? orc_quantize_trit(src[c], thr, mode) : 0;
                }
                dst[j] = tryte_of(t[0], t[1], t[2]);
            }
        }
    }
}

/* Packs already-quantized trits (int8 in -1..1) row-wise; same layout. */
void orc_pack_trits_rows(const int8_t *t, int64_t rows, int64_t cols, uint8_t *out) {
    const int64_t L = (cols + TRITS - 1) / TRITS;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t l = 0; l < L; ++l) {
            uint8_t *dst = out + (r * L + l) * TRYTES;
            for (int j = 0; j < TRYTES; ++j) {
                int v[3];
                for (int p = 0; p < 3; ++p) {
                    const int64_t c = l * TRITS + 3 * j + p;
                    v[p] = (c < cols) ? t[r * cols + c] : 0;
                }
                dst[j] = tryte_of(v[0], v[1], v[2]);
            }
        }
    }
}

/* ---------------------------------------------------------------- a5 ----
 * Column-wise packer for activations.  t81/torch/__init__.py:257-262 and
 * :83-97: the (tokens x K) input is transposed to (K x tokens), quantized,
 * and limb l of column n lands at out[(l*tokens + n)*16]. */
void orc_pack_cols(const float *x, int64_t tokens, int64_t k, float thr, int mode,
                   uint8_t *out) {
    const int64_t L = (k + TRITS - 1) / TRITS;
    for (int64_t l = 0; l < L; ++l) {
        for (int64_t n = 0; n < tokens; ++n) {
            uint8_t *dst = out + (l * tokens + n) * TRYTES;
            for (int j = 0; j < TRYTES; ++j) {
                int t[3];
                for (int p = 0; p < 3; ++p) {
                    const int64_t c = l * TRITS + 3 * j + p;
                    t[p] = (c < k) ? orc_quantize_trit(x[n * k + c], thr, mode) : 0;
                }
                dst[j] = tryte_of(t[0], t[1], t[2]);
            }
        }
    }
}

/* ---------------------------------------------------------------- a6 ----
 * unpack_packed_limbs, python/bindings.cpp:640-686: rejects a byte > 26
 * (limb::from_bytes, limb.hpp:160-168) and cols > 48*L; returns trits of the
 * first `cols` columns.  Returns 0, -1 (cols too large) or -2 (bad byte). */
int orc_unpack(const uint8_t *packed, int64_t rows, int64_t L, int64_t cols, int8_t *out) {
    if (rows < 0 || cols < 0) return -1;
    if (cols > L * TRITS) return -1;
    for (int64_t i = 0; i < rows * L * TRYTES; ++i) {
        if (packed[i] > 26) return -2;
    }
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < cols; ++c) {
            int8_t t[3];
            trits_of(packed[(r * L + c / TRITS) * TRYTES + (c % TRITS) / 3], t);
            out[r * cols + c] = t[c % 3];
        }
    }
    return 0;
}

/* --------------------------------------------------------------- a11 ----
 * Exact 96-trit product of two limbs.  include/t81/core/detail/simd_impl.hpp:
 * 212-223 (48x48 trit convolution), :185-199 (normalize_accumulator: six
 * forward balanced-carry sweeps, one backward sweep, a final digit) and
 * :201-210 (split into low/high limbs); balanced digit and carry as in
 * include/t81/core/limb.hpp:80-85 (C truncating division). */
static inline void balanced_digit_carry(int v, int *digit, int *carry) {
    const int c = (v >= 0) ? (v + 1) / 3 : (v - 1) / 3;
    *carry = c;
    *digit = v - c * 3;
}

void orc_mul_wide(const uint8_t *a, const uint8_t *b, uint8_t *lo, uint8_t *hi) {
    int8_t ta[TRITS], tb[TRITS];
    for (int j = 0; j < TRYTES; ++j) {
        trits_of(a[j], ta + 3 * j);
        trits_of(b[j], tb + 3 * j);
    }
    int acc[2 * TRITS];
    memset(acc, 0, sizeof(acc));
    for (int i = 0; i < TRITS; ++i)
        for (int j = 0; j < TRITS; ++j) acc[i + j] += ta[i] * tb[j];
    for (int pass = 0; pass < 6; ++pass) {
        for (int k = 0; k < 2 * TRITS - 1; ++k) {
            int d, c;
            balanced_digit_carry(acc[k], &d, &c);
            acc[k] = d;
            acc[k + 1] += c;
        }
    }
    for (int k = 2 * TRITS - 1; k > 0; --k) {
        int d, c;
        balanced_digit_carry(acc[k], &d, &c);
        acc[k] = d;
        acc[k - 1] += c;
    }
    {
        int d, c;
        balanced_digit_carry(acc[0], &d, &c);
        acc[0] = d;
    }
    for (int j = 0; j < TRYTES; ++j) {
        lo[j] = tryte_of(acc[3 * j], acc[3 * j + 1], acc[3 * j + 2]);
        hi[j] = tryte_of(acc[TRITS + 3 * j], acc[TRITS + 3 * j + 1], acc[TRITS + 3 * j + 2]);
    }
}

/* --------------------------------------------------------------- a10 ----
 * limb -> double.  include/t81/linalg/gemm.hpp:28-41 builds
 *   table[p][u] = t0*w + t1*w*3.0 + t2*w*9.0,   w = 27^p by repeated *27.0
 * (evaluated left to right, each operation rounded), and :48-56 sums
 * table[p][tryte_p] for p = 0..15 into 0.0 in that order. */
void orc_tryte_table(double *out) {
    double w = 1.0;
    for (int p = 0; p < TRYTES; ++p) {
        for (int u = 0; u < 27; ++u) {
            int8_t t[3];
            trits_of((uint8_t)u, t);
            volatile double a = (double)t[0] * w;
            volatile double b = ((double)t[1] * w) * 3.0;
            volatile double c = ((double)t[2] * w) * 9.0;
            volatile double ab = a + b;
            out[p * 27 + u] = ab + c;
        }
        w *= 27.0;
    }
}

static double g_table[TRYTES * 27];
static int g_table_ready = 0;

static const double *table(void) {
    if (!g_table_ready) {
        orc_tryte_table(g_table);
        g_table_ready = 1;
    }
    return g_table;
}

double orc_limb_to_double(const uint8_t *a) {
    const double *t = table();
    double r = 0.0;
    for (int p = 0; p < TRYTES; ++p) r += t[p * 27 + a[p]];
    return r;
}

/* gemm.hpp:58-64: low + high * (double)RADIX, RADIX = 3^48 (exact integer,
 * rounded once to double). */
static double radix_double(void) {
    unsigned __int128 r = 1;
    for (int i = 0; i < TRITS; ++i) r *= 3;
    return (double)r;
}

double orc_multiply_to_double(const uint8_t *a, const uint8_t *b) {
    uint8_t lo[TRYTES], hi[TRYTES];
    orc_mul_wide(a, b, lo, hi);
    const double low = orc_limb_to_double(lo);
    const double high = orc_limb_to_double(hi);
    volatile double scaled = high * radix_double();
    return low + scaled;
}

/* src/linalg/gemm_cpu.cpp:8-71 with the checks of gemm_gpu.hpp:171-190:
 * C[i,j] = float( C[i,j]*beta + sum_k (product(A[i,k], B[k,j]) * alpha) ),
 * accumulated in double with k ascending (the 8x8x4 blocking of the
 * reference does not change the per-element order).  A is (M, K/48) limbs,
 * B is (K/48, N) limbs, C is (M, N) float32, read then written.
 * Returns 0, or -1 for a shape the reference rejects. */
int orc_gemm_limb(const uint8_t *A, const uint8_t *B, float *C, int M, int N, int K,
                  float alpha, float beta) {
    if (M < 0 || N < 0 || K < 0 || K % TRITS != 0) return -1;
    const int KL = K / TRITS;
    for (int i = 0; i < M; ++i) {
        for (int j = 0; j < N; ++j) {
            double acc = (double)C[(int64_t)i * N + j] * (double)beta;
            for (int k = 0; k < KL; ++k) {
                const double p = orc_multiply_to_double(A + ((int64_t)i * KL + k) * TRYTES,
                                                        B + ((int64_t)k * N + j) * TRYTES);
                volatile double scaled = p * (double)alpha;
                acc = acc + scaled;
            }
            C[(int64_t)i * N + j] = (float)acc;
        }
    }
    return 0;
}

/* ----------------------------------------------------- trit-dot oracle ----
 * The dot-product reading of the same packed weights used by every other
 * consumer in the reference (backward grad = T^T g, t81/torch/__init__.py:
 * 291-304; training forward F.linear(x, ternary(w)), t81/nn/linear.py:43-45):
 *   out[m, n] = sum_{k<K} X[m, k] * T[n, k],  T = trits of packed row n.
 * Double accumulation for float activations; exact int64 for integer ones. */
static void unpack_row(const uint8_t *row, int64_t L, int64_t K, int8_t *t) {
    for (int64_t c = 0; c < K; ++c) {
        int8_t tr[3];
        trits_of(row[(c / TRITS) * TRYTES + (c % TRITS) / 3], tr);
        t[c] = tr[c % 3];
    }
    (void)L;
}

void orc_trit_matmul_f64(const double *x, int64_t M, int64_t K, const uint8_t *w,
                         int64_t N, int8_t *scratch_k, double *out) {
    const int64_t L = (K + TRITS - 1) / TRITS;
    for (int64_t n = 0; n < N; ++n) {
        unpack_row(w + n * L * TRYTES, L, K, scratch_k);
        for (int64_t m = 0; m < M; ++m) {
            const double *xr = x + m * K;
            double s = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                if (scratch_k[k] > 0) s += xr[k];
                else if (scratch_k[k] < 0) s -= xr[k];
            }
            out[m * N + n] = s;
        }
    }
}

/* Also returns sum_k |X[m,k]*T[n,k]| per output, the scale the floating-point
 * tolerances of the tests are relative to. */
void orc_trit_matmul_abs_f64(const double *x, int64_t M, int64_t K, const uint8_t *w,
                             int64_t N, int8_t *scratch_k, double *out) {
    const int64_t L = (K + TRITS - 1) / TRITS;
    for (int64_t n = 0; n < N; ++n) {
        unpack_row(w + n * L * TRYTES, L, K, scratch_k);
        for (int64_t m = 0; m < M; ++m) {
            const double *xr = x + m * K;
            double s = 0.0;
            for (int64_t k = 0; k < K; ++k)
                if (scratch_k[k] != 0) s += fabs(xr[k]);
            out[m * N + n] = s;
        }
    }
}

void orc_trit_matmul_i64(const int8_t *x, int64_t M, int64_t K, const uint8_t *w, int64_t N,
                         int8_t *scratch_k, int64_t *out) {
    const int64_t L = (K + TRITS - 1) / TRITS;
    for (int64_t n = 0; n < N; ++n) {
        unpack_row(w + n * L * TRYTES, L, K, scratch_k);
        for (int64_t m = 0; m < M; ++m) {
            const int8_t *xr = x + m * K;
            int64_t s = 0;
            for (int64_t k = 0; k < K; ++k) s += (int64_t)xr[k] * scratch_k[k];
            out[m * N + n] = s;
        }
    }
}

/* ------------------------------------------------------------- §8(f)4 ----
 * Elementwise float32 ops of the backend contract: the CPU loops of
 * src/linalg/gemm_dispatch.cpp:145-211 (cpu_where :145-161, cpu_clamp :163-177,
 * cpu_lerp :179-194, cpu_addcmul :196-211), each operation rounded separately
 * (this file is built with -ffp-contract=off). */
void orc_where(const float *cond, const float *x, const float *y, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = cond[i] != 0.0f ? x[i] : y[i];
}

void orc_clamp(const float *in, float *out, int64_t n, float lo, float hi) {
    for (int64_t i = 0; i < n; ++i) {
        const float v = in[i];
        out[i] = v < lo ? lo : (v > hi ? hi : v);
    }
}

void orc_lerp(const float *s, const float *e, const float *w, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = s[i] + w[i] * (e[i] - s[i]);
}

void orc_addcmul(const float *in, const float *t1, const float *t2, float value, float *out,
                 int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = in[i] + value * t1[i] * t2[i];
}

/* ---------------------------------------------------------- spmm_simple ----
 * include/t81/sparse/simple.hpp:37-94: C = beta * C (each element through double,
 * or zero when beta == 0), then for every entry in order: weight = double(value) *
 * alpha (a limb built from a long long holds it exactly, limb_to_double sums its
 * trits in int128 and rounds once, python/bindings.cpp:916-918), and for each k
 * C[row, k] = float(double(C[row, k]) + weight * double(B[col, k])).  Returns -1 at
 * the first out-of-range index (the reference throws there, after updating C for the
 * entries before it), -2 for negative dimensions, else 0. */
int orc_spmm_simple(const long long *values, const int32_t *row_idx, const int32_t *col_idx,
                    int64_t nnz, int rows, int cols, const float *B, float *C, int N,
                    float alpha, float beta) {
    if (N < 0 || rows < 0 || cols < 0) return -2;
    const int64_t total = (int64_t)rows * N;
    if (beta == 0.0f) {
        for (int64_t i = 0; i < total; ++i) C[i] = 0.0f;
    } else {
        const double bd = (double)beta;
        for (int64_t i = 0; i < total; ++i) C[i] = (float)((double)C[i] * bd);
    }
    const double ad = (double)alpha;
    for (int64_t e = 0; e < nnz; ++e) {
        const int r = row_idx[e], c = col_idx[e];
        if (r < 0 || r >= rows || c < 0 || c >= cols) return -1;
        const double w = (double)values[e] * ad;
        for (int k = 0; k < N; ++k) {
            const double p = w * (double)B[(int64_t)c * N + k];
            C[(int64_t)r * N + k] = (float)((double)C[(int64_t)r * N + k] + p);
        }
    }
    return 0;
}

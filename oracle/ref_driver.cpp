// oracle/ref_driver.cpp -- C-ABI shim around the reference's own CPU GEMM path.
//
// TEST INFRASTRUCTURE ONLY.  This file is compiled together with the
// reference's unmodified sources (/root/reference/src/linalg/gemm_cpu.cpp and
// the headers under /root/reference/include) into oracle/_ref/libt81ref.so by
// oracle/Makefile.  Nothing from the reference is copied here: the shim only
// calls the reference's functions so that tests and the CPU baseline can reach
// them through plain pointers.  Only tests/, __graft_entry__.smoke() and the
// cpu_baseline leg of bench.py may load the resulting library.
//
// Reference entry points reached:
//   t81::linalg::detail::gemm_ternary_cpu_impl   src/linalg/gemm_cpu.cpp:8-71
//   t81::linalg::detail::build_tryte_contributions include/t81/linalg/gemm.hpp:28-41
//   t81::linalg::detail::limb_to_double           include/t81/linalg/gemm.hpp:48-56
//   t81::linalg::detail::multiply_to_double       include/t81/linalg/gemm.hpp:58-64
//   t81::core::limb::mul_wide                     include/t81/core/limb.hpp:466-471
//   t81::core::detail::mul_wide_scalar            include/t81/core/detail/simd_impl.hpp:212-223
//   t81::core::limb::from_value / from_trits      include/t81/core/limb.hpp:131-158
//   random_limb (mt19937_64 + uniform_int(0,26))  tests/unit/test_limb_basic.cpp:58-66 (restated)
//   t81::linalg::detail::where / clamp / lerp / addcmul on Backend::CPU
//                                                 src/linalg/gemm_dispatch.cpp:239-322
//   t81::core::gguf::compute_scale / quantize_row_tq1_0 / dequantize_row_tq1_0 /
//   half_to_float                                 src/t81/core/gguf_quants.h:55-168

#include <array>
#include <cstdint>
#include <cstring>
#include <random>
#include <span>
#include <stdexcept>

#include <t81/core/gguf_quants.h>
#include <t81/linalg/gemm.hpp>
#include <t81/linalg/gemm_gpu.hpp>
#include <t81/sparse/simple.hpp>
#include <t81/tensor_metadata.hpp>

using t81::core::limb;

namespace {

limb limb_from_raw(const std::uint8_t *bytes) {
    std::array<std::uint8_t, limb::BYTES> raw{};
    std::memcpy(raw.data(), bytes, limb::BYTES);
    return limb::from_bytes(raw);
}

void limb_to_raw(const limb &value, std::uint8_t *bytes) {
    const auto raw = value.to_bytes();
    std::memcpy(bytes, raw.data(), limb::BYTES);
}

} // namespace

extern "C" {

// Writes the 16x27 tryte-contribution table used by limb_to_double.
void t81ref_tryte_table(double *out) {
    const auto &table = t81::linalg::detail::tryte_contribution_table();
    for (int p = 0; p < limb::TRYTES; ++p) {
        for (int u = 0; u < 27; ++u) {
            out[p * 27 + u] = table[p][u];
        }
    }
}

int t81ref_mul_wide(const std::uint8_t *a, const std::uint8_t *b, std::uint8_t *lo,
                    std::uint8_t *hi) {
    try {
        const auto [low, high] = limb::mul_wide(limb_from_raw(a), limb_from_raw(b));
        limb_to_raw(low, lo);
        limb_to_raw(high, hi);
        return 0;
    } catch (const std::exception &) {
        return -1;
    }
}

int t81ref_mul_wide_scalar(const std::uint8_t *a, const std::uint8_t *b, std::uint8_t *lo,
                           std::uint8_t *hi) {
    try {
        const auto [low, high] =
            t81::core::detail::mul_wide_scalar(limb_from_raw(a), limb_from_raw(b));
        limb_to_raw(low, lo);
        limb_to_raw(high, hi);
        return 0;
    } catch (const std::exception &) {
        return -1;
    }
}

double t81ref_limb_to_double(const std::uint8_t *a) {
    return t81::linalg::detail::limb_to_double(limb_from_raw(a));
}

double t81ref_multiply_to_double(const std::uint8_t *a, const std::uint8_t *b) {
    return t81::linalg::detail::multiply_to_double(limb_from_raw(a), limb_from_raw(b));
}

// Balanced-ternary encoding of a signed 64-bit value (|v| < 2^63 always fits a limb).
int t81ref_limb_from_value(long long value, std::uint8_t *out) {
    try {
        limb_to_raw(limb::from_value(static_cast<t81::core::detail::limb_int128>(value)), out);
        return 0;
    } catch (const std::exception &) {
        return -1;
    }
}

// Packs 48 trits (values -1..1) into a limb with the reference's from_trits.
int t81ref_limb_from_trits(const std::int8_t *trits, std::uint8_t *out) {
    try {
        std::array<std::int8_t, limb::TRITS> values{};
        std::memcpy(values.data(), trits, limb::TRITS);
        limb_to_raw(limb::from_trits(values), out);
        return 0;
    } catch (const std::exception &) {
        return -1;
    }
}

void t81ref_limb_min_max(std::uint8_t *min_out, std::uint8_t *max_out) {
    limb_to_raw(limb::min(), min_out);
    limb_to_raw(limb::max(), max_out);
}

// The limb sequence of tests/unit/test_limb_basic.cpp:58-66 (same engine, same
// distribution, same libstdc++), so fixtures can reproduce that test's inputs.
void t81ref_random_limbs(unsigned long long seed, int count, std::uint8_t *out) {
    std::mt19937_64 rng(seed);
    std::uniform_int_distribution<int> dist(0, 26);
    for (int i = 0; i < count * limb::TRYTES; ++i) {
        out[i] = static_cast<std::uint8_t>(dist(rng));
    }
}

// The reference CPU kernel, called with the shape checks of
// gemm_ternary_dispatch (include/t81/linalg/gemm_gpu.hpp:171-190).
// Returns 0, or -1 for an invalid shape (the reference throws std::invalid_argument).
int t81ref_gemm_ternary(const std::uint8_t *A, const std::uint8_t *B, float *C, int M, int N,
                        int K, float alpha, float beta) {
    if (M < 0 || N < 0 || K < 0 || K % limb::TRITS != 0) {
        return -1;
    }
    const int k_limbs = K / limb::TRITS;
    const std::size_t a_count = static_cast<std::size_t>(M) * k_limbs;
    const std::size_t b_count = static_cast<std::size_t>(k_limbs) * N;
    const std::size_t c_count = static_cast<std::size_t>(M) * N;
    if (M == 0 || N == 0) {
        return 0;
    }
    static_assert(sizeof(limb) == limb::BYTES, "limb must be 16 bytes");
    try {
        std::span<const limb> a_span(reinterpret_cast<const limb *>(A), a_count);
        std::span<const limb> b_span(reinterpret_cast<const limb *>(B), b_count);
        std::span<float> c_span(C, c_count);
        t81::linalg::detail::gemm_ternary_cpu_impl(a_span, b_span, c_span, M, N, K, k_limbs,
                                                   alpha, beta);
    } catch (const std::exception &) {
        return -2;
    }
    return 0;
}

// Same kernel over a block of output rows only (used to bound CPU-baseline samples).
int t81ref_gemm_ternary_rows(const std::uint8_t *A, const std::uint8_t *B, float *C, int M,
                             int N, int K, int row_begin, int row_end, float alpha, float beta) {
    if (row_begin < 0 || row_end > M || row_begin > row_end || K % limb::TRITS != 0) {
        return -1;
    }
    const int k_limbs = K / limb::TRITS;
    const int rows = row_end - row_begin;
    return t81ref_gemm_ternary(A + static_cast<std::size_t>(row_begin) * k_limbs * limb::BYTES, B,
                               C + static_cast<std::size_t>(row_begin) * N, rows, N, K, alpha,
                               beta);
}

const char *t81ref_simd_path(void) {
    if (t81::core::detail::cpu_supports_avx512f()) {
        return "avx512f";
    }
    if (t81::core::detail::cpu_supports_avx2()) {
        return "avx2";
    }
    return "scalar";
}

// Elementwise ops through the reference's public dispatch, forced to the CPU loops.
static t81::TensorMetadata f32(const float *p, long long n) {
    return t81::make_contiguous_metadata(static_cast<std::size_t>(n), const_cast<float *>(p));
}

void t81ref_where(const float *cond, const float *x, const float *y, float *out, long long n) {
    auto mc = f32(cond, n), mx = f32(x, n), my = f32(y, n), mo = f32(out, n);
    t81::linalg::detail::where(mc, mx, my, mo, t81::linalg::Backend::CPU);
}

void t81ref_clamp(const float *in, float *out, long long n, float lo, float hi) {
    auto mi = f32(in, n), mo = f32(out, n);
    t81::linalg::detail::clamp(mi, mo, lo, hi, t81::linalg::Backend::CPU);
}

void t81ref_lerp(const float *s, const float *e, const float *w, float *out, long long n) {
    auto ms = f32(s, n), me = f32(e, n), mw = f32(w, n), mo = f32(out, n);
    t81::linalg::detail::lerp(ms, me, mw, mo, t81::linalg::Backend::CPU);
}

void t81ref_addcmul(const float *in, const float *t1, const float *t2, float value, float *out,
                    long long n) {
    auto mi = f32(in, n), m1 = f32(t1, n), m2 = f32(t2, n), mo = f32(out, n);
    t81::linalg::detail::addcmul(mi, m1, m2, value, mo, t81::linalg::Backend::CPU);
}

// t81::sparse::spmm_simple (include/t81/sparse/simple.hpp:37-94) on limbs built from
// long long values, as the pybind11 binding does (python/bindings.cpp:910-928).
// Returns -1 if it throws (C keeps what it held at that point).
int t81ref_spmm_simple(const long long *values, const int *row_idx, const int *col_idx,
                       long long nnz, int rows, int cols, const float *B, float *C, int N,
                       float alpha, float beta) {
    try {
        t81::sparse::SimpleSparseTernary m;
        m.rows = rows;
        m.cols = cols;
        m.row_indices.assign(row_idx, row_idx + nnz);
        m.col_indices.assign(col_idx, col_idx + nnz);
        m.values.reserve(static_cast<std::size_t>(nnz));
        for (long long i = 0; i < nnz; ++i) m.values.emplace_back(values[i]);
        const std::size_t nb = static_cast<std::size_t>(cols) * static_cast<std::size_t>(N < 0 ? 0 : N);
        const std::size_t nc = static_cast<std::size_t>(rows) * static_cast<std::size_t>(N < 0 ? 0 : N);
        t81::sparse::spmm_simple(m, std::span<const float>(B, nb), std::span<float>(C, nc), N,
                                 alpha, beta);
        return 0;
    } catch (const std::exception &) {
        return -1;
    }
}

// ---- the TQ1_0 row codec of src/t81/core/gguf_quants.h, called as it stands ----
float t81ref_tq1_compute_scale(const float *values, long long n) {
    return t81::core::gguf::compute_scale(values, n);
}

void t81ref_tq1_quantize_row(const float *values, long long n, float threshold, float scale,
                             std::uint16_t *dst) {
    t81::core::gguf::quantize_row_tq1_0(values, n, threshold, scale, dst);
}

void t81ref_tq1_dequantize_row(const std::uint16_t *src, long long n, float scale, float *dst) {
    t81::core::gguf::dequantize_row_tq1_0(src, n, scale, dst);
}

float t81ref_tq1_half_to_float(std::uint16_t bits) { return t81::core::gguf::half_to_float(bits); }

} // extern "C"

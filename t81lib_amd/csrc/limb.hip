// t81lib_amd/csrc/limb.hip -- K4: the reference's literal gemm_ternary over limb integers.
//
//   C[i, j] = float( double(C[i, j]) * beta + sum_l product(A[i, l], B[l, j]) * alpha )
//
// product(a, b) is the reference's multiply_to_double (include/t81/linalg/
// gemm.hpp:58-64): the exact 96-trit product split into balanced low/high limbs
// (limb::mul_wide, limb.hpp:466-471), each converted by summing the 16 tryte
// contributions table[p][u_p] in order (gemm.hpp:48-56), then low + high * 3^48.
// The exact product is formed here in balanced base 27 -- one digit per tryte,
// digit = u - 13 in -13..13: a 16x16 digit convolution (|sum| <= 16*169) and one
// carry sweep.  Balanced representations are unique, so the digits equal the
// trytes the reference's 48x48 trit convolution and carry passes
// (simd_impl.hpp:185-223) produce, and the double sums below -- same table, same
// order, no FMA contraction -- are bit-identical to gemm_cpu.cpp:8-71.
// This kernel is the parity path, not the roofline-graded one: one thread per
// output, l ascending.
#include "t81_device.hpp"
#include "t81_kernels.hpp"

#pragma clang fp contract(off)

namespace t81hip {

struct TrTable {
    double v[kTrytes][27];
};

// include/t81/linalg/gemm.hpp:28-41: t0*w + t1*w*3.0 + t2*w*9.0 with w = 27^p by
// repeated *27.0; constant-evaluated, every operation rounded separately.
constexpr TrTable make_tryte_table() {
    TrTable t{};
    double w = 1.0;
    for (int p = 0; p < kTrytes; ++p) {
        for (int u = 0; u < 27; ++u) {
            const double t0 = trit_of(u, 0), t1 = trit_of(u, 1), t2 = trit_of(u, 2);
            t.v[p][u] = t0 * w + t1 * w * 3.0 + t2 * w * 9.0;
        }
        w *= 27.0;
    }
    return t;
}

constexpr double make_radix() {
    unsigned __int128 r = 1;
    for (int i = 0; i < kTrits; ++i) r *= 3;
    return static_cast<double>(r);  // 3^48 rounded once, as static_cast<double>(RADIX)
}

__constant__ TrTable kTable = make_tryte_table();
constexpr TrTable kHostTable = make_tryte_table();
constexpr double kRadix = make_radix();

__device__ __forceinline__ double limb_value_double(const int (&digit)[32], int base) {
    double r = 0.0;
#pragma unroll
    for (int p = 0; p < kTrytes; ++p) r = r + kTable.v[p][digit[base + p] + 13];
    return r;
}

__device__ __forceinline__ double multiply_to_double(const uint4 &a4, const uint4 &b4) {
    int a[kTrytes], b[kTrytes];
    const uint32_t aw[4] = {a4.x, a4.y, a4.z, a4.w};
    const uint32_t bw[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            a[4 * i + j] = static_cast<int>((aw[i] >> (8 * j)) & 0xFFu) - 13;
            b[4 * i + j] = static_cast<int>((bw[i] >> (8 * j)) & 0xFFu) - 13;
        }
    }
    int conv[32];
#pragma unroll
    for (int s = 0; s < 32; ++s) conv[s] = 0;
#pragma unroll
    for (int p = 0; p < kTrytes; ++p)
#pragma unroll
        for (int q = 0; q < kTrytes; ++q) conv[p + q] += a[p] * b[q];
    // balanced base-27 carry sweep: digit in -13..13
    int carry = 0;
#pragma unroll
    for (int s = 0; s < 32; ++s) {
        const int v = conv[s] + carry;
        // floor((v + 13) / 27) without relying on the sign of integer division
        const int c = (v + 13 >= 0) ? (v + 13) / 27 : -((-(v + 13) + 26) / 27);
        conv[s] = v - 27 * c;
        carry = c;
    }
    const double low = limb_value_double(conv, 0);
    const double high = limb_value_double(conv, kTrytes);
    const double scaled = high * kRadix;
    return low + scaled;
}

__global__ __launch_bounds__(256) void gemm_limb_kernel(const uint8_t *__restrict__ a,
                                                        const uint8_t *__restrict__ b,
                                                        float *__restrict__ c, int M, int N,
                                                        int KL, float alpha, float beta) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= static_cast<int64_t>(M) * N) return;
    const int64_t i = t / N;
    const int64_t j = t - i * N;
    double acc = static_cast<double>(c[t]) * static_cast<double>(beta);
    const uint4 *arow = reinterpret_cast<const uint4 *>(a) + i * KL;
    const uint4 *bcol = reinterpret_cast<const uint4 *>(b) + j;
    for (int l = 0; l < KL; ++l) {
        const double p = multiply_to_double(arow[l], bcol[static_cast<int64_t>(l) * N]);
        const double scaled = p * static_cast<double>(alpha);
        acc = acc + scaled;
    }
    c[t] = static_cast<float>(acc);
}

hipError_t launch_gemm_limb(const uint8_t *a, const uint8_t *b, float *c, int m, int n,
                            int k_limbs, float alpha, float beta, hipStream_t s) {
    const int64_t total = static_cast<int64_t>(m) * n;
    if (total == 0) return hipSuccess;
    gemm_limb_kernel<<<dim3((total + 255) / 256), dim3(256), 0, s>>>(a, b, c, m, n, k_limbs,
                                                                     alpha, beta);
    return hipGetLastError();
}

void host_tryte_table(double *out) {
    for (int p = 0; p < kTrytes; ++p)
        for (int u = 0; u < 27; ++u) out[p * 27 + u] = kHostTable.v[p][u];
}

}  // namespace t81hip

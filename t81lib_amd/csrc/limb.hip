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
#include "pack_common.hpp"
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

// The reference's literal matmul_input in one pass (t81/torch/__init__.py:241-276):
// the activations x (tokens x K, row-major) are quantized with the torch form of the
// threshold and packed column-wise (_pack_columnwise, :83-97) inside the kernel, then
// multiplied as limbs exactly as gemm_limb_kernel does.  A workgroup owns 16 weight
// rows x 16 tokens; per chunk of limbs it packs its tokens' limbs (once, into LDS) and
// stages its rows' limbs, and each thread then runs its output's limbs in ascending
// order -- the same operations as pack_cols followed by gemm_limb_kernel, so the same
// bits.  C is rows x tokens.
constexpr int kFuseTile = 16;
constexpr int kFuseChunk = 32;  // limbs per staged chunk

template <typename T, bool kVec>
__global__ __launch_bounds__(256) void gemm_limb_fused_kernel(
    const uint8_t *__restrict__ a, const T *__restrict__ x, float *__restrict__ c, int M, int N,
    int64_t K, int KL, float thr, float alpha, float beta) {
    __shared__ uint4 xs[kFuseTile][kFuseChunk];
    __shared__ uint4 as[kFuseTile][kFuseChunk];
    const int tid = threadIdx.x;
    const int ti = tid / kFuseTile;
    const int tj = tid % kFuseTile;
    const int64_t i0 = static_cast<int64_t>(blockIdx.y) * kFuseTile;
    const int64_t j0 = static_cast<int64_t>(blockIdx.x) * kFuseTile;
    const int64_t i = i0 + ti;
    const int64_t j = j0 + tj;
    const bool live = i < M && j < N;
    double acc = live ? static_cast<double>(c[i * N + j]) * static_cast<double>(beta) : 0.0;
    const uint4 *arows = reinterpret_cast<const uint4 *>(a);
    for (int l0 = 0; l0 < KL; l0 += kFuseChunk) {
        const int cl = KL - l0 < kFuseChunk ? KL - l0 : kFuseChunk;
        for (int d = tid; d < kFuseTile * cl * 4; d += 256) {
            const int tok = d / (cl * 4);
            const int rem = d - tok * cl * 4;
            const int l = rem >> 2;
            const int q = rem & 3;
            const int64_t jj = j0 + tok;
            const uint32_t word =
                jj < N ? pack12<T, kVec>(x + jj * K, static_cast<int64_t>(l0 + l) * kTrits + 12 * q,
                                         K, thr, 1)
                       : 0x0D0D0D0Du;
            reinterpret_cast<uint32_t *>(&xs[tok][l])[q] = word;
        }
        for (int d = tid; d < kFuseTile * cl; d += 256) {
            const int r = d / cl;
            const int l = d - r * cl;
            const int64_t ii = i0 + r;
            as[r][l] = ii < M ? arows[ii * KL + l0 + l]
                              : make_uint4(0x0D0D0D0Du, 0x0D0D0D0Du, 0x0D0D0D0Du, 0x0D0D0D0Du);
        }
        __syncthreads();
        if (live) {
            for (int l = 0; l < cl; ++l) {
                const double p = multiply_to_double(as[ti][l], xs[tj][l]);
                const double scaled = p * static_cast<double>(alpha);
                acc = acc + scaled;
            }
        }
        __syncthreads();
    }
    if (live) c[i * N + j] = static_cast<float>(acc);
}

template <typename T>
hipError_t launch_fused_t(const uint8_t *a, const void *x, float *c, int m, int n, int64_t k,
                          float thr, float alpha, float beta, hipStream_t s) {
    const int KL = static_cast<int>((k + kTrits - 1) / kTrits);
    const dim3 grid((n + kFuseTile - 1) / kFuseTile, (m + kFuseTile - 1) / kFuseTile);
    // vector loads as in the column packer: K % 4 == 0 and a 16-byte aligned x
    const bool vec = (k % 4 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
    if (vec)
        gemm_limb_fused_kernel<T, true><<<grid, 256, 0, s>>>(a, static_cast<const T *>(x), c, m, n,
                                                             k, KL, thr, alpha, beta);
    else
        gemm_limb_fused_kernel<T, false><<<grid, 256, 0, s>>>(a, static_cast<const T *>(x), c, m, n,
                                                              k, KL, thr, alpha, beta);
    return hipGetLastError();
}

hipError_t launch_gemm_limb_fused(const uint8_t *a, const void *x, int x_dtype, float *c, int m,
                                  int n, int64_t k, float thr, float alpha, float beta,
                                  hipStream_t s) {
    if (static_cast<int64_t>(m) * n == 0) return hipSuccess;
    switch (x_dtype) {
        case kDtypeF32: return launch_fused_t<float>(a, x, c, m, n, k, thr, alpha, beta, s);
        case kDtypeBF16: return launch_fused_t<uint16_t>(a, x, c, m, n, k, thr, alpha, beta, s);
        default: return launch_fused_t<_Float16>(a, x, c, m, n, k, thr, alpha, beta, s);
    }
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

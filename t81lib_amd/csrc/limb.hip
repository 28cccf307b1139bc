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
// The convolution runs as signed 4-byte dot products (v_dot4_i32_i8) of a's digits
// against b's digits reversed, and the carry sweep as a multiply-shift; the table lives
// in LDS.  Several lanes per output each form one product, and the output's first lane
// adds them in limb order -- the reference's order, so the same bits.  This is the parity
// path, not the roofline-graded one.
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

constexpr int kTableEntries = kTrytes * 27;

// The tryte table in the workgroup's LDS (tab[27 p + u] = table[p][u]); published by the
// caller's next barrier.
__device__ __forceinline__ void tryte_table_fill(double *tab) {
    for (int e = threadIdx.x; e < kTableEntries; e += blockDim.x)
        tab[e] = kTable.v[e / 27][e % 27];
}

// include/t81/linalg/gemm.hpp:48-56: the 16 tryte contributions of one limb, in order.
__device__ __forceinline__ double limb_value_double(const double *tab, const int (&digit)[32],
                                                    int base) {
    double r = 0.0;
#pragma unroll
    for (int p = 0; p < kTrytes; ++p) r = r + tab[27 * p + digit[base + p] + 13];
    return r;
}

// Four trytes (bytes < 27) -> their digits u - 13 as signed bytes: with bit 7 of every
// byte set, the per-byte subtraction never borrows across bytes.
__device__ __forceinline__ uint32_t tryte_digits(uint32_t w) {
    return ((w | 0x80808080u) - 0x0D0D0D0Du) ^ 0x80808080u;
}

__device__ __forceinline__ double multiply_to_double(const double *tab, const uint4 &a4,
                                                     const uint4 &b4) {
    const uint32_t aw[4] = {a4.x, a4.y, a4.z, a4.w};
    const uint32_t bw[4] = {b4.x, b4.y, b4.z, b4.w};
    // ad: a's digits; pb: b's digits reversed (b[15 - x] at byte x of dwords 4..7) with
    // four zero dwords either side
    uint32_t ad[4], pb[12];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        ad[i] = tryte_digits(aw[i]);
        pb[4 + i] = __builtin_bswap32(tryte_digits(bw[3 - i]));
        pb[i] = 0u;
        pb[8 + i] = 0u;
    }
    // conv[s] = sum_p a[p] b[s - p] (|conv| <= 16 * 169): per 4-digit block k of a, the
    // reversed b's bytes from offset 31 - s + 4k (compile-time offsets)
    auto window = [&](int off) -> int {
        const int d = off >> 2, r = off & 3;
        return static_cast<int>(r == 0 ? pb[d] : __builtin_amdgcn_alignbyte(pb[d + 1], pb[d], r));
    };
    int conv[32];
#pragma unroll
    for (int s = 0; s < 31; ++s) {
        int acc = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k)
            acc = __builtin_amdgcn_sdot4(static_cast<int>(ad[k]), window(31 - s + 4 * k), acc,
                                         false);
        conv[s] = acc;
    }
    conv[31] = 0;
    // balanced base-27 carry sweep, digit in -13..13: |v| < 2810, so n = v + 5413 lies in
    // [2603, 8223] and floor((v + 13) / 27) = floor(n / 27) - 200 = (n * 38837 >> 20) - 200
    // (the multiply-shift is exact for 0 <= n < 45590)
    int carry = 0;
#pragma unroll
    for (int s = 0; s < 32; ++s) {
        const int v = conv[s] + carry;
        const int c = static_cast<int>((static_cast<uint32_t>(v + 5413) * 38837u) >> 20) - 200;
        conv[s] = v - 27 * c;
        carry = c;
    }
    const double low = limb_value_double(tab, conv, 0);
    const double high = limb_value_double(tab, conv, kTrytes);
    const double scaled = high * kRadix;
    return low + scaled;
}

// LPO lanes per output: each forms one limb product (scaled by alpha) per pass of LPO
// limbs, and the output's first lane adds them to its sum in limb order -- the
// operations and order of gemm_cpu.cpp:8-71.
template <int LPO>
__global__ __launch_bounds__(256) void gemm_limb_kernel(const uint8_t *__restrict__ a,
                                                        const uint8_t *__restrict__ b,
                                                        float *__restrict__ c, int M, int N,
                                                        int KL, float alpha, float beta) {
    __shared__ double prod[256];
    __shared__ double tab[kTableEntries];
    tryte_table_fill(tab);
    __syncthreads();
    const int g = threadIdx.x / LPO;   // output within the workgroup
    const int ln = threadIdx.x % LPO;  // limb lane
    const int64_t t = static_cast<int64_t>(blockIdx.x) * (256 / LPO) + g;
    const bool live = t < static_cast<int64_t>(M) * N;
    const int64_t i = live ? t / N : 0;
    const int64_t j = live ? t - i * N : 0;
    double acc = live && ln == 0 ? static_cast<double>(c[t]) * static_cast<double>(beta) : 0.0;
    const uint4 *arow = reinterpret_cast<const uint4 *>(a) + i * KL;
    const uint4 *bcol = reinterpret_cast<const uint4 *>(b) + j;
    for (int l0 = 0; l0 < KL; l0 += LPO) {
        const int l = l0 + ln;
        double scaled = 0.0;
        if (live && l < KL) {
            const double p = multiply_to_double(tab, arow[l], bcol[static_cast<int64_t>(l) * N]);
            scaled = p * static_cast<double>(alpha);
        }
        prod[threadIdx.x] = scaled;
        __syncthreads();
        if (live && ln == 0) {
            const int cnt = KL - l0 < LPO ? KL - l0 : LPO;
            for (int q = 0; q < cnt; ++q) acc = acc + prod[g * LPO + q];
        }
        __syncthreads();
    }
    if (live && ln == 0) c[t] = static_cast<float>(acc);
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
    __shared__ double tab[kTableEntries];
    tryte_table_fill(tab);   // published by the first chunk's barrier
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
                const double p = multiply_to_double(tab, as[ti][l], xs[tj][l]);
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
    // lanes per output: the limb count rounded up to 16, 32 or 64 (config 1: 22 limbs, 32
    // lanes: 70.5 -> 30.6 us against one thread per output with the convolution as
    // multiply-adds and a branching carry sweep; 512 x 128 x 100 limbs 313.6 -> 114.4 us)
    if (k_limbs <= 16)
        gemm_limb_kernel<16><<<dim3((total + 15) / 16), dim3(256), 0, s>>>(a, b, c, m, n, k_limbs,
                                                                          alpha, beta);
    else if (k_limbs <= 32)
        gemm_limb_kernel<32><<<dim3((total + 7) / 8), dim3(256), 0, s>>>(a, b, c, m, n, k_limbs,
                                                                         alpha, beta);
    else
        gemm_limb_kernel<64><<<dim3((total + 3) / 4), dim3(256), 0, s>>>(a, b, c, m, n, k_limbs,
                                                                         alpha, beta);
    return hipGetLastError();
}

void host_tryte_table(double *out) {
    for (int p = 0; p < kTrytes; ++p)
        for (int u = 0; u < 27; ++u) out[p * 27 + u] = kHostTable.v[p][u];
}

}  // namespace t81hip

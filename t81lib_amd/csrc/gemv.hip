// t81lib_amd/csrc/gemv.hip -- K2: decode-shaped ternary matmul (M <= 16 tokens).
//
//   C[m, n] = alpha * sum_k X[m, k] * T[n, k] + beta * C[m, n] + bias[n]
//
// The packed weights (N x L x 16 bytes, the reference layout) are the only large
// stream, so the kernel is HBM-bound: every weight byte is read exactly once,
// with 16-byte loads, and decoded in registers.  The multiply-accumulate runs
// on the matrix cores (v_mfma_f32_16x16x32_bf16): decoded trits are exact in
// bf16, and the MFMA keeps the per-byte VALU cost at the decode alone (about
// 1.75 VALU ops + one 8-byte LDS read per weight byte) whatever M is, where a
// VALU dot product would add 3*M multiply-adds per byte.
//
// Work split.  A workgroup of 4 waves owns 16*G consecutive weight rows; the
// waves split the K dimension (4-limb sub-blocks, round-robin) and their
// partial 16x16 tiles are summed through LDS at the end, so no atomics and a
// fixed summation order (results are deterministic run to run).
//
// Operand layout.  In one sub-block, lane (r, q) = (lane % 16, lane / 16) loads
// limb 4*s + q of row r (16 bytes, 48 trits) and decodes it into six 8-trit
// A fragments in natural trit order.  MFMA j pairs A-lane (r, q) slots with
// B-lane (m, q) slots, so B-lane (m, q) supplies X[m, 48*(4s+q) + 8j .. +8] --
// eight consecutive activations, one 16-byte load.  Which k an MFMA slot means
// internally is irrelevant: A and B use the same (lane/16, slot) -> k map.
// Output tile: lane (m, q) holds rows n = 4q + i (i < 4) of column m.
#include "t81_device.hpp"
#include "t81_kernels.hpp"

namespace t81hip {

namespace {

constexpr int kWaves = 4;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// ---- activation fragments: 8 consecutive X[m, k0 .. k0+8) as bf16 (hi, lo) ----
template <int XT, bool kAligned>
__device__ __forceinline__ void load_x8(const void *x, int64_t row_off, int64_t k0, int64_t K,
                                        bool valid, bf16x8 &hi, bf16x8 &lo) {
    u32x4 zero = {0u, 0u, 0u, 0u};
    hi = __builtin_bit_cast(bf16x8, zero);
    lo = hi;
    if (!valid) return;
    if constexpr (XT == kDtypeBF16) {
        const uint16_t *p = static_cast<const uint16_t *>(x) + row_off + k0;
        if (kAligned && k0 + 8 <= K) {
            hi = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(p));
        } else {
            uint16_t v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = (k0 + i < K) ? p[i] : static_cast<uint16_t>(0);
            hi = __builtin_bit_cast(bf16x8, v);
        }
    } else if constexpr (XT == kDtypeF32) {
        const float *p = static_cast<const float *>(x) + row_off + k0;
        float v[8];
        if (kAligned && k0 + 8 <= K) {
            const float4 a = reinterpret_cast<const float4 *>(p)[0];
            const float4 b = reinterpret_cast<const float4 *>(p)[1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = (k0 + i < K) ? p[i] : 0.0f;
        }
        // x = hi + lo with hi = bf16(x), lo = bf16(x - hi): |x - hi - lo| <= 2^-18 |x|
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const __bf16 h = static_cast<__bf16>(v[i]);
            hi[i] = h;
            lo[i] = static_cast<__bf16>(v[i] - static_cast<float>(h));
        }
    } else {  // int8: exact in bf16
        const int8_t *p = static_cast<const int8_t *>(x) + row_off + k0;
        int8_t v[8];
        if (kAligned && k0 + 8 <= K) {
            const uint2 raw = *reinterpret_cast<const uint2 *>(p);
            __builtin_memcpy(v, &raw, 8);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = (k0 + i < K) ? p[i] : static_cast<int8_t>(0);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) hi[i] = static_cast<__bf16>(static_cast<float>(v[i]));
    }
}

__device__ __forceinline__ u32x4 load_limb(const uint8_t *w, int64_t row, int64_t limb,
                                           int64_t N, int64_t L) {
    if (row < N && limb < L) {
        const u32x4 *p = reinterpret_cast<const u32x4 *>(w + (row * L + limb) * kTrytes);
        return __builtin_nontemporal_load(p);
    }
    const u32x4 pad = {0x0D0D0D0Du, 0x0D0D0D0Du, 0x0D0D0D0Du, 0x0D0D0D0Du};  // all-zero trits
    return pad;
}

template <int XT, int G, bool kAligned>
__global__ __launch_bounds__(256) void gemv_kernel(const void *__restrict__ x,
                                                   const uint8_t *__restrict__ w,
                                                   void *__restrict__ c, int M, int64_t N,
                                                   int64_t K, int64_t L, float alpha, float beta,
                                                   const float *__restrict__ bias) {
    __shared__ __attribute__((aligned(16))) uint8_t lut[kLutBytes];
    __shared__ __attribute__((aligned(16))) floatx4 red[kWaves][G][64];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int r = lane & 15;   // A row within a 16-row group / B column (token)
    const int q = lane >> 4;   // k-quarter
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * (16 * G);
    const int64_t S = (L + 3) / 4;  // 4-limb sub-blocks

    lut_init(lut, tid, 256);

    floatx4 acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = floatx4{0.f, 0.f, 0.f, 0.f};

    const bool xvalid = r < M;
    const int64_t xrow = static_cast<int64_t>(r) * K;

    int64_t s = wave;
    u32x4 wcur[G];
#pragma unroll
    for (int g = 0; g < G; ++g) wcur[g] = load_limb(w, n0 + 16 * g + r, 4 * s + q, N, L);

    for (; s < S; s += kWaves) {
        // prefetch the next sub-block's weights while this one is decoded
        u32x4 wnext[G];
        const int64_t sn = s + kWaves;
#pragma unroll
        for (int g = 0; g < G; ++g) wnext[g] = load_limb(w, n0 + 16 * g + r, 4 * sn + q, N, L);

        const int64_t kbase = (4 * s + q) * kTrits;
        bf16x8 bh[6], bl[6];
#pragma unroll
        for (int j = 0; j < 6; ++j)
            load_x8<XT, kAligned>(x, xrow, kbase + 8 * j, K, xvalid && (4 * s + q) < L, bh[j],
                                  bl[j]);

#pragma unroll
        for (int g = 0; g < G; ++g) {
            uint32_t pairs[24];
#pragma unroll
            for (int d = 0; d < 4; ++d) decode_dword(lut, wcur[g][d], pairs + 6 * d);
#pragma unroll
            for (int j = 0; j < 6; ++j) {
                const u32x4 araw = {pairs[4 * j], pairs[4 * j + 1], pairs[4 * j + 2],
                                    pairs[4 * j + 3]};
                const bf16x8 a = __builtin_bit_cast(bf16x8, araw);
                acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bh[j], acc[g], 0, 0, 0);
                if constexpr (XT == kDtypeF32)
                    acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl[j], acc[g], 0, 0, 0);
            }
            wcur[g] = wnext[g];
        }
    }

    // ---- split-K reduction over the 4 waves, then the epilogue ----
#pragma unroll
    for (int g = 0; g < G; ++g) red[wave][g][lane] = acc[g];
    __syncthreads();

    for (int g = wave; g < G; g += kWaves) {
        floatx4 v = red[0][g][lane];
#pragma unroll
        for (int ww = 1; ww < kWaves; ++ww) v += red[ww][g][lane];
        if (r >= M) continue;
        const int64_t nb = n0 + 16 * g + 4 * q;
        if constexpr (XT == kDtypeI8) {
            int32_t *cr = static_cast<int32_t *>(c) + static_cast<int64_t>(r) * N;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (nb + i < N) {
                    int32_t y = static_cast<int32_t>(v[i]);
                    if (beta != 0.0f) y += cr[nb + i];
                    cr[nb + i] = y;
                }
            }
        } else {
            float *cr = static_cast<float *>(c) + static_cast<int64_t>(r) * N;
            float y[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t n = nb + i;
                float t = alpha * v[i];
                if (n < N) {
                    if (beta != 0.0f) t = t + beta * cr[n];
                    if (bias != nullptr) t = t + bias[n];
                }
                y[i] = t;
            }
            if (nb + 3 < N && (reinterpret_cast<uintptr_t>(cr + nb) & 15u) == 0) {
                *reinterpret_cast<float4 *>(cr + nb) = make_float4(y[0], y[1], y[2], y[3]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (nb + i < N) cr[nb + i] = y[i];
            }
        }
    }
}

template <int XT, int G>
hipError_t launch_gemv_t(const void *x, const uint8_t *w, void *c, int m, int64_t n, int64_t k,
                         float alpha, float beta, const float *bias, hipStream_t s) {
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t blocks = (n + 16 * G - 1) / (16 * G);
    const int elem = XT == kDtypeF32 ? 4 : (XT == kDtypeBF16 ? 2 : 1);
    const bool aligned = (k % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % (8 * elem) == 0);
    if (aligned)
        gemv_kernel<XT, G, true><<<dim3(blocks), dim3(256), 0, s>>>(x, w, c, m, n, k, L, alpha,
                                                                    beta, bias);
    else
        gemv_kernel<XT, G, false><<<dim3(blocks), dim3(256), 0, s>>>(x, w, c, m, n, k, L, alpha,
                                                                     beta, bias);
    return hipGetLastError();
}

template <int XT>
hipError_t launch_gemv_g(const void *x, const uint8_t *w, void *c, int m, int64_t n, int64_t k,
                         float alpha, float beta, const float *bias, hipStream_t s) {
    // more rows per wave amortise the activation loads once several tokens are live
    if (m <= 4) return launch_gemv_t<XT, 1>(x, w, c, m, n, k, alpha, beta, bias, s);
    return launch_gemv_t<XT, 2>(x, w, c, m, n, k, alpha, beta, bias, s);
}

}  // namespace

hipError_t launch_gemv(const void *x, int x_dtype, const uint8_t *w, void *c, int m, int64_t n,
                       int64_t k, float alpha, float beta, const float *bias, hipStream_t s) {
    if (m == 0 || n == 0) return hipSuccess;
    switch (x_dtype) {
        case kDtypeBF16: return launch_gemv_g<kDtypeBF16>(x, w, c, m, n, k, alpha, beta, bias, s);
        case kDtypeF32: return launch_gemv_g<kDtypeF32>(x, w, c, m, n, k, alpha, beta, bias, s);
        default: return launch_gemv_g<kDtypeI8>(x, w, c, m, n, k, alpha, beta, bias, s);
    }
}

}  // namespace t81hip

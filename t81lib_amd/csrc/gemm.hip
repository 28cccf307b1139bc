// t81lib_amd/csrc/gemm.hip -- K3: prefill-shaped ternary matmul (any M, tuned for M >= 64).
//
//   C[m, n] = alpha * sum_k X[m, k] * T[n, k] + beta * C[m, n] + bias[n]
//
// At prefill sizes the product is a dense contraction (2*M*N*K flops against
// ~N*K/3 weight bytes), so the kernel is built around v_mfma_f32_32x32x16_bf16.
// Decoded trits (-1, 0, +1) are exact in bf16; bf16 activations feed the MFMA
// directly, fp32 activations as a hi + lo bf16 pair (two MFMAs, |error| <=
// 2^-18 |x| per product), int8 activations exactly (fp32 sums of integers stay
// exact while |sum| < 2^24, which the ABI enforces through K <= 131071).
//
// Tiling.  A workgroup of WN x WM waves computes a (32*RN*WN) x (32*CM*WM)
// tile of C^T (weight rows x tokens).  Per k-step of LK limbs (48 * LK trits):
//  * the activation tile (tokens x 96) goes global -> registers -> LDS,
//    double-buffered, one barrier per k-step;
//  * every wave loads its own weight rows straight into registers -- lane
//    (r, h) = (lane % 32, lane / 32) takes bytes 8h..8h+7 of a limb of row r,
//    24 trits that decode (LDS lookup table) into the A fragments of the three
//    MFMAs of that limb; B-lane (c, h) then needs X[c, 48l + 24h + 8j .. +8],
//    16 contiguous bytes of the LDS tile.  The weight stream never touches LDS.
// Output: lane (c, h) of a 32x32 block holds rows 8a + 4h + b (a, b < 4) of
// column c, so each lane stores 4 consecutive outputs of one token.
#include "t81_device.hpp"
#include "t81_kernels.hpp"

namespace t81hip {

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <int XT, int RN, int CM, int WN, int WM, int LK>
struct GemmCfg {
    static constexpr int kLK = LK;                        // limbs per k-step
    static constexpr int kStepK = kLK * kTrits;           // trits per k-step
    static constexpr int kRowBytes = kStepK * 2 + 16;     // bf16 tile row + pad (bank spread)
    static constexpr int kThreads = 64 * WN * WM;
    static constexpr int kBN = 32 * RN * WN;  // weight rows per workgroup
    static constexpr int kBM = 32 * CM * WM;  // tokens per workgroup
    static constexpr int kPlanes = XT == kDtypeF32 ? 2 : 1;  // hi (+ lo) bf16 tiles
    static constexpr int kTileBytes = kBM * kRowBytes;
    static constexpr int kChunks = kBM * (kStepK / 8);  // 8-element chunks per tile
    static constexpr int kChunksPerThread = (kChunks + kThreads - 1) / kThreads;
};

// Loads 8 consecutive activations X[m, k0..k0+8) and returns them as bf16 hi/lo bits.
template <int XT, bool kAligned>
__device__ __forceinline__ void fetch_x8(const void *x, int64_t m, int64_t k0, int64_t M,
                                         int64_t K, u32x4 &hi, u32x4 &lo) {
    hi = u32x4{0u, 0u, 0u, 0u};
    lo = hi;
    if (m >= M) return;
    if constexpr (XT == kDtypeBF16) {
        const uint16_t *p = static_cast<const uint16_t *>(x) + m * K + k0;
        if (kAligned && k0 + 8 <= K) {
            hi = *reinterpret_cast<const u32x4 *>(p);
        } else {
            uint16_t v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = (k0 + i < K) ? p[i] : static_cast<uint16_t>(0);
            hi = __builtin_bit_cast(u32x4, v);
        }
    } else if constexpr (XT == kDtypeF32) {
        const float *p = static_cast<const float *>(x) + m * K + k0;
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
        bf16x8 h, l;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const __bf16 t = static_cast<__bf16>(v[i]);
            h[i] = t;
            l[i] = static_cast<__bf16>(v[i] - static_cast<float>(t));
        }
        hi = __builtin_bit_cast(u32x4, h);
        lo = __builtin_bit_cast(u32x4, l);
    } else {
        const int8_t *p = static_cast<const int8_t *>(x) + m * K + k0;
        int8_t v[8];
        if (kAligned && k0 + 8 <= K) {
            const uint2 raw = *reinterpret_cast<const uint2 *>(p);
            __builtin_memcpy(v, &raw, 8);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = (k0 + i < K) ? p[i] : static_cast<int8_t>(0);
        }
        bf16x8 h;
#pragma unroll
        for (int i = 0; i < 8; ++i) h[i] = static_cast<__bf16>(static_cast<float>(v[i]));
        hi = __builtin_bit_cast(u32x4, h);
    }
}

__device__ __forceinline__ u32x2 load_half_limb(const uint8_t *w, int64_t row, int64_t limb,
                                                int h, int64_t N, int64_t L) {
    if (row < N && limb < L) {
        const u32x2 *p = reinterpret_cast<const u32x2 *>(w + (row * L + limb) * kTrytes + 8 * h);
        return *p;
    }
    return u32x2{0x0D0D0D0Du, 0x0D0D0D0Du};  // all-zero trits
}

template <int XT, int RN, int CM, int WN, int WM, int LK, bool kAligned>
__global__ __launch_bounds__(64 * WN * WM) void gemm_kernel(
    const void *__restrict__ x, const uint8_t *__restrict__ w, void *__restrict__ c, int64_t M,
    int64_t N, int64_t ldc, int64_t K, int64_t L, float alpha, float beta,
    const float *__restrict__ bias) {
    using Cfg = GemmCfg<XT, RN, CM, WN, WM, LK>;
    constexpr int kLK = Cfg::kLK;
    constexpr int kStepK = Cfg::kStepK;
    constexpr int kRowBytes = Cfg::kRowBytes;
    __shared__ __attribute__((aligned(16))) uint8_t lut[kLutBytes];
    __shared__ __attribute__((aligned(16))) uint8_t xs[2][Cfg::kPlanes][Cfg::kTileBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave % WN;
    const int wm = wave / WN;
    const int r = lane & 31;
    const int h = lane >> 5;

    // blockIdx.x walks the weight-row tiles fastest so that workgroups running
    // together share the same activation rows (they stay hot in L2).
    const int64_t tiles_n = (N + Cfg::kBN - 1) / Cfg::kBN;
    const int64_t tn = blockIdx.x % tiles_n;
    const int64_t tm = blockIdx.x / tiles_n;
    const int64_t n0 = tn * Cfg::kBN + 32 * RN * wn;
    const int64_t m0 = tm * Cfg::kBM;
    const int64_t nsteps = (L + kLK - 1) / kLK;

    lut_init(lut, tid, Cfg::kThreads);

    floatx16 acc[RN][CM];
#pragma unroll
    for (int i = 0; i < RN; ++i)
#pragma unroll
        for (int j = 0; j < CM; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    // ---- activation tile staging ----
    u32x4 xh[Cfg::kChunksPerThread], xl[Cfg::kChunksPerThread];
    auto fetch_tile = [&](int64_t step) {
#pragma unroll
        for (int i = 0; i < Cfg::kChunksPerThread; ++i) {
            const int chunk = tid + i * Cfg::kThreads;
            xh[i] = u32x4{0u, 0u, 0u, 0u};
            xl[i] = xh[i];
            if (chunk < Cfg::kChunks) {
                const int row = chunk / (kStepK / 8);
                const int col = chunk % (kStepK / 8);
                fetch_x8<XT, kAligned>(x, m0 + row, step * kStepK + 8 * col, M, K, xh[i], xl[i]);
            }
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < Cfg::kChunksPerThread; ++i) {
            const int chunk = tid + i * Cfg::kThreads;
            if (chunk < Cfg::kChunks) {
                const int row = chunk / (kStepK / 8);
                const int col = chunk % (kStepK / 8);
                *reinterpret_cast<u32x4 *>(&xs[buf][0][row * kRowBytes + 16 * col]) = xh[i];
                if constexpr (Cfg::kPlanes == 2)
                    *reinterpret_cast<u32x4 *>(&xs[buf][1][row * kRowBytes + 16 * col]) = xl[i];
            }
        }
    };

    // ---- weight fragments (registers only) ----
    u32x2 wc[RN][kLK], wnx[RN][kLK];
    auto fetch_w = [&](int64_t step, u32x2 (&dst)[RN][kLK]) {
#pragma unroll
        for (int i = 0; i < RN; ++i)
#pragma unroll
            for (int l = 0; l < kLK; ++l)
                dst[i][l] = load_half_limb(w, n0 + 32 * i + r, step * kLK + l, h, N, L);
    };

    if (nsteps > 0) {
        fetch_tile(0);
        fetch_w(0, wc);
        store_tile(0);
    }
    __syncthreads();

    for (int64_t step = 0; step < nsteps; ++step) {
        const int buf = static_cast<int>(step & 1);
        const bool more = step + 1 < nsteps;
        if (more) {
            fetch_tile(step + 1);
            fetch_w(step + 1, wnx);
        }
#pragma unroll
        for (int l = 0; l < kLK; ++l) {
            // A fragments: 3 MFMAs x RN row blocks
            bf16x8 a[RN][3];
#pragma unroll
            for (int i = 0; i < RN; ++i) {
                uint32_t pairs[12];
                decode_dword(lut, wc[i][l].x, pairs);
                decode_dword(lut, wc[i][l].y, pairs + 6);
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    const u32x4 raw = {pairs[4 * j], pairs[4 * j + 1], pairs[4 * j + 2],
                                       pairs[4 * j + 3]};
                    a[i][j] = __builtin_bit_cast(bf16x8, raw);
                }
            }
#pragma unroll
            for (int cb = 0; cb < CM; ++cb) {
                const int trow = 32 * (CM * wm + cb) + r;
                const int tcol = (kTrits * l + 24 * h) * 2;  // byte offset in the tile row
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    const u32x4 braw = *reinterpret_cast<const u32x4 *>(
                        &xs[buf][0][trow * kRowBytes + tcol + 16 * j]);
                    const bf16x8 b = __builtin_bit_cast(bf16x8, braw);
#pragma unroll
                    for (int i = 0; i < RN; ++i)
                        acc[i][cb] =
                            __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][j], b, acc[i][cb], 0, 0, 0);
                    if constexpr (Cfg::kPlanes == 2) {
                        const u32x4 lraw = *reinterpret_cast<const u32x4 *>(
                            &xs[buf][1][trow * kRowBytes + tcol + 16 * j]);
                        const bf16x8 bl = __builtin_bit_cast(bf16x8, lraw);
#pragma unroll
                        for (int i = 0; i < RN; ++i)
                            acc[i][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][j], bl,
                                                                                 acc[i][cb], 0, 0, 0);
                    }
                }
            }
        }
        if (more) {
            store_tile(buf ^ 1);
#pragma unroll
            for (int i = 0; i < RN; ++i)
#pragma unroll
                for (int l = 0; l < kLK; ++l) wc[i][l] = wnx[i][l];
        }
        __syncthreads();
    }

    // ---- epilogue ----
#pragma unroll
    for (int i = 0; i < RN; ++i) {
#pragma unroll
        for (int cb = 0; cb < CM; ++cb) {
            const int64_t m = m0 + 32 * (CM * wm + cb) + r;
            if (m >= M) continue;
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                const int64_t nb = n0 + 32 * i + 8 * a4 + 4 * h;
                if constexpr (XT == kDtypeI8) {
                    int32_t *cr = static_cast<int32_t *>(c) + m * ldc;
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        if (nb + b < N) {
                            int32_t y = static_cast<int32_t>(acc[i][cb][4 * a4 + b]);
                            if (beta != 0.0f) y += cr[nb + b];
                            cr[nb + b] = y;
                        }
                    }
                } else {
                    float *cr = static_cast<float *>(c) + m * ldc;
                    float y[4];
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const int64_t n = nb + b;
                        float t = alpha * acc[i][cb][4 * a4 + b];
                        if (n < N) {
                            if (beta != 0.0f) t = t + beta * cr[n];
                            if (bias != nullptr) t = t + bias[n];
                        }
                        y[b] = t;
                    }
                    if (nb + 3 < N && (reinterpret_cast<uintptr_t>(cr + nb) & 15u) == 0) {
                        *reinterpret_cast<float4 *>(cr + nb) = make_float4(y[0], y[1], y[2], y[3]);
                    } else {
#pragma unroll
                        for (int b = 0; b < 4; ++b)
                            if (nb + b < N) cr[nb + b] = y[b];
                    }
                }
            }
        }
    }
}

// Rows [0, n) of W and columns [0, n) of C, whose rows are ldc elements apart.
template <int XT, int RN, int CM, int WN, int WM, int LK>
hipError_t launch_gemm_t(const void *x, const uint8_t *w, void *c, int64_t m, int64_t n,
                         int64_t ldc, int64_t k, float alpha, float beta, const float *bias,
                         hipStream_t s) {
    using Cfg = GemmCfg<XT, RN, CM, WN, WM, LK>;
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t tiles = ((n + Cfg::kBN - 1) / Cfg::kBN) * ((m + Cfg::kBM - 1) / Cfg::kBM);
    const int elem = XT == kDtypeF32 ? 4 : (XT == kDtypeBF16 ? 2 : 1);
    const bool aligned = (k % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % (8 * elem) == 0);
    if (aligned)
        gemm_kernel<XT, RN, CM, WN, WM, LK, true><<<dim3(tiles), dim3(Cfg::kThreads), 0, s>>>(
            x, w, c, m, n, ldc, k, L, alpha, beta, bias);
    else
        gemm_kernel<XT, RN, CM, WN, WM, LK, false><<<dim3(tiles), dim3(Cfg::kThreads), 0, s>>>(
            x, w, c, m, n, ldc, k, L, alpha, beta, bias);
    return hipGetLastError();
}

// Compute units of the current device (one workgroup of the big tile fits per CU).
int cu_count() {
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

template <int XT>
hipError_t launch_gemm_x(const void *x, const uint8_t *w, void *c, int64_t m, int64_t n,
                         int64_t k, float alpha, float beta, const float *bias, hipStream_t s) {
    constexpr int LK = 2;  // limbs per k-step
    if (m <= 32) return launch_gemm_t<XT, 2, 1, 4, 1, LK>(x, w, c, m, n, n, k, alpha, beta, bias, s);
    if (m <= 64) return launch_gemm_t<XT, 2, 2, 4, 1, LK>(x, w, c, m, n, n, k, alpha, beta, bias, s);
    if constexpr (XT != kDtypeF32) {
        // Eight waves (two per SIMD, so one wave's waits are covered by the other's
        // MFMAs): 256 x 256 tiles while there are enough of them to spread over the
        // GPU, 256 weight rows x 128 tokens otherwise (measured crossover ~160 tiles).
        const int64_t tiles_m = (m + 255) / 256;
        const int64_t tiles_big = ((n + 255) / 256) * tiles_m;
        if (tiles_big < 160)
            return launch_gemm_t<XT, 2, 2, 4, 2, LK>(x, w, c, m, n, n, k, alpha, beta, bias, s);
        // One big-tile workgroup per CU at a time: when the last round of big tiles would
        // be at most half full, the rows of whole rounds take big tiles and the rest
        // (fewer rows) the half-height tiles, one short round instead of a half-empty one.
        const int64_t cus = cu_count();
        const int64_t rem = tiles_big % cus;
        const int64_t n1 = (tiles_big - rem) / tiles_m * 256;
        if (tiles_big > cus && rem != 0 && 2 * rem <= cus && n1 > 0 && n1 < n) {
            hipError_t e = launch_gemm_t<XT, 2, 4, 4, 2, LK>(x, w, c, m, n1, n, k, alpha, beta,
                                                           bias, s);
            if (e != hipSuccess) return e;
            const int64_t L = (k + kTrits - 1) / kTrits;
            return launch_gemm_t<XT, 2, 2, 4, 2, LK>(x, w + n1 * L * kTrytes,
                                                   static_cast<uint8_t *>(c) + 4 * n1, m, n - n1,
                                                   n, k, alpha, beta, bias ? bias + n1 : nullptr, s);
        }
        return launch_gemm_t<XT, 2, 4, 4, 2, LK>(x, w, c, m, n, n, k, alpha, beta, bias, s);
    }
    // fp32 activations: two LDS planes; four waves with 256 x 128 tiles
    return launch_gemm_t<XT, 2, 4, 4, 1, LK>(x, w, c, m, n, n, k, alpha, beta, bias, s);
}

}  // namespace

hipError_t launch_gemm(const void *x, int x_dtype, const uint8_t *w, void *c, int64_t m,
                       int64_t n, int64_t k, float alpha, float beta, const float *bias,
                       hipStream_t s) {
    if (m == 0 || n == 0) return hipSuccess;
    switch (x_dtype) {
        case kDtypeBF16: return launch_gemm_x<kDtypeBF16>(x, w, c, m, n, k, alpha, beta, bias, s);
        case kDtypeF32: return launch_gemm_x<kDtypeF32>(x, w, c, m, n, k, alpha, beta, bias, s);
        default: return launch_gemm_x<kDtypeI8>(x, w, c, m, n, k, alpha, beta, bias, s);
    }
}

}  // namespace t81hip

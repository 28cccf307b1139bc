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
#include <type_traits>

#include "t81_device.hpp"
#include "t81_kernels.hpp"

namespace t81hip {

// Compute units of the current device, cached per device.
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

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

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

// Split-K: with part != nullptr, workgroup (split sp, tile t) runs k-steps
// [sp * sps, (sp + 1) * sps) and writes its raw sums (float; int32 for int8 activations,
// exact) to part + sp * M * N as a row-major M x N matrix; gemm_split_sum_kernel adds
// the splits in order and applies alpha, beta and bias.
template <int XT, int RN, int CM, int WN, int WM, int LK, bool kAligned>
__global__ __launch_bounds__(64 * WN * WM) void gemm_kernel(
    const void *__restrict__ x, const uint8_t *__restrict__ w, void *__restrict__ c, int64_t M,
    int64_t N, int64_t ldc, int64_t K, int64_t L, float alpha, float beta,
    const float *__restrict__ bias, int64_t sps, void *__restrict__ part) {
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
    const int64_t tiles = tiles_n * ((M + Cfg::kBM - 1) / Cfg::kBM);
    const int64_t sp = blockIdx.x / tiles;
    const int64_t tt = blockIdx.x - sp * tiles;
    const int64_t tn = tt % tiles_n;
    const int64_t tm = tt / tiles_n;
    const int64_t n0 = tn * Cfg::kBN + 32 * RN * wn;
    const int64_t m0 = tm * Cfg::kBM;
    const int64_t all_steps = (L + kLK - 1) / kLK;
    const int64_t s_begin = sp * sps;
    const int64_t s_end = s_begin + sps < all_steps ? s_begin + sps : all_steps;
    if (part != nullptr) {  // this split's raw sums, row-major M x N
        c = static_cast<uint8_t *>(part) + sp * M * N * 4;
        ldc = N;
        alpha = 1.0f;
        beta = 0.0f;
        bias = nullptr;
    }

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

    if (s_begin < s_end) {
        fetch_tile(s_begin);
        fetch_w(s_begin, wc);
        store_tile(0);
    }
    __syncthreads();

    for (int64_t step = s_begin; step < s_end; ++step) {
        const int buf = static_cast<int>((step - s_begin) & 1);
        const bool more = step + 1 < s_end;
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

// ---------------------------------------------------------------------------
// Big-tile kernel for bf16 activations: one wave per SIMD.
//
// A workgroup of four waves computes a 256 x 256 tile of C^T; wave (wn, wm) owns
// 128 weight rows x 128 tokens, i.e. 4 x 4 blocks of v_mfma_f32_32x32x16_bf16
// (256 accumulator registers).  WR = 4 ("tall" tiles):
// the four waves side by side along the rows instead of 2 x 2, a 512 x 128 tile -- each
// wave's MFMAs, decode and B reads as before, but the workgroup's activation tile is
// half as large, so a step issues half the global -> LDS tile loads (7 per wave instead
// of 13; gate_up M = 2048 367 -> 356 us, M = 8192 1398 -> 1356 us, qkv / down at M =
// 8192 -3 % / -2 %, bit-identical), for twice the weight bytes per token tile (read from
// L2 and the MALL).  (RB = 3, WR = 4: 384 x 128 tiles, three row blocks per wave, for
// shapes whose 256-row tiles leave CUs idle; whole tiles only.)  A k-step is two limbs
// (96 trits):
//  * lane (r, h) loads all 16 bytes of limb 2s + h of row 32 rb + r, so one
//    32-trit slice of the MFMA pairs trits 8J..8J+7 of limb 2s (h = 0) with the
//    same trits of limb 2s + 1 (h = 1), J = 0..5; B lane (c, h) reads
//    X[c, 96s + 48h + 8J .. +8], 16 bytes of the activation tile;
//  * the weights decode (LDS table) half a limb at a time: half p gives the
//    A fragments of J = 3p..3p+2 for all four row blocks.  The decode of the
//    next half runs while the MFMAs of the current one do; the weights of a step
//    are loaded two steps ahead;
//  * the activation tile of step s + 1 goes straight from global memory into the
//    other LDS buffer (buffer loads with the LDS bit, no registers) at the start
//    of step s; one barrier per step.  Tile rows are 13 16-byte slots (12 chunks of
//    8 activations + 1 pad slot), so the 16-byte B reads of 16 lanes fall on
//    distinct banks.  Chunks past K or past M, and the pad slots, load zeros
//    (out-of-range buffer offsets).
constexpr int kW4Threads = 256;
constexpr int kW4Rows = 256;                        // weight rows per workgroup
constexpr int kW4Tokens = 256;                      // tokens per workgroup
constexpr int kW4StepK = 2 * kTrits;                // trits per k-step
constexpr int kW4RowSlots = kW4StepK / 8 + 1;       // 16-byte slots per tile row (+1 pad)
constexpr int kW4RowBytes = 16 * kW4RowSlots;       // 208
constexpr int kW4TileBytes = kW4Tokens * kW4RowBytes;
constexpr uint32_t kW4Oob = 0x80000000u;
constexpr int kW4StageStride = 68;   // floats per staged output row: 64 columns + 4 pad
constexpr int kW4StageBytes = 4 * 32 * kW4StageStride * 4;   // four waves' staging regions

// A raw buffer descriptor over [base, base + bytes) (clamped to 2^31 - 1 bytes) whose
// fields are forced into scalar registers: the loads then need no per-lane
// descriptor checks.  base and bytes must be the same in every lane.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void *base, int64_t bytes) {
    const uint64_t p = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32));
    const int n = __builtin_amdgcn_readfirstlane(bytes < 0x7FFFFFFF ? static_cast<int>(bytes)
                                                                    : 0x7FFFFFFF);
    return __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void *>((static_cast<uint64_t>(hi) << 32) | lo), 0, n, 0x00020000);
}

// Work items.  Weight rows [0, n1) run as whole 256 x 256 tiles (512 x 128 for WR = 4;
// all k-steps, result to C).  Rows [n1, N) run either as split-K items (nsplit > 0): item
// (split sp, tile t of that region) runs k-steps [sp * sps, (sp + 1) * sps) and stores its
// raw accumulators (no alpha, beta, bias) to part in the order (sp, t, wave, block, a4,
// lane) as float4s -- every store is 1 KB contiguous; gemm_split_reduce_kernel<WR> then
// sums the splits in order -- or (half != 0) as half-width tiles of 256 rows x 128 tokens
// (512 x 64) over all k-steps, result to C: when those fill about one round of the CUs
// they need no workspace and no second launch.  Half of the remainder's items come first
// and half last in the item order, so the workgroups that start with a (shorter)
// remainder item finish their whole tiles half a tile out of step with the others, and
// the C stores of the two halves do not all land at once.
template <int XT, int RB, bool kBeta, int WR = 2>
__global__ __launch_bounds__(kW4Threads) void gemm_w4_kernel(
    const void *__restrict__ x, const uint8_t *__restrict__ w, void *__restrict__ c, int M, int N,
    int ldc, int K, int L, float alpha, float beta, const float *__restrict__ bias, int n1,
    int sps, float4 *__restrict__ part, int nsplit, int half) {
    static_assert(XT == kDtypeBF16, "the LDS tile is filled straight from bf16 activations");
    static_assert(RB == 3 || RB == 4, "three or four 32-row blocks per wave");
    if constexpr (RB == 3) {
        // the 384-row instance has no remainder path: every row is in a whole tile
        n1 = N;
        nsplit = 0;
        half = 0;
    }
    static_assert((WR == 2 && RB == 4) || WR == 4, "waves 2 x 2, or 4 along the rows");
    constexpr int WT = 4 / WR;            // waves along the tokens
    constexpr int kRows = 32 * RB * WR;   // weight rows per tile
    constexpr int kTokW = 128 * WT;       // tokens per whole tile
    // Two separate tile objects (not one array indexed by a run-time parity): the
    // loads into one buffer then provably do not alias the reads of the other, and
    // the compiler need not wait for them before every LDS read.  A half-width item
    // (and every WR = 4 item) uses the first half of each, or less.
    // (The table's larger alignment places it at LDS address 0, so a table address is
    // just the byte field, with no base to add.)
    __shared__ __attribute__((aligned(1024))) uint8_t lut[kLutBytes];
    __shared__ __attribute__((aligned(16))) uint8_t xs0[kW4TileBytes];
    __shared__ __attribute__((aligned(16))) uint8_t xs1[kW4TileBytes];
    // Epilogue staging, one region per wave (32 tokens x 64 weight rows of results), in the
    // first tile buffer: past an item's last barrier no tile byte that is used is read or
    // written any more (the last step's tile loads have landed and its last B reads fetch
    // unused bytes), and each item starts with a barrier, so no wave's next tile loads
    // overwrite a region another wave is still using.  The static LDS is then the table
    // and the two tiles only, below the bound for global -> LDS load targets wherever the
    // compiler places them.
    static_assert(kW4StageBytes <= kW4TileBytes, "the epilogue staging must fit a tile buffer");
    // (the table plus the most alignment padding any placement can add: 1024 bytes)
    static_assert(1024 + 2 * kW4TileBytes + 1024 <= kLdsDmaLimit, "LDS-load targets past 128 KiB");
    auto tile = [&](auto bufc) -> uint8_t * {
        if constexpr (decltype(bufc)::value == 0) return xs0;
        else return xs1;
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = WR == 4 ? wave : wave & 1;
    const int wm = WR == 4 ? 0 : wave >> 1;

    // Items walk the weight-row tiles fastest: items running together share their
    // activation rows.  (Tile indices are uniform: readfirstlane keeps them, and the
    // buffer descriptors built from them, in scalar registers.)  The grid is
    // persistent, one workgroup per CU taking items blockIdx.x, + gridDim.x, ...: a
    // new workgroup per tile started only after the C stores of the whole previous
    // round had drained (~15 us a round at M = 2048).
    const int tiles_m = (M + kTokW - 1) / kTokW;
    const int tiles_mh = (M + kTokW / 2 - 1) / (kTokW / 2);   // half-width tiles
    const int tn1 = (n1 + kRows - 1) / kRows;        // row tiles of whole tiles
    const int tn2 = (N - n1 + kRows - 1) / kRows;    // row tiles of the remainder
    const int full_items = tn1 * tiles_m;
    const int tiles2 = tn2 * tiles_m;
    const int rem_items = half ? tn2 * tiles_mh : (nsplit > 0 ? tiles2 * nsplit : 0);
    const int head = rem_items / 2;                      // remainder items placed first
    const int total = full_items + rem_items;
    const int all_steps = (L + 1) / 2;
    lut_fill(lut, tid, kW4Threads);  // published by the first item's barrier

    // One item: 32 RB WR weight rows (nwg..) x 32 CB WT tokens (m0..) over k-steps
    // [s_begin, s_end); wave (wn, wm) owns 32 RB rows x 32 CB tokens.  CB = 4: whole or
    // split-K tiles; CB = 2: half-width tiles.
    auto run_item = [&](auto cbc, int nwg, int m0, int s_begin, int s_end, bool split, int sp,
                        int tt) {
        constexpr int CB = decltype(cbc)::value;      // 32-token blocks per wave
        constexpr int kTok = 32 * CB * WT;             // tokens per workgroup
        // every wave is past the previous item's epilogue (staged in xs0) before this
        // item's tile loads
        __syncthreads();
        // tile loads per workgroup (52, 26, 13) and per wave (13; 7, the last wave 5; 4, the
        // last wave 1)
        constexpr int kTL = kTok * kW4RowSlots / 64;
        constexpr int LPW = (kTL + 3) / 4;
        constexpr int NCH = 6 * CB;                    // chunks of four MFMAs per step
        constexpr int HALF = 3 * CB;                   // chunks per half step
        constexpr int NF = CB == 4 ? 2 * RB : RB;      // chunks of a half that read the table
        constexpr int FPC = 2 * RB / NF;               // weight dwords looked up per such chunk
        constexpr int kWLoads = RB;                    // loads of fetch_w: one per row block
        constexpr int kWaitW = waitcnt_vm<kWLoads>();  // all but the newest fetch_w
        // the half-width prologue's two tiles: all but the newest fetch_w and tile loads
        constexpr int kWaitTwo = waitcnt_vm<kWLoads + LPW>();

        // The lane index passes through an empty asm once per item, so the per-lane
        // offsets derived from it are recomputed per item instead of being hoisted out of
        // the loop and kept live across the epilogue (where they would spill).
        int lane = tid & 63;
        asm volatile("" : "+v"(lane));
        const int r = lane & 31;
        const int h = lane >> 5;

        // Weights through a buffer based at the workgroup's first row: rows past N read
        // zeros.  A limb index past L (odd L, last step) reads the next row's first limb
        // or zeros; either decodes to finite trits that meet zero activations.
        const __amdgpu_buffer_rsrc_t wsrc = uniform_rsrc(
            w + static_cast<int64_t>(nwg) * L * kTrytes, static_cast<int64_t>(N - nwg) * L * kTrytes);
        uint32_t woff[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
            woff[rb] = (static_cast<uint32_t>(32 * RB * wn + 32 * rb + r) * static_cast<uint32_t>(L) +
                        static_cast<uint32_t>(h)) * kTrytes;
        auto fetch_w = [&](int step, u32x4 (&dst)[RB]) {
            const uint32_t koff = static_cast<uint32_t>(step) * (2 * kTrytes);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
                dst[rb] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(wsrc, woff[rb] + koff, 0, 0));
        };

        // Activation tile: load i of wave w fills slots q = 64 (LPW w + i) + lane, tile row
        // q / 13, slot q % 13 (loads past kTL are not issued).  Activations through a
        // buffer based at token m0: tokens past M read zeros.
        const __amdgpu_buffer_rsrc_t xsrc =
            uniform_rsrc(static_cast<const uint16_t *>(x) + static_cast<int64_t>(m0) * K,
                         static_cast<int64_t>(M - m0) * K * 2);
        // Per-lane constants of the loads: the byte offset of the chunk for k0 = 0 (or an
        // out-of-range offset for a pad slot) and, packed four to a register, 8 * slot,
        // the chunk's first trit within the step (past K the chunk loads zeros).
        uint32_t tbase[LPW];
        uint32_t tslot[(LPW + 3) / 4];
#pragma unroll
        for (int i = 0; i < (LPW + 3) / 4; ++i) tslot[i] = 0u;
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const uint32_t q = static_cast<uint32_t>(64 * (LPW * wave + i) + lane);
            const uint32_t row = q / kW4RowSlots;
            const uint32_t slot = q - row * kW4RowSlots;
            tbase[i] = slot < kW4RowSlots - 1
                           ? (row * static_cast<uint32_t>(K) + 8 * slot) * 2
                           : kW4Oob;
            tslot[i / 4] |= (8 * slot) << (8 * (i % 4));
        }
        // Load i of the wave's share of the tile of k-step `step` into LDS buffer buf
        // (all zeros past the last step).  The last wave's spare loads of a half-width
        // tile (slots 26, 27: LDS bytes 26624..28671, inside the buffer and never read)
        // load zeros -- an out-of-range offset, not a branch, which would split the
        // chunk's scheduling region.
        auto load_tile_part = [&](int step, auto bufc, int i) {
            const bool spare = LPW * 4 != kTL && i >= kTL - 3 * LPW && LPW * wave + i >= kTL;
            const int k0 = step * kW4StepK;
            const uint32_t lim = k0 < K && !spare ? static_cast<uint32_t>(K - k0) : 0u;
            const uint32_t slot8 = (tslot[i / 4] >> (8 * (i % 4))) & 0xFFu;
            const uint32_t off = slot8 < lim ? tbase[i] + static_cast<uint32_t>(k0) * 2 : kW4Oob;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xsrc,
                (__attribute__((address_space(3))) void *)(
                    &tile(bufc)[16 * 64 * (LPW * wave + i)]),
                16, off, 0, 0, 0);
        };
        auto load_tile = [&](int step, auto bufc) {
#pragma unroll
            for (int i = 0; i < LPW; ++i) load_tile_part(step, bufc, i);
        };

        // Half p of the lane's limbs -> A fragments J = 3p + j of the four row blocks.
        auto decode_half = [&](const u32x4 (&wl)[RB], int p, bf16x8 (&a)[RB][3]) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                uint32_t pairs[12];
                decode_dword(lut, wl[rb][2 * p], pairs);
                decode_dword(lut, wl[rb][2 * p + 1], pairs + 6);
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    const u32x4 raw = {pairs[4 * j], pairs[4 * j + 1], pairs[4 * j + 2],
                                       pairs[4 * j + 3]};
                    a[rb][j] = __builtin_bit_cast(bf16x8, raw);
                }
            }
        };

        floatx16 acc[RB][CB];
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int j = 0; j < CB; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

        // B fragment gi of a step (gi < NCH): half p = gi / HALF, J = 3p + (gi % HALF) / CB,
        // token block cb = gi % CB.  B lane (c, h): token 32 CB wm + 32 cb + c of the tile,
        // trits 48h + 8J.. of the step.
        const int brow = (32 * CB * wm + r) * kW4RowBytes + 96 * h;
        auto read_b = [&](auto bufc, int gi) -> u32x4 {
            const int p = gi / HALF;
            const int gg = gi % HALF;
            return *reinterpret_cast<const u32x4 *>(
                &tile(bufc)[brow + 32 * (gg % CB) * kW4RowBytes + 16 * (3 * p + gg / CB)]);
        };
        // decode_dword in two parts, so the table reads can be issued ahead of the merge
        // that needs them.
        auto table_fetch = [&](uint32_t wd, uint2 (&e)[4]) {
            const uint32_t w8 = wd << 3;
            e[0] = *reinterpret_cast<const uint2 *>(lut + kLutE + (w8 & 0xFFu));
            e[1] = *reinterpret_cast<const uint2 *>(lut + kLutF + ((w8 >> 8) & 0xFFu));
            e[2] = *reinterpret_cast<const uint2 *>(lut + kLutE + ((w8 >> 16) & 0xFFu));
            e[3] = *reinterpret_cast<const uint2 *>(lut + kLutF + (w8 >> 24));
        };
        auto table_merge = [&](const uint2 (&e)[4], uint32_t *out) {
            out[0] = e[0].x;
            out[1] = e[0].y | e[1].x;
            out[2] = e[1].y;
            out[3] = e[2].x;
            out[4] = e[2].y | e[3].x;
            out[5] = e[3].y;
        };
        u32x4 wcur[RB], wnxt[RB], wnn[RB];
        bf16x8 a0[RB][3], a1[RB][3];
        if (s_begin < s_end) {
            fetch_w(s_begin, wcur);
            load_tile(s_begin, B0());
        }
        fetch_w(s_begin + 1, wnxt);   // stays in flight across the barrier
        if constexpr (CB == 4) {
            // vmcnt(RB): the tile's LDS writes have landed before the barrier publishes them
            __builtin_amdgcn_s_waitcnt(kWaitW);
        } else {
            // a half-width step is too short to cover its tile loads, so every step
            // loads the tile of the step after next: here the second step's tile too.
            // Issued after the first tile: the weights of the second step (kWLoads loads)
            // and the second tile (LPW loads, every wave, spare ones included), which may
            // stay in flight.  One step only: the weight loads.
            if (s_begin + 1 < s_end) {
                load_tile(s_begin + 1, B1());
                __builtin_amdgcn_s_waitcnt(kWaitTwo);
            } else {
                __builtin_amdgcn_s_waitcnt(kWaitW);
            }
        }
        __syncthreads();
        if (s_begin < s_end) decode_half(wcur, 0, a0);
        u32x4 bq[4];
        bq[0] = read_b(B0(), 0);
        bq[1] = read_b(B0(), 1);
        bq[2] = read_b(B0(), 2);

        // One k-step as NCH chunks of four MFMAs (the first half with a0, the second with
        // a1), one B fragment each, read three chunks ahead.  Chunks are fenced so that
        // each also carries its share of the decode -- the first NF chunks of the first
        // half: half 1 of wcur into a1; of the second half: half 0 of wnxt (the next
        // step) into a0; table reads two chunks ahead of their merge -- and of the loads.
        // Whole tiles (CB = 4): the tile of the next step (chunks 0 .. LPW - 2, two loads
        // in the last), then the weights of the step after it (chunk LPW - 1); issued
        // after the tile loads, the weight loads
        // can stay in flight across the step's wait (vmcnt(RB)), so they have a step and a
        // half to land, not half a step.  Half-width tiles (CB = 2): the weights of the
        // step after next (chunk 0), and, past the barrier, the tile of the step after
        // next into this step's buffer (chunks 9-11; not in the item's last step, so no
        // LDS write is left pending when the item ends).  (All other loads are
        // unconditional: past the last step they read zeros or unused weight bytes.)
        // Steps alternate between the two tile buffers, so the loop below runs two steps
        // per iteration.
        // The step's barrier comes after chunk NCH - 4, whose B read is the last of this
        // step's buffer: past it the next tile is complete (every wave's loads waited
        // for) and no wave reads this buffer again, so the last three chunks read the
        // next step's first three B fragments (the next step starts with its operands in
        // registers, not waiting on LDS), and the buffer may be refilled.  In an item's
        // last step those three reads fetch bytes that are never used.
        auto step_body = [&](int step, auto bufc, auto otherc) {
            uint2 e[3][FPC][4];
            uint32_t pairs[RB][12];
#pragma unroll
            for (int g = 0; g < NCH; ++g) {
                const int p = g / HALF;
                const int gg = g % HALF;
                if (g + 3 < NCH) bq[(g + 3) % 4] = read_b(bufc, g + 3);
                else bq[(g + 3) % 4] = read_b(otherc, g + 3 - NCH);
                if (gg < NF) {
#pragma unroll
                    for (int f2 = 0; f2 < FPC; ++f2) {
                        const int f = gg * FPC + f2;
                        table_fetch((p == 0 ? wcur : wnxt)[f / 2][2 * (1 - p) + (f % 2)],
                                    e[gg % 3][f2]);
                    }
                }
                if (gg >= 2 && gg < NF + 2) {
#pragma unroll
                    for (int f2 = 0; f2 < FPC; ++f2) {
                        const int f = (gg - 2) * FPC + f2;
                        table_merge(e[(gg - 2) % 3][f2], &pairs[f / 2][6 * (f % 2)]);
                    }
                }
                if constexpr (CB == 4) {
                    if (g < LPW - 1) load_tile_part(step + 1, otherc, g);
                    if (g == LPW - 2) load_tile_part(step + 1, otherc, LPW - 1);
                    if (g == LPW - 1) fetch_w(step + 2, wnn);
                } else {
                    if (g == 0) fetch_w(step + 2, wnn);
                    if (step + 1 < s_end) {
                        if (g == 9) {
                            load_tile_part(step + 2, bufc, 0);
                            if (LPW > 1) load_tile_part(step + 2, bufc, 1);
                            if (LPW > 2) load_tile_part(step + 2, bufc, 2);
                        }
                        if (g == 10) {
                            if (LPW > 3) load_tile_part(step + 2, bufc, 3);
                            if (LPW > 4) load_tile_part(step + 2, bufc, 4);
                        }
                        if (g == 11) {
                            if (LPW > 5) load_tile_part(step + 2, bufc, 5);
                            if (LPW > 6) load_tile_part(step + 2, bufc, 6);
                        }
                    }
                }
                const bf16x8 b = __builtin_bit_cast(bf16x8, bq[g % 4]);
                const bf16x8(&a)[RB][3] = p == 0 ? a0 : a1;
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
                    acc[rb][gg % CB] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        a[rb][gg / CB], b, acc[rb][gg % CB], 0, 0, 0);
                if (gg == HALF - 1) {
                    bf16x8(&next)[RB][3] = p == 0 ? a1 : a0;
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                        for (int j = 0; j < 3; ++j) {
                            const u32x4 raw = {pairs[rb][4 * j], pairs[rb][4 * j + 1],
                                               pairs[rb][4 * j + 2], pairs[rb][4 * j + 3]};
                            next[rb][j] = __builtin_bit_cast(bf16x8, raw);
                        }
                }
                // Each MFMA followed by a few of the chunk's other instructions (two LDS
                // reads, three VALU / SALU, one buffer load): with one wave per SIMD, issue
                // is in order, so three MFMAs issued back to back (the default schedule)
                // left the matrix pipe idle while the rest of the chunk issued after them.
#pragma unroll
                for (int k = 0; k < RB; ++k) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // LDS read
                    __builtin_amdgcn_sched_group_barrier(0x006, 3, 0);   // VALU, SALU
                    __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);   // buffer load
                }
                __builtin_amdgcn_sched_barrier(0);
                if (g == NCH - 4) {
                    // vmcnt(RB): the tile loads are older than the RB weight loads of
                    // step + 2
                    __builtin_amdgcn_s_waitcnt(kWaitW);
                    __syncthreads();
                }
            }
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                wcur[rb] = wnxt[rb];
                wnxt[rb] = wnn[rb];
            }
        };
        int step = s_begin;
        for (; step + 1 < s_end; step += 2) {
            step_body(step, B0(), B1());
            step_body(step + 1, B1(), B0());
        }
        if (step < s_end)  // odd step count: the last step, peeled (no join inside the loop)
            step_body(step, B0(), B1());

        if constexpr (CB == 4 && RB == 4) {
            if (split) {
                float4 *dst =
                    part + (((static_cast<int64_t>(sp) * tiles2 + tt) * 4 + wave) * 64) * 64 + lane;
#pragma unroll
                for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                        for (int a4 = 0; a4 < 4; ++a4)
                            dst[((rb * 4 + cb) * 4 + a4) * 64] =
                                make_float4(acc[rb][cb][4 * a4], acc[rb][cb][4 * a4 + 1],
                                            acc[rb][cb][4 * a4 + 2], acc[rb][cb][4 * a4 + 3]);
                return;
            }
        }

        // ---- epilogue: lane (c, h) of block (rb, cb) holds rows 8 a4 + 4 h + b of token c ----
        // The results go out 32 tokens x 64 weight rows at a time through the wave's LDS
        // region: written there in the MFMA layout, read back as four tokens x 64
        // consecutive rows per instruction, so each global store (and each C read for
        // beta) covers four 256-byte runs instead of 32 runs of 32 bytes.  A wave's LDS
        // operations complete in order, so the region needs no barrier.
        float *cdst = static_cast<float *>(c);
        const int col0 = nwg;
        const int ldv = ldc;
        const int nv = N;
        const float al = alpha;
        const float be = beta;
        const float *bi = bias;
        const bool vec4 = ldv % 4 == 0 && (reinterpret_cast<uintptr_t>(cdst) & 15u) == 0;
        float *st = reinterpret_cast<float *>(xs0) + wave * (32 * kW4StageStride);
        const int tq = lane >> 4;          // token within a group of four
        const int tc = 4 * (lane & 15);    // first of the lane's four rows within the 64
        // With beta != 0 (the kBeta instance) the C values of each pass (32 tokens x 64
        // rows) are loaded one pass ahead, so only the first pass waits for them: issued
        // inside the pass, every pass had waited for its own C reads (gate_up M = 2048 with
        // beta = 1: 444.7 -> 417.5 us, M = 8192 1794 -> 1610 us).  The beta = 0 instance
        // has none of this code (with it, beta = 0 ran ~1 % slower).
        constexpr int kRP = (RB + 1) / 2;
        constexpr int kPasses = CB * kRP;
        auto c_pass = [&](int p, float4 (&cv)[8]) {
            const int cb = p / kRP;
            const int rp = p % kRP;
            const int prow = 2 * rp + 1 < RB ? 64 : 32;
            const int nb = col0 + 32 * RB * wn + 64 * rp + tc;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int tok = 4 * i + tq;
                const int m = m0 + 32 * CB * wm + 32 * cb + tok;
                const bool ok = vec4 && m < M && tc < prow && nb + 3 < nv;
                // non-temporal: each C value is read once (gate_up beta = 1 M = 2048
                // 394.0 -> 384.3 us, M = 8192 1518 -> 1496)
                f32x4 t = {0.f, 0.f, 0.f, 0.f};
                if (ok)
                    t = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(
                        cdst + static_cast<int64_t>(m) * ldv + nb));
                cv[i] = make_float4(t[0], t[1], t[2], t[3]);
            }
        };
        float4 cva[8], cvb[8];
        if constexpr (kBeta) c_pass(0, cva);
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
            for (int rp = 0; rp < kRP; ++rp) {
                const int pass = cb * kRP + rp;
                float4 (&cvc)[8] = pass % 2 == 0 ? cva : cvb;
                float4 (&cvn)[8] = pass % 2 == 0 ? cvb : cva;
                if constexpr (kBeta)
                    if (pass + 1 < kPasses) c_pass(pass + 1, cvn);
                // rows of this pass: 64, or 32 for the third block of three
                const int prow = 2 * rp + 1 < RB ? 64 : 32;
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    if (2 * rp + j < RB)
#pragma unroll
                    for (int a4 = 0; a4 < 4; ++a4)
                        *reinterpret_cast<float4 *>(&st[r * kW4StageStride + 32 * j + 8 * a4 + 4 * h]) =
                            make_float4(acc[2 * rp + j][cb][4 * a4], acc[2 * rp + j][cb][4 * a4 + 1],
                                        acc[2 * rp + j][cb][4 * a4 + 2], acc[2 * rp + j][cb][4 * a4 + 3]);
                const int nb = col0 + 32 * RB * wn + 64 * rp + tc;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int tok = 4 * i + tq;
                    const float4 v = *reinterpret_cast<const float4 *>(&st[tok * kW4StageStride + tc]);
                    const int m = m0 + 32 * CB * wm + 32 * cb + tok;
                    if (m >= M || tc >= prow) continue;
                    float *cr = cdst + static_cast<int64_t>(m) * ldv;
                    float y[4] = {al * v.x, al * v.y, al * v.z, al * v.w};
                    if (vec4 && nb + 3 < nv) {
                        if constexpr (kBeta) {
                            const float4 cv = cvc[i];
                            y[0] += be * cv.x;
                            y[1] += be * cv.y;
                            y[2] += be * cv.z;
                            y[3] += be * cv.w;
                        }
                        if (bi != nullptr) {
                            const float4 bv = *reinterpret_cast<const float4 *>(bi + nb);
                            y[0] += bv.x;
                            y[1] += bv.y;
                            y[2] += bv.z;
                            y[3] += bv.w;
                        }
                        // non-temporal: C is not read again here, and every CU stores a
                        // whole tile's C at about the same time (gate_up M = 2048 373 -> 363 us)
                        const f32x4 yv = {y[0], y[1], y[2], y[3]};
                        __builtin_nontemporal_store(yv, reinterpret_cast<f32x4 *>(cr + nb));
                    } else {
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            const int n = nb + b;
                            if (n < nv) {
                                float t = y[b];
                                if (be != 0.0f) t = t + be * cr[n];
                                if (bi != nullptr) t = t + bi[n];
                                cr[n] = t;
                            }
                        }
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    for (int q = static_cast<int>(blockIdx.x); q < total; q += static_cast<int>(gridDim.x)) {
        const bool rem = q < head || q >= head + full_items;
        const int item =
            __builtin_amdgcn_readfirstlane(q < head ? q : (rem ? q - full_items : q - head));
        if (half && rem) {
            // (unreachable for RB = 3, whose remainder is forced empty above)
            if constexpr (RB == 4) {
                const int tn = __builtin_amdgcn_readfirstlane(item % tn2);
                const int tm = __builtin_amdgcn_readfirstlane(item / tn2);
                run_item(std::integral_constant<int, 2>(), n1 + tn * kRows, tm * (kTokW / 2),
                         0, all_steps, false, 0, 0);
            }
        } else {
            const bool split = rem;
            const int sp = split ? item / tiles2 : 0;
            const int tt = split ? item - sp * tiles2 : item;   // tile within its region
            const int tiles_n = split ? tn2 : tn1;
            const int tn = __builtin_amdgcn_readfirstlane(tt % tiles_n);
            const int tm = __builtin_amdgcn_readfirstlane(tt / tiles_n);
            const int s_begin = split ? sp * sps : 0;
            const int s_end = split && s_begin + sps < all_steps ? s_begin + sps : all_steps;
            run_item(std::integral_constant<int, 4>(), (split ? n1 : 0) + tn * kRows,
                     tm * kTokW, s_begin, s_end, split, sp, tt);
        }
    }  // work items
}

// Whether the big-tile kernel takes this shape: bf16 activations, 16-byte rows of
// whole chunks, 32-bit buffer offsets for a workgroup's weights and activations, and
// tile counts (< 2^26) whose work items fit the kernel's int indices (split plans only
// arise below 160 tiles).
bool gemm_w4_fits(const void *x, int64_t m, int64_t n, int64_t k) {
    const int64_t L = (k + kTrits - 1) / kTrits;
    return k % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
           int64_t(kW4Rows) * L * kTrytes < 0x7FFFFFFF &&
           int64_t(kW4Tokens) * k * 2 < 0x7FFFFFFF && m > 0 && m < (int64_t(1) << 30) &&
           n < (int64_t(1) << 30) &&
           ((m + kW4Tokens - 1) / kW4Tokens) * ((n + kW4Rows - 1) / kW4Rows) < (int64_t(1) << 26);
}

// C from the split partials.  Workgroup (tile, wave, token block cb) sums that
// block's 1024 float4 slots over the splits in split order (coalesced: 1 KB runs in the
// order the big-tile kernel stored them), stages its 32 tokens x 128 weight rows in LDS,
// then writes them as 512-byte runs of C rows, applying alpha, beta and bias as the
// kernel's own epilogue does.
constexpr int kReducePitch = 132;   // floats per staged token row: 128 + 4 pad

// WR = 4: the partials of tall split items (512 x 128 tiles, wave w on rows 128 w ..).
template <int WR = 2>
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(
    const float4 *__restrict__ part, float *__restrict__ c, int64_t M, int64_t N, int64_t ldc,
    int tiles, int nsplit, float alpha, float beta, const float *__restrict__ bias) {
    __shared__ __attribute__((aligned(16))) float st[32 * kReducePitch];
    const int tt = static_cast<int>(blockIdx.x >> 4);
    const int wave = static_cast<int>((blockIdx.x >> 2) & 3);
    const int cb = static_cast<int>(blockIdx.x & 3);
    const int wn = WR == 4 ? wave : wave & 1, wm = WR == 4 ? 0 : wave >> 1;
    const int tiles_n = static_cast<int>((N + 128 * WR - 1) / (128 * WR));
    const int64_t m0 = static_cast<int64_t>(tt / tiles_n) * (512 / WR) + 128 * wm + 32 * cb;
    if (m0 >= M) return;
    const int64_t per_split = static_cast<int64_t>(tiles) * 4 * 64 * 64;
    const float4 *src = part + (static_cast<int64_t>(tt) * 4 + wave) * 4096;
    for (int i = threadIdx.x; i < 1024; i += 256) {
        // slot ((rb * 4 + cb) * 4 + a4) * 64 + lane, lane (r, h): token 32 cb + r, weight
        // rows 32 rb + 8 a4 + 4 h + (0..3)
        const int lane = i & 63, a4 = (i >> 6) & 3, rb = i >> 8;
        const int slot = ((rb * 4 + cb) * 4 + a4) * 64 + lane;
        float4 v = src[slot];
        for (int sp = 1; sp < nsplit; ++sp) {
            const float4 t = src[sp * per_split + slot];
            v.x += t.x;
            v.y += t.y;
            v.z += t.z;
            v.w += t.w;
        }
        const int r = lane & 31, h = lane >> 5;
        *reinterpret_cast<float4 *>(&st[r * kReducePitch + 32 * rb + 8 * a4 + 4 * h]) = v;
    }
    __syncthreads();
    const int64_t n0 = static_cast<int64_t>(tt % tiles_n) * (128 * WR) + 128 * wn;
    const bool vec4 = ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(c) & 15u) == 0;
    for (int i = threadIdx.x; i < 32 * 32; i += 256) {
        const int tok = i >> 5, c4 = i & 31;
        const int64_t m = m0 + tok;
        if (m >= M) continue;
        const float4 v = *reinterpret_cast<const float4 *>(&st[tok * kReducePitch + 4 * c4]);
        const float accv[4] = {v.x, v.y, v.z, v.w};
        const int64_t nb = n0 + 4 * c4;
        float *cr = c + m * ldc;
        float y[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int64_t n = nb + b;
            float t = alpha * accv[b];
            if (n < N) {
                if (beta != 0.0f) t = t + beta * cr[n];
                if (bias != nullptr) t = t + bias[n];
            }
            y[b] = t;
        }
        if (vec4 && nb + 3 < N) {
            *reinterpret_cast<float4 *>(cr + nb) = make_float4(y[0], y[1], y[2], y[3]);
        } else {
#pragma unroll
            for (int b = 0; b < 4; ++b)
                if (nb + b < N) cr[nb + b] = y[b];
        }
    }
}

// Weight rows that run as whole rounds of 256 x 256 tiles, one workgroup per CU at a
// time: all of them, none (fewer than 160 tiles: the GPU would be mostly idle), or,
// when the last round would be at most half full, the rows of the whole rounds only.
int64_t gemm_rows_whole_rounds(int64_t m, int64_t n) {
    const int64_t tiles_m = (m + kW4Tokens - 1) / kW4Tokens;
    const int64_t tiles_big = ((n + kW4Rows - 1) / kW4Rows) * tiles_m;
    if (tiles_big < 160) return 0;
    const int64_t cus = cu_count();
    const int64_t rem = tiles_big % cus;
    const int64_t n1 = (tiles_big - rem) / tiles_m * kW4Rows;
    if (tiles_big > cus && rem != 0 && 2 * rem <= cus && n1 > 0 && n1 < n) return n1;
    return n;
}

// Half-width tiles (256 weight rows x 128 tokens) over rows: their count, and whether
// the rows [n1, n) left after whole rounds of big tiles run as one round of them -- three
// quarters of the CUs or more, none waiting for a second round -- instead of as split-K
// items (no workspace, no second launch).  Only after whole rounds: a half-width step
// costs about as much outside its MFMAs as a whole one (the same 128 weight rows per wave
// to decode), so with no whole tiles to run beside them (Llama down at M = 2048, every
// row) they measured slower than split-K (199 -> 222 us); as gate_up's remainder at
// M = 2048 they replace the split items and their sum (388 -> 382 us).
int64_t gemm_half_tiles(int64_t m, int64_t rows) {
    return ((rows + kW4Rows - 1) / kW4Rows) * ((m + kW4Tokens / 2 - 1) / (kW4Tokens / 2));
}
bool gemm_use_half(int64_t m, int64_t n, int64_t n1) {
    const int64_t t = gemm_half_tiles(m, n - n1);
    const int64_t cus = cu_count();
    return n1 > 0 && n1 < n && m > 64 && t <= cus && 4 * t >= 3 * cus;
}

// How the big-tile kernel splits K for a shape: with few tiles (< 160), about one
// workgroup per CU in total, at least four k-steps per split.  nsplit == 1: no split.
struct SplitPlan {
    int64_t nsplit, sps, tiles;
};
SplitPlan gemm_split_plan(int64_t m, int64_t n, int64_t k) {
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t nsteps = (L + 1) / 2;
    const int64_t tiles = ((n + kW4Rows - 1) / kW4Rows) * ((m + kW4Tokens - 1) / kW4Tokens);
    SplitPlan p{1, nsteps, tiles};
    if (m <= 64 || tiles >= 160 || tiles <= 0) return p;
    int64_t ns = (cu_count() + tiles / 2) / tiles;
    if (ns > nsteps / 4) ns = nsteps / 4;
    if (ns < 2) return p;
    p.sps = (nsteps + ns - 1) / ns;
    p.nsplit = (nsteps + p.sps - 1) / p.sps;
    return p;
}
int64_t split_workspace_bytes(const SplitPlan &p) {
    return p.nsplit > 1 ? p.nsplit * p.tiles * kW4Rows * kW4Tokens * 4 : 0;
}

// 384 x 128 tiles (three 32-row blocks per wave, the waves along the rows: the RB = 3,
// WR = 4 instance) when a shape has fewer 256 x 256 tiles than CUs but 160 or more (no
// split), and its 384 x 128 tiles still fit one round: every CU then runs one tile of
// about three quarters the work instead of three quarters of the CUs one tile each (qkv
// at M = 2048: 192 -> 256 tiles).  The 2 x 2 form of the same tiles (192 x 256) measured
// slower: qkv M = 2048 83.2 -> 80.7 us, with beta = 1 95.4 -> 89.8 us, 3072 -> 3072 at
// M = 4096 66.2 -> 64.7 us, a ragged 2000 x 4104 -> 6000 95.9 -> 90.9 us.
bool gemm_use_384(int64_t m, int64_t n, int64_t k) {
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t t4 = ((n + kW4Rows - 1) / kW4Rows) * ((m + kW4Tokens - 1) / kW4Tokens);
    const int64_t t3 = ((n + 383) / 384) * ((m + 127) / 128);
    const int64_t cus = cu_count();
    return m > 64 && t4 >= 160 && t4 < cus && t3 <= cus &&
           int64_t(384) * L * kTrytes < 0x7FFFFFFF;
}
hipError_t launch_gemm_w4_384(const void *x, const uint8_t *w, void *c, int64_t m, int64_t n,
                              int64_t ldc, int64_t k, float alpha, float beta, const float *bias,
                              hipStream_t s) {
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t items = ((n + 383) / 384) * ((m + 127) / 128);
    const int64_t cus = cu_count();
    auto kernel = beta != 0.0f ? gemm_w4_kernel<kDtypeBF16, 3, true, 4>
                               : gemm_w4_kernel<kDtypeBF16, 3, false, 4>;
    kernel<<<dim3(items < cus ? items : cus), dim3(kW4Threads), 0, s>>>(
        x, w, c, static_cast<int>(m), static_cast<int>(n), static_cast<int>(ldc),
        static_cast<int>(k), static_cast<int>(L), alpha, beta, bias, static_cast<int>(n), 0,
        nullptr, 0, 0);
    return hipGetLastError();
}

// Rows [0, n1) of W as whole big tiles and, with plan != nullptr (nsplit > 1) and part
// (room for the plan's partial tiles), rows [n1, n) as split-K items, in one launch;
// then the split partials are summed into C.  With half, rows [n1, n) run instead as
// half-width tiles (256 rows x 128 tokens, all k-steps) in the same launch.  C rows are
// ldc elements apart.
hipError_t launch_gemm_w4(const void *x, const uint8_t *w, void *c, int64_t m, int64_t n,
                          int64_t n1, int64_t ldc, int64_t k, float alpha, float beta,
                          const float *bias, hipStream_t s, const SplitPlan *plan = nullptr,
                          void *part = nullptr, bool half = false) {
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t tiles_m = (m + kW4Tokens - 1) / kW4Tokens;
    const bool split = !half && plan != nullptr && plan->nsplit > 1 && part != nullptr && n1 < n;
    const bool rem = half && n1 < n;
    const int64_t items = ((n1 + kW4Rows - 1) / kW4Rows) * tiles_m +
                          (split ? plan->nsplit * plan->tiles : 0) +
                          (rem ? gemm_half_tiles(m, n - n1) : 0);
    if (items <= 0) return hipSuccess;
    const int64_t cus = cu_count();
    // (split items store raw sums: beta is applied by the split sum, and the whole tiles of
    // the same launch take the kBeta instance)
    auto kernel = beta != 0.0f ? gemm_w4_kernel<kDtypeBF16, 4, true>
                               : gemm_w4_kernel<kDtypeBF16, 4, false>;
    kernel<<<dim3(items < cus ? items : cus), dim3(kW4Threads), 0, s>>>(
        x, w, c, static_cast<int>(m), static_cast<int>(split || rem ? n : n1),
        static_cast<int>(ldc), static_cast<int>(k), static_cast<int>(L), alpha, beta, bias,
        static_cast<int>(n1), split ? static_cast<int>(plan->sps) : 0,
        static_cast<float4 *>(part), split ? static_cast<int>(plan->nsplit) : 0, rem ? 1 : 0);
    if (!split) return hipGetLastError();
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t tiles = plan->tiles;
    gemm_split_reduce_kernel<2><<<dim3(static_cast<unsigned>(tiles * 16)), dim3(256), 0, s>>>(
        static_cast<const float4 *>(part), static_cast<float *>(c) + n1, m, n - n1, ldc,
        static_cast<int>(tiles), static_cast<int>(plan->nsplit), alpha, beta,
        bias ? bias + n1 : nullptr);
    return hipGetLastError();
}

}  // namespace

// Tall tiles (the big-tile kernels' WR = 4 instances: 512 weight rows x 128 tokens) for
// shapes with at least a round of them: when whole rounds cover the rows, or whole rounds
// and then one round of their 512 x 64 half-width tiles (three quarters of the CUs or
// more), as for 256 x 256 tiles.  Otherwise (fewer tiles, or a remainder that fits
// neither) the 256 x 256 rules below.  Also needs the 32-bit buffer offsets of a
// workgroup's 512 weight rows.
bool gemm_tall_plan(int64_t m, int64_t n, int64_t k, int64_t *n1_out, bool *half_out) {
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t cus = cu_count();
    const int64_t tiles_m = (m + 127) / 128;
    const int64_t tiles = ((n + 511) / 512) * tiles_m;
    if (m <= 64 || tiles < cus || int64_t(512) * L * kTrytes >= 0x7FFFFFFF) return false;
    const int64_t rem = tiles % cus;
    if (rem == 0) {
        *n1_out = n;
        *half_out = false;
        return true;
    }
    const int64_t n1 = (tiles - rem) / tiles_m * 512;
    if (n1 <= 0 || n1 >= n) return false;
    const int64_t t = ((n - n1 + 511) / 512) * ((m + 63) / 64);
    if (t > cus || 4 * t < 3 * cus) return false;
    *n1_out = n1;
    *half_out = true;
    return true;
}
namespace {

hipError_t launch_gemm_w4_tall(const void *x, const uint8_t *w, void *c, int64_t m, int64_t n,
                               int64_t n1, bool half, int64_t k, float alpha, float beta,
                               const float *bias, hipStream_t s) {
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t items = ((n1 + 511) / 512) * ((m + 127) / 128) +
                          (half ? ((n - n1 + 511) / 512) * ((m + 63) / 64) : 0);
    const int64_t cus = cu_count();
    auto kernel = beta != 0.0f ? gemm_w4_kernel<kDtypeBF16, 4, true, 4>
                               : gemm_w4_kernel<kDtypeBF16, 4, false, 4>;
    kernel<<<dim3(items < cus ? items : cus), dim3(kW4Threads), 0, s>>>(
        x, w, c, static_cast<int>(m), static_cast<int>(n), static_cast<int>(n),
        static_cast<int>(k), static_cast<int>(L), alpha, beta, bias, static_cast<int>(n1), 0,
        nullptr, 0, half ? 1 : 0);
    return hipGetLastError();
}

// Split-K over tall tiles, for shapes whose rows all split (fewer than 160 big tiles): the
// plan of gemm_split_plan over 512 x 128 tiles, each split item storing its raw sums as a
// 2 x 2 item does (1 KB per wave per block), summed by gemm_split_reduce_kernel<4>.  Half
// the tile loads per step, the same partial traffic: down 14336 -> 4096 at M = 2048 193.9
// -> 189.2 us, at M = 512 69.3 -> 68.5 us, qkv at M = 512 the same (43.5 us); bit-identical
// to the 2 x 2 split (each output's splits hold the same k-steps).
SplitPlan gemm_split_plan_tall(int64_t m, int64_t n, int64_t k) {
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t nsteps = (L + 1) / 2;
    const int64_t tiles = ((n + 511) / 512) * ((m + 127) / 128);
    SplitPlan p{1, nsteps, tiles};
    if (m <= 64 || tiles >= 160 || tiles <= 0 || int64_t(512) * L * kTrytes >= 0x7FFFFFFF)
        return p;
    int64_t ns = (cu_count() + tiles / 2) / tiles;
    if (ns > nsteps / 4) ns = nsteps / 4;
    if (ns < 2) return p;
    p.sps = (nsteps + ns - 1) / ns;
    p.nsplit = (nsteps + p.sps - 1) / p.sps;
    return p;
}
hipError_t launch_gemm_w4_tall_split(const void *x, const uint8_t *w, void *c, int64_t m,
                                     int64_t n, int64_t k, float alpha, float beta,
                                     const float *bias, hipStream_t s, const SplitPlan &plan,
                                     void *part) {
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t items = plan.nsplit * plan.tiles;
    const int64_t cus = cu_count();
    const dim3 grid(static_cast<unsigned>(items < cus ? items : cus));
    gemm_w4_kernel<kDtypeBF16, 4, false, 4><<<grid, dim3(kW4Threads), 0, s>>>(
        x, w, c, static_cast<int>(m), static_cast<int>(n), static_cast<int>(n),
        static_cast<int>(k), static_cast<int>(L), alpha, beta, bias, 0,
        static_cast<int>(plan.sps), static_cast<float4 *>(part), static_cast<int>(plan.nsplit), 0);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    gemm_split_reduce_kernel<4><<<dim3(static_cast<unsigned>(plan.tiles * 16)), dim3(256), 0, s>>>(
        static_cast<const float4 *>(part), static_cast<float *>(c), m, n, n,
        static_cast<int>(plan.tiles), static_cast<int>(plan.nsplit), alpha, beta, bias);
    return hipGetLastError();
}

// C from the splits of the eight-wave kernel: sums part[0..nsplit) (row-major M x N
// each) in split order -- int32 exactly for int8 activations -- then applies alpha,
// beta and bias as the kernel's epilogue does.  C rows are ldc elements apart.
template <int XT>
__global__ __launch_bounds__(256) void gemm_split_sum_kernel(
    const void *__restrict__ part, void *__restrict__ c, int64_t M, int64_t N, int64_t ldc,
    int nsplit, float alpha, float beta, const float *__restrict__ bias) {
    const int64_t total = M * N;
    for (int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; g < total;
         g += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t m = g / N;
        const int64_t n = g - m * N;
        if constexpr (XT == kDtypeI8) {
            const int32_t *p = static_cast<const int32_t *>(part);
            int32_t y = p[g];
            for (int sp = 1; sp < nsplit; ++sp) y += p[sp * total + g];
            int32_t *cp = static_cast<int32_t *>(c) + m * ldc + n;
            if (beta != 0.0f) y += *cp;
            *cp = y;
        } else {
            const float *p = static_cast<const float *>(part);
            float v = p[g];
            for (int sp = 1; sp < nsplit; ++sp) v += p[sp * total + g];
            float *cp = static_cast<float *>(c) + m * ldc + n;
            float y = alpha * v;
            if (beta != 0.0f) y = y + beta * *cp;
            if (bias != nullptr) y = y + bias[n];
            *cp = y;
        }
    }
}

// K split for a launch of `tiles` workgroups over `nsteps` k-steps: about per_cu
// workgroups per CU in total, at least two k-steps per split; nsplit == 1: no split.
SplitPlan small_split_plan(int64_t tiles, int64_t nsteps, int64_t per_cu = 1) {
    SplitPlan p{1, nsteps, tiles};
    if (tiles <= 0 || tiles >= 128) return p;
    int64_t ns = (per_cu * cu_count() + tiles / 2) / tiles;
    if (ns > nsteps / 2) ns = nsteps / 2;
    if (ns < 2) return p;
    p.sps = (nsteps + ns - 1) / ns;
    p.nsplit = (nsteps + p.sps - 1) / p.sps;
    return p;
}

template <int XT, int RN, int CM, int WN, int WM, int LK>
SplitPlan gemm_t_plan(int64_t m, int64_t n, int64_t k) {
    using Cfg = GemmCfg<XT, RN, CM, WN, WM, LK>;
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t tiles = ((n + Cfg::kBN - 1) / Cfg::kBN) * ((m + Cfg::kBM - 1) / Cfg::kBM);
    // 32-token tiles over wide N (>= 64 tiles): two workgroups per CU, whose partials
    // are small at this M (llama.gate_up M = 32: 47 -> 35 us); the 128-row tiles of a long
    // K (gemm_small_rows) too; elsewhere one.
    const bool two = (CM == 1 && tiles >= 64) || (RN == 1 && LK == 4);
    return small_split_plan(tiles, (L + LK - 1) / LK, two ? 2 : 1);
}

// Up to 64 tokens over a long K: the eight-wave kernel takes four limbs per k-step instead
// of two, so each step's loads (issued one step ahead) meet twice the MFMA work and a launch
// waits at half as many barriers.  A sweep of two, four and six limbs (float32 at 17..64
// tokens, bf16 at 49 and 64) on 14336 -> 4096, 11008 -> 4096, 8192 -> 3072, 8192 -> 8192:
// four wins over K = 14336 (float32 M = 17 29.9 -> 25.1 us, M = 32 34.6 -> 30.9, M = 64
// 48.7 -> 45.9; bf16 M = 49 34.4 -> 29.4, M = 64 35.8 -> 31.0) and K = 8192 at <= 32
// tokens (M = 17 on 8192 -> 8192 31.4 -> 27.6), not at 33..64 tokens over K = 8192 (8192 ->
// 3072 M = 64 30.9 -> 31.6) nor over K = 4096 (4096 -> 6144 M = 48 22.3 -> 34.8, the
// float32 tiles then fill 102 KB of LDS and a CU holds one workgroup); six measured slower
// than four except on 8192 -> 8192.  At <= 32 tokens the same form (with the 128-row tiles
// below) also wins over a short K on 8192 or more rows (float32 4096 -> 14336 at 17 / 32
// tokens 26.5 / 29.0 -> 21.7 / 25.4 us, 3072 -> 9216 18.6 / 20.5 -> 15.8 / 18.6, 3072 ->
// 16384 19.0 / 22.9 -> 18.9 / 23.2) and loses on 4096 -> 6144 (14.8 / 15.8 -> 16.2 / 19.1)
// and 4096 -> 4096 (12.8 / 14.0 -> 14.2 / 16.4).
bool gemm_small_long_k(int64_t m, int64_t n, int64_t k) {
    return m <= 32 ? k >= 8192 || n >= 8192 : k > 8192;
}

// On that path, 128-row tiles (two workgroups per CU) instead of 256-row ones where the
// 256-row grid has fewer than 64 tiles: more workgroups share the K split, and two per CU
// hide each other's step latency.  Not for float32 at 33..64 tokens, whose 64-token tiles
// of two planes already fill 102 KB of LDS (14336 -> 4096 at 64 tokens 45.9 -> 63.5 us).
// Same box, against 256-row tiles: bf16 14336 -> 4096 at 49 / 64 tokens 29.3 / 31.0 ->
// 25.9 / 26.8 us, 11008 -> 4096 23.9 / 25.1 -> 23.7 / 23.4; float32 at 17 / 32 tokens
// 14336 -> 4096 25.2 / 31.1 -> 24.0 / 27.2, 8192 -> 8192 27.7 / 32.7 -> 24.8 / 28.2,
// 8192 -> 3072 18.1 / 21.1 -> 17.1 / 19.5.
template <int XT>
bool gemm_small_rows(int64_t m, int64_t n) {
    return (XT != kDtypeF32 || m <= 32) && n < 64 * 256;
}

// Rows [0, n) of W and columns [0, n) of C, whose rows are ldc elements apart.  With a
// workspace of at least nsplit * m * n * 4 bytes, a launch of few tiles splits K.
template <int XT, int RN, int CM, int WN, int WM, int LK>
hipError_t launch_gemm_t(const void *x, const uint8_t *w, void *c, int64_t m, int64_t n,
                         int64_t ldc, int64_t k, float alpha, float beta, const float *bias,
                         hipStream_t s, void *ws = nullptr, int64_t ws_bytes = 0) {
    using Cfg = GemmCfg<XT, RN, CM, WN, WM, LK>;
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t tiles = ((n + Cfg::kBN - 1) / Cfg::kBN) * ((m + Cfg::kBM - 1) / Cfg::kBM);
    const int elem = XT == kDtypeF32 ? 4 : (XT == kDtypeBF16 ? 2 : 1);
    const bool aligned = (k % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % (8 * elem) == 0);
    SplitPlan plan{1, (L + LK - 1) / LK, tiles};
    void *part = nullptr;
    if (ws != nullptr) {
        const SplitPlan p = gemm_t_plan<XT, RN, CM, WN, WM, LK>(m, n, k);
        if (p.nsplit > 1 && ws_bytes >= p.nsplit * m * n * 4) {
            plan = p;
            part = ws;
        }
    }
    const dim3 grid(static_cast<unsigned>(tiles * plan.nsplit));
    if (aligned)
        gemm_kernel<XT, RN, CM, WN, WM, LK, true><<<grid, dim3(Cfg::kThreads), 0, s>>>(
            x, w, c, m, n, ldc, k, L, alpha, beta, bias, plan.sps, part);
    else
        gemm_kernel<XT, RN, CM, WN, WM, LK, false><<<grid, dim3(Cfg::kThreads), 0, s>>>(
            x, w, c, m, n, ldc, k, L, alpha, beta, bias, plan.sps, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || part == nullptr) return e;
    const int64_t total = m * n;
    const int64_t blocks = (total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096;
    gemm_split_sum_kernel<XT><<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(
        part, c, m, n, ldc, static_cast<int>(plan.nsplit), alpha, beta, bias);
    return hipGetLastError();
}

// ---- float32 activations past 64 tokens, given a workspace ----
// The tokens are cut into equal chunks; each chunk is split into its bf16 planes in the
// workspace (x = hi + lo, hi = bf16(x), lo = bf16(x - hi), |x - hi - lo| <= 2^-18 |x|),
// and the chunk's rows of C are two bf16 launches: C = alpha * hi T + beta * C + bias,
// then C = alpha * lo T + C.  The bf16 launches run the big-tile kernel, against the
// float32 eight-wave kernel that stages both planes for 256 x 128 tiles: gate_up M = 2048
// 1604 -> 794 us, M = 8192 6701 -> 3100, M = 512 456 -> 220; qkv M = 2048 458 -> 203.
// A chunk's two planes fit kF32PlaneBytes (so the workspace stays within the
// no-allocation entry's static scratch), and the path is taken only where the bf16
// launches of its chunks need no split-K workspace of their own: with one (down 14336 ->
// 4096 at M = 2048: 1024-token chunks of 64 tiles) the two launches measured slower than
// the eight-wave kernel (834 -> 1126 us), as at 65 tokens.
constexpr int64_t kF32PlaneBytes = int64_t{64} << 20;

template <int XT>
int64_t gemm_workspace_x(int64_t m, int64_t n, int64_t k);

struct F32Chunks {
    int64_t rows = 0;    // tokens per chunk (the last may hold fewer)
    int64_t count = 0;   // 0: the planes path does not take the shape
};

F32Chunks f32_chunks(int64_t m, int64_t n, int64_t k) {
    F32Chunks ch;
    if (m <= 64 || k % 8 != 0 || n <= 0) return ch;
    const int64_t cap = kF32PlaneBytes / (4 * k);   // tokens whose planes fit
    if (cap < 256) return ch;
    const int64_t count = (m + cap - 1) / cap;
    const int64_t rows = (m + count - 1) / count;
    const int64_t last = m - (count - 1) * rows;
    if (gemm_workspace_x<kDtypeBF16>(rows, n, k) != 0 ||
        gemm_workspace_x<kDtypeBF16>(last, n, k) != 0)
        return ch;
    ch.rows = rows;
    ch.count = count;
    return ch;
}

// The workspace the planes path needs (0: it does not take the shape).
int64_t f32_planes_bytes(int64_t m, int64_t n, int64_t k) {
    const F32Chunks ch = f32_chunks(m, n, k);
    return ch.count > 0 ? 4 * ch.rows * k : 0;
}

__global__ __launch_bounds__(256) void f32_planes_kernel(const float *__restrict__ x,
                                                         uint32_t *__restrict__ hi,
                                                         uint32_t *__restrict__ lo,
                                                         int64_t pairs) {
    // pairs of consecutive values (K % 8 == 0 keeps a pair inside a row)
    for (int64_t p = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; p < pairs;
         p += static_cast<int64_t>(gridDim.x) * 256) {
        const float f0 = x[2 * p], f1 = x[2 * p + 1];
        const __bf16 h0 = static_cast<__bf16>(f0), h1 = static_cast<__bf16>(f1);
        const __bf16 l0 = static_cast<__bf16>(f0 - static_cast<float>(h0));
        const __bf16 l1 = static_cast<__bf16>(f1 - static_cast<float>(h1));
        hi[p] = __builtin_bit_cast(uint16_t, h0) |
                (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h1)) << 16);
        lo[p] = __builtin_bit_cast(uint16_t, l0) |
                (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, l1)) << 16);
    }
}

template <int XT>
hipError_t launch_gemm_x(const void *x, const uint8_t *w, void *c, int64_t m, int64_t n,
                         int64_t k, float alpha, float beta, const float *bias, hipStream_t s,
                         void *ws, int64_t ws_bytes);

hipError_t launch_gemm_f32_planes(const float *x, const uint8_t *w, float *c, int64_t m,
                                  int64_t n, int64_t k, float alpha, float beta,
                                  const float *bias, hipStream_t s, void *ws) {
    const int64_t mc = f32_chunks(m, n, k).rows;
    uint16_t *hi = static_cast<uint16_t *>(ws);
    for (int64_t t0 = 0; t0 < m; t0 += mc) {
        const int64_t rows = m - t0 < mc ? m - t0 : mc;
        uint16_t *lo = hi + rows * k;
        const int64_t pairs = rows * k / 2;
        int64_t blocks = (pairs + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        f32_planes_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(
            x + t0 * k, reinterpret_cast<uint32_t *>(hi), reinterpret_cast<uint32_t *>(lo), pairs);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        float *cc = c + t0 * n;
        e = launch_gemm_x<kDtypeBF16>(hi, w, cc, rows, n, k, alpha, beta, bias, s, nullptr, 0);
        if (e != hipSuccess) return e;
        e = launch_gemm_x<kDtypeBF16>(lo, w, cc, rows, n, k, alpha, 1.0f, nullptr, s, nullptr, 0);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <int XT>
hipError_t launch_gemm_x(const void *x, const uint8_t *w, void *c, int64_t m, int64_t n,
                         int64_t k, float alpha, float beta, const float *bias, hipStream_t s,
                         void *ws, int64_t ws_bytes) {
    constexpr int LK = 2;  // limbs per k-step
    if constexpr (XT == kDtypeF32) {
        const int64_t planes = f32_planes_bytes(m, n, k);
        if (planes > 0 && ws != nullptr && ws_bytes >= planes &&
            reinterpret_cast<uintptr_t>(ws) % 16 == 0)
            return launch_gemm_f32_planes(static_cast<const float *>(x), w,
                                          static_cast<float *>(c), m, n, k, alpha, beta, bias, s,
                                          ws);
    }
    if constexpr (XT == kDtypeBF16 || XT == kDtypeI8) {
        // 17..64 tokens, aligned: the column-block stream kernel of K2 (gemv.hip)
        bool handled = false;
        const hipError_t e = launch_gemv_column_blocks(&handled, x, XT, w, c, static_cast<int>(m),
                                                       n, k, alpha, beta, bias, s);
        if (handled || e != hipSuccess) return e;
    }
    // 17..64 tokens that the column-block kernel does not take (float32, long K, unaligned
    // x): the eight-wave kernel, four limbs per k-step over a long K, or over many rows at
    // <= 32 tokens (gemm_small_long_k)
    if (m <= 64 && gemm_small_long_k(m, n, k)) {
        const bool rows128 = gemm_small_rows<XT>(m, n);
        if (m <= 32)
            return rows128 ? launch_gemm_t<XT, 1, 1, 4, 1, 2 * LK>(x, w, c, m, n, n, k, alpha, beta,
                                                                   bias, s, ws, ws_bytes)
                           : launch_gemm_t<XT, 2, 1, 4, 1, 2 * LK>(x, w, c, m, n, n, k, alpha, beta,
                                                                   bias, s, ws, ws_bytes);
        return rows128 ? launch_gemm_t<XT, 1, 2, 4, 1, 2 * LK>(x, w, c, m, n, n, k, alpha, beta,
                                                               bias, s, ws, ws_bytes)
                       : launch_gemm_t<XT, 2, 2, 4, 1, 2 * LK>(x, w, c, m, n, n, k, alpha, beta,
                                                               bias, s, ws, ws_bytes);
    }
    if (m <= 32)
        return launch_gemm_t<XT, 2, 1, 4, 1, LK>(x, w, c, m, n, n, k, alpha, beta, bias, s, ws,
                                                 ws_bytes);
    if (m <= 64)
        return launch_gemm_t<XT, 2, 2, 4, 1, LK>(x, w, c, m, n, n, k, alpha, beta, bias, s, ws,
                                                 ws_bytes);
    if constexpr (XT == kDtypeI8) {
        // int8 activations on the integer matrix cores (gemm_i8.hip) when the shape allows
        if (gemm_i8_fits(x, m, n, k))
            return launch_gemm_i8(x, w, static_cast<int32_t *>(c), m, n, k, beta != 0.0f, s, ws,
                                  ws_bytes);
    }
    if constexpr (XT != kDtypeF32) {
        // Rows [0, n1): whole rounds of 256 x 256 tiles -- the one-wave-per-SIMD kernel
        // for bf16, else the eight-wave kernel (two waves per SIMD).  Rows [n1, n) (all
        // of them when there are few tiles, the remainder that would leave the last round
        // at most half full otherwise): split-K over big tiles when the caller gave a
        // workspace, else 256 x 128 tiles of the eight-wave kernel.
        const int64_t n1 = gemm_rows_whole_rounds(m, n);
        const int64_t L = (k + kTrits - 1) / kTrits;
        const bool w4 = XT == kDtypeBF16 && gemm_w4_fits(x, m, n, k);
        int64_t tn1 = 0;
        bool thalf = false;
        if (w4 && gemm_tall_plan(m, n, k, &tn1, &thalf))
            // one launch of 512 x 128 tiles for rows [0, tn1), 512 x 64 for the rest
            return launch_gemm_w4_tall(x, w, c, m, n, tn1, thalf, k, alpha, beta, bias, s);
        if (w4 && gemm_use_384(m, n, k))
            return launch_gemm_w4_384(x, w, c, m, n, n, k, alpha, beta, bias, s);
        if (w4 && gemm_use_half(m, n, n1))
            // one launch: whole tiles for rows [0, n1), one round of half-width tiles for
            // the rest
            return launch_gemm_w4(x, w, c, m, n, n1, n, k, alpha, beta, bias, s, nullptr, nullptr,
                                  true);
        if (w4 && ws != nullptr && n1 == 0) {
            // every row split over the workspace: tall split-K items, then their sum
            const SplitPlan tp = gemm_split_plan_tall(m, n, k);
            if (tp.nsplit > 1 && ws_bytes >= split_workspace_bytes(tp))
                return launch_gemm_w4_tall_split(x, w, c, m, n, k, alpha, beta, bias, s, tp, ws);
        }
        if (w4 && ws != nullptr && n1 < n) {
            // one launch: whole tiles for rows [0, n1), split-K items for the rest
            const SplitPlan plan = gemm_split_plan(m, n - n1, k);
            if (plan.nsplit > 1 && ws_bytes >= split_workspace_bytes(plan))
                return launch_gemm_w4(x, w, c, m, n, n1, n, k, alpha, beta, bias, s, &plan, ws);
        }
        if (n1 > 0) {
            const hipError_t e =
                w4 ? launch_gemm_w4(x, w, c, m, n1, n1, n, k, alpha, beta, bias, s)
                   : launch_gemm_t<XT, 2, 4, 4, 2, LK>(x, w, c, m, n1, n, k, alpha, beta, bias, s);
            if (e != hipSuccess || n1 == n) return e;
        }
        const uint8_t *w_rest = w + n1 * L * kTrytes;
        void *c_rest = static_cast<uint8_t *>(c) + 4 * n1;
        const float *bias_rest = bias ? bias + n1 : nullptr;
        return launch_gemm_t<XT, 2, 2, 4, 2, LK>(x, w_rest, c_rest, m, n - n1, n, k, alpha, beta,
                                               bias_rest, s, ws, ws_bytes);
    }
    // fp32 activations: two LDS planes; four waves with 256 x 128 tiles
    return launch_gemm_t<XT, 2, 4, 4, 1, LK>(x, w, c, m, n, n, k, alpha, beta, bias, s, ws,
                                             ws_bytes);
}

}  // namespace

hipError_t launch_gemm(const void *x, int x_dtype, const uint8_t *w, void *c, int64_t m,
                       int64_t n, int64_t k, float alpha, float beta, const float *bias,
                       hipStream_t s, void *ws, int64_t ws_bytes) {
    if (m == 0 || n == 0) return hipSuccess;
    switch (x_dtype) {
        case kDtypeBF16:
            return launch_gemm_x<kDtypeBF16>(x, w, c, m, n, k, alpha, beta, bias, s, ws, ws_bytes);
        case kDtypeF32:
            return launch_gemm_x<kDtypeF32>(x, w, c, m, n, k, alpha, beta, bias, s, ws, ws_bytes);
        default:
            return launch_gemm_x<kDtypeI8>(x, w, c, m, n, k, alpha, beta, bias, s, ws, ws_bytes);
    }
}

namespace {

// Workspace of an eight-wave launch over m x n: nsplit row-major m x n partials.
template <int XT, int RN, int CM, int WN, int WM, int LK = 2>
int64_t gemm_t_workspace(int64_t m, int64_t n, int64_t k) {
    const SplitPlan p = gemm_t_plan<XT, RN, CM, WN, WM, LK>(m, n, k);
    return p.nsplit > 1 ? p.nsplit * m * n * 4 : 0;
}

template <int XT>
int64_t gemm_workspace_x(int64_t m, int64_t n, int64_t k) {
    if constexpr (XT == kDtypeF32) {
        // the bf16 planes of float32 activations past 64 tokens (f32_planes_bytes), or the
        // eight-wave kernel's split where a misaligned workspace leaves the planes out
        const int64_t planes = f32_planes_bytes(m, n, k);
        if (planes > 0) {
            const int64_t eight = gemm_t_workspace<XT, 2, 4, 4, 1>(m, n, k);
            return planes > eight ? planes : eight;
        }
    }
    if (m <= 64 && gemm_small_long_k(m, n, k)) {
        const bool rows128 = gemm_small_rows<XT>(m, n);
        if (m <= 32)
            return rows128 ? gemm_t_workspace<XT, 1, 1, 4, 1, 4>(m, n, k)
                           : gemm_t_workspace<XT, 2, 1, 4, 1, 4>(m, n, k);
        return rows128 ? gemm_t_workspace<XT, 1, 2, 4, 1, 4>(m, n, k)
                       : gemm_t_workspace<XT, 2, 2, 4, 1, 4>(m, n, k);
    }
    if (m <= 32) return gemm_t_workspace<XT, 2, 1, 4, 1>(m, n, k);
    if (m <= 64) return gemm_t_workspace<XT, 2, 2, 4, 1>(m, n, k);
    if constexpr (XT == kDtypeF32) {
        return gemm_t_workspace<XT, 2, 4, 4, 1>(m, n, k);
    } else {
        // the rows after whole rounds of big tiles: split-K big tiles (bf16, aligned
        // activations) or eight-wave 256 x 128 tiles; the larger of the two
        int64_t i8 = 0;
        if constexpr (XT == kDtypeI8) {
            // the integer big-tile kernel's split-K plan (K % 16 == 0), or the eight-wave
            // kernel's when the activations turn out misaligned; the larger of the two
            if (k % 16 == 0) i8 = gemm_i8_workspace_bytes(m, n, k);
        }
        const int64_t n1 = gemm_rows_whole_rounds(m, n);
        if (n1 == n) return i8;
        const int64_t eight = gemm_t_workspace<XT, 2, 2, 4, 2>(m, n - n1, k);
        if constexpr (XT == kDtypeI8) return eight > i8 ? eight : i8;
        if constexpr (XT != kDtypeBF16) return eight;
        // aligned activations whose remaining rows fill a round of half-width tiles run
        // without a workspace
        int64_t big = k % 8 == 0 && !gemm_use_half(m, n, n1)
                          ? split_workspace_bytes(gemm_split_plan(m, n - n1, k))
                          : 0;
        if (k % 8 == 0 && n1 == 0) {
            // (the tall split's plan, which its tile count can change)
            const int64_t t = split_workspace_bytes(gemm_split_plan_tall(m, n, k));
            if (t > big) big = t;
        }
        return big > eight ? big : eight;
    }
}

}  // namespace

int64_t gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int x_dtype) {
    if (m <= 0 || n <= 0 || k <= 0) return 0;
    switch (x_dtype) {
        case kDtypeBF16:
            // the column-block stream kernel's shapes (17..gemv_column_blocks_max_tokens
            // tokens, K % 8 == 0): no workspace
            if (m >= 17 && m <= gemv_column_blocks_max_tokens(k, x_dtype) && k % 8 == 0)
                return 0;
            return gemm_workspace_x<kDtypeBF16>(m, n, k);
        case kDtypeF32: return gemm_workspace_x<kDtypeF32>(m, n, k);
        default:
            // int8 the same with K % 16 == 0
            if (m >= 17 && m <= gemv_column_blocks_max_tokens(k, x_dtype) && k % 16 == 0)
                return 0;
            return gemm_workspace_x<kDtypeI8>(m, n, k);
    }
}

}  // namespace t81hip

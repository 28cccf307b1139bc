// t81lib_amd/csrc/gemv.hip -- K2: decode-shaped ternary matmul (M <= 16 tokens).
//
//   C[m, n] = alpha * sum_k X[m, k] * T[n, k] + beta * C[m, n] + bias[n]
//
// launch_gemv sends M <= 4 to the column-strip kernel (gemv_strip.hip); the kernels
// here take M = 5 .. 16 and the shapes the strip kernel declines.
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
#include <algorithm>

#include "gemv_common.hpp"
#include "t81_device.hpp"
#include "t81_kernels.hpp"

namespace t81hip {

namespace {

// Applies alpha / beta / bias to a finished 16x16 tile and stores it.  Lane (m, q)
// holds rows n0 + 4q + i (i < 4) of token m.
template <int XT>
__device__ __forceinline__ void store_tile_rq(floatx4 v, int r, int q, int M, int64_t N,
                                              int64_t n0, void *c, float alpha, float beta,
                                              const float *bias) {
    if (r >= M) return;
    const int64_t nb = n0 + 4 * q;
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

template <int XT>
__device__ __forceinline__ void store_tile(floatx4 v, int lane, int M, int64_t N, int64_t n0,
                                           void *c, float alpha, float beta, const float *bias) {
    store_tile_rq<XT>(v, lane & 15, lane >> 4, M, N, n0, c, alpha, beta, bias);
}

// Sums the per-wave partial tiles of G 16-row groups and stores them.  kSplit: B column
// 2 t holds token t's hi plane and 2 t + 1 its lo plane; the two are added (the lane
// pair next to each other) and the even lane stores token t.
template <int XT, int G, int KS, bool kSplit = false>
__device__ __forceinline__ void reduce_store(floatx4 (&acc)[G], floatx4 *red, int wave, int lane,
                                             int M, int64_t N, int64_t n0, void *c, float alpha,
                                             float beta, const float *bias) {
#pragma unroll
    for (int g = 0; g < G; ++g) red[(wave * G + g) * 64 + lane] = acc[g];
    __syncthreads();
    for (int g = wave; g < G; g += KS) {
        floatx4 v = red[g * 64 + lane];
#pragma unroll
        for (int ww = 1; ww < KS; ++ww) v += red[(ww * G + g) * 64 + lane];
        if constexpr (kSplit) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] += __shfl_xor(v[e], 1);
            if ((lane & 1) == 0)
                store_tile_rq<XT>(v, (lane & 15) >> 1, lane >> 4, M, N, n0 + 16 * g, c, alpha,
                                  beta, bias);
        } else {
            store_tile<XT>(v, lane, M, N, n0 + 16 * g, c, alpha, beta, bias);
        }
    }
}

// ---------------------------------------------------------------------------------
// gemv_wave_kernel: a workgroup of W waves covers G = W / Wg 16-row groups, Wg waves
// per group, each wave a contiguous run of nsbw <= R 4-limb sub-blocks of its
// group's K (up to 12 KB of weights).  Everything a wave needs up to the final
// reduction is private to it, so there is no barrier before the stream:
//   1. raw loads of the activations of its K range (M rows, zero past K), then
//      R weight loads, one per sub-block: all of them are in flight before the
//      first is used.  The count is a template constant, so the compiler counts
//      outstanding loads exactly (a load issued under a condition would make every
//      later wait a full drain); a wave with nsbw < R points the spare loads past
//      the buffer's range, where they return zeros without touching memory;
//   2. its own copy of the decode tables and of its activations in LDS (bf16;
//      fp32 as hi and lo planes; int8 exactly), ordered against its own reads by a
//      wavefront fence;
//   3. per sub-block: decode from the tables, six MFMAs;
//   4. partial tiles summed through LDS per group (one barrier), wave order fixed.
// Tokens m >= M: their lanes read activation row 0.  Column m of the MFMA result
// depends only on column m of B, and those columns are never stored.
// Weights come through a buffer resource based at the group's first row: the
// hardware range check returns zeros past the end of the matrix (rows >= N).
// Limbs past L at the end of a row read the next row's first limbs; their
// activations are staged as zero and every byte decodes to 0 or +-1, so they add
// exactly nothing.
template <int XT>
struct WaveLayout {
    static constexpr int kPlanes = XT == kDtypeF32 ? 2 : 1;
    static constexpr int kElem = XT == kDtypeF32 ? 4 : (XT == kDtypeBF16 ? 2 : 1);
    static constexpr int kChunkVals = 16 / kElem;                // activations per load
    static constexpr int kChunksPerSb = 4 * kTrits / kChunkVals;  // loads per sub-block row
};

constexpr int kSbBytes = 4 * kTrits * 2;  // one staged sub-block row: 192 bf16
constexpr int kMaxRun = 12;               // sub-blocks per wave
constexpr int kDepth = 4;                 // weight loads in flight per wave
constexpr int kMaxChunksPerLane = 8;      // activation loads per lane, all in flight at once
constexpr uint32_t kOobOffset = 0x80000000u;

// Per-wave LDS: planes x M rows x pitch; pitch = nsbw_max sub-blocks plus 16 bytes,
// which moves consecutive rows to other banks.
__host__ __device__ inline int wave_pitch(int nsbw_max) { return nsbw_max * kSbBytes + 16; }
__host__ __device__ inline int wave_lds_bytes(int M, int nsbw_max, int planes) {
    return planes * M * wave_pitch(nsbw_max);
}

// bf16 activations of one 4-limb sub-block (16 tokens x 192 values) through a wave's own
// LDS region.  Loaded as B fragments, lane (r, q) reads 16 bytes of token r, so each
// 16-lane pass of a load touches 16 token rows and the address unit handles a cache line
// per row; loaded as pieces, piece p = 64 i + lane (token p / 24, values 8 (p % 24) ..
// + 8), a pass reads consecutive bytes of one or two rows.  The pieces go to LDS (rows of
// 400 bytes, so the fragment reads of 16 lanes spread over the banks) and come back as the
// fragments: llama.down at 16 tokens 17.0 -> 14.3 us.  Requires K % 8 == 0 and x 16-byte
// aligned; tokens >= M and values past K are zero.
constexpr int kXStagePitch = 4 * kTrits * 2 + 16;
constexpr int kXStageBytes = 16 * kXStagePitch;   // per wave

__device__ __forceinline__ void load_x_pieces(const void *x, int M, int64_t K, int64_t sb,
                                              int64_t S, int lane, u32x4 (&xp)[6]) {
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        const int p = 64 * i + lane;
        const int t = p / 24;
        const int64_t k = sb * (4 * kTrits) + 8 * (p - 24 * t);
        const bool ok = t < M && sb < S && k < K;   // sub-block sb of S exists
        const uint8_t *src = ok ? static_cast<const uint8_t *>(x) + (t * K + k) * 2
                                : reinterpret_cast<const uint8_t *>(kZeroBlock);
        xp[i] = *reinterpret_cast<const u32x4 *>(src);
    }
}

// Writes the pieces to the wave's region xs and reads back lane (r, q)'s six fragments
// (values 48 q + 8 j .. + 8 of token r).  The wave's own LDS operations complete in order,
// so no barrier: a later call's writes come after this call's reads.
template <typename T>
__device__ __forceinline__ void stage_x_pieces(uint8_t *xs, int lane, const u32x4 (&xp)[6],
                                               T (&frag)[6]) {
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        const int p = 64 * i + lane;
        const int t = p / 24;
        *reinterpret_cast<u32x4 *>(xs + t * kXStagePitch + 16 * (p - 24 * t)) = xp[i];
    }
    const int r = lane & 15;
    const int q = lane >> 4;
#pragma unroll
    for (int j = 0; j < 6; ++j)
        frag[j] = *reinterpret_cast<const T *>(xs + r * kXStagePitch + 96 * q + 16 * j);
}

template <int XT, int W, int SU, int R>
__global__ __launch_bounds__(64 * W) void gemv_wave_kernel(
    const void *__restrict__ x, const uint8_t *__restrict__ w, void *__restrict__ c, int M,
    int64_t N, int64_t K, int L, int nsb, int wg, int nsbw_max, uint32_t cpr_magic,
    int x_aligned, float alpha, float beta, const float *__restrict__ bias) {
    using LY = WaveLayout<XT>;
    constexpr int kElem = LY::kElem;
    constexpr int CV = LY::kChunkVals;
    __shared__ __attribute__((aligned(16))) uint8_t lut[kLutBytes];
    __shared__ __attribute__((aligned(16))) floatx4 red[W * 64];
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave-uniform, and known to be: every quantity derived from it stays scalar and
    // every condition on it is a scalar branch
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15;
    const int q = lane >> 4;
    const int G = W / wg;
    const int g = wave / wg;
    const int p = wave - g * wg;
    const int64_t group = static_cast<int64_t>(blockIdx.x) * G + g;
    const int64_t groups = (N + 15) / 16;
    const int64_t n0 = group * 16;
    const int s0 = (p * nsb) / wg;
    const int nsbw = group < groups ? ((p + 1) * nsb) / wg - s0 : 0;
    const int pitch = wave_pitch(nsbw_max);
    const int plane_bytes = M * pitch;
    uint8_t *xs = smem + wave * wave_lds_bytes(M, nsbw_max, LY::kPlanes);

    // ---- 1a. activation chunks of this wave: u = m * cpr + cc ----
    const int cpr = nsbw_max * LY::kChunksPerSb;
    const int chunks = M * cpr;
    const int cc_end = nsbw * LY::kChunksPerSb;
    const int64_t kbase = static_cast<int64_t>(s0) * 4 * kTrits;
    const uint8_t *xb8 = static_cast<const uint8_t *>(x);
    const uint8_t *zero8 = reinterpret_cast<const uint8_t *>(kZeroBlock);
    auto load_chunks = [&](int base, u32x4 (&raw)[SU]) {
#pragma unroll
        for (int i = 0; i < SU; ++i) {
            const int u = base + lane + 64 * i;
            const int m = static_cast<int>(__umulhi(static_cast<uint32_t>(u), cpr_magic));
            const int cc = u - m * cpr;
            const bool ok = u < chunks && cc < cc_end;
            const int64_t k0 = kbase + static_cast<int64_t>(cc) * CV;
            if (x_aligned) {  // K % CV == 0: a chunk lies wholly inside K or wholly past it
                const uint8_t *ptr = ok && k0 < K ? xb8 + (m * K + k0) * kElem : zero8;
                raw[i] = *reinterpret_cast<const u32x4 *>(ptr);
            } else {
                uint32_t e[CV];
#pragma unroll
                for (int v = 0; v < CV; ++v) {
                    const uint8_t *ptr =
                        ok && k0 + v < K ? xb8 + (m * K + k0 + v) * kElem : zero8;
                    if constexpr (kElem == 4) e[v] = *reinterpret_cast<const uint32_t *>(ptr);
                    else if constexpr (kElem == 2) e[v] = *reinterpret_cast<const uint16_t *>(ptr);
                    else e[v] = *ptr;
                }
                uint32_t wd[4];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    if constexpr (kElem == 4) wd[d] = e[d];
                    else if constexpr (kElem == 2) wd[d] = e[2 * d] | (e[2 * d + 1] << 16);
                    else
                        wd[d] = e[4 * d] | (e[4 * d + 1] << 8) | (e[4 * d + 2] << 16) |
                                (e[4 * d + 3] << 24);
                }
                raw[i] = u32x4{wd[0], wd[1], wd[2], wd[3]};
            }
        }
    };
    auto stage_chunks = [&](int base, const u32x4 (&raw)[SU]) {
#pragma unroll
        for (int i = 0; i < SU; ++i) {
            const int u = base + lane + 64 * i;
            if (u < chunks) {
                const int m = static_cast<int>(__umulhi(static_cast<uint32_t>(u), cpr_magic));
                uint8_t *dst = xs + m * pitch + (u - m * cpr) * (CV * 2);
                if constexpr (XT == kDtypeBF16) {
                    *reinterpret_cast<u32x4 *>(dst) = raw[i];
                } else if constexpr (XT == kDtypeF32) {
                    // x = hi + lo, hi = bf16(x), lo = bf16(x - hi): |x - hi - lo| <= 2^-18 |x|
                    uint32_t h[4], l[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float f = __uint_as_float(raw[i][e]);
                        h[e] = bf16_bits_rne(f);
                        l[e] = bf16_bits_rne(f - bf16_bits_to_float(h[e]));
                    }
                    *reinterpret_cast<uint2 *>(dst) =
                        make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
                    *reinterpret_cast<uint2 *>(dst + plane_bytes) =
                        make_uint2(l[0] | (l[1] << 16), l[2] | (l[3] << 16));
                } else {  // int8 -> bf16, exact
                    uint32_t o[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const uint32_t wd0 = raw[i][e / 2];
                        const int8_t b0 = static_cast<int8_t>((wd0 >> (16 * (e % 2))) & 0xFFu);
                        const int8_t b1 =
                            static_cast<int8_t>((wd0 >> (16 * (e % 2) + 8)) & 0xFFu);
                        o[e] = bf16_bits_rne(static_cast<float>(b0)) |
                               (bf16_bits_rne(static_cast<float>(b1)) << 16);
                    }
                    reinterpret_cast<u32x4 *>(dst)[0] = u32x4{o[0], o[1], o[2], o[3]};
                    reinterpret_cast<u32x4 *>(dst)[1] = u32x4{o[4], o[5], o[6], o[7]};
                }
            }
        }
    };

    // ---- 1b. weights: every sub-block of the run, issued before any is used ----
    const int64_t remain = group < groups ? (N - n0) * L * kTrytes : 0;
    const int nrec = remain < 0x7FFFFFFF ? static_cast<int>(remain) : 0x7FFFFFFF;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(group < groups ? w + n0 * L * kTrytes : w), 0, nrec, 0x00020000);
    const uint32_t lane_base = static_cast<uint32_t>((r * L + 4 * s0 + q) * kTrytes);

    u32x4 raw[SU];
    load_chunks(0, raw);
    constexpr int D = R < kDepth ? R : kDepth;
    u32x4 ring[D];  // sub-block f lives in ring[f % D]
    auto fetch = [&](int f) -> u32x4 {
        const uint32_t off = f < nsbw ? lane_base + 64u * static_cast<uint32_t>(f) : kOobOffset;
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
    };
#pragma unroll
    for (int i = 0; i < D; ++i) ring[i] = fetch(i);

    // ---- 2. decode tables (shared, at a fixed address: lookups need no base add),
    //         then this wave's activations into its own LDS ----
    lut_fill(lut, tid, 64 * W);
    __syncthreads();
    stage_chunks(0, raw);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- 3. stream: lane (r, q) pairs row r of the group with token row r ----
    // Two accumulators (even / odd MFMAs of a sub-block) halve the dependency chain.
    const uint8_t *xl = xs + (r < M ? r : 0) * pitch + q * (kTrits * 2);
    floatx4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int f = 0; f < R; ++f) {
        uint32_t pairs[24];
        if (f < nsbw) {
#pragma unroll
            for (int d = 0; d < 4; ++d) decode_dword(lut, ring[f % D][d], pairs + 6 * d);
        }
        // the refill reuses the slot's registers once they are decoded; its count
        // is fixed at compile time, so the loads stay counted exactly
        __builtin_amdgcn_sched_barrier(0);
        if (f + D < R) ring[f % D] = fetch(f + D);
        if (f < nsbw) {
            const uint8_t *src = xl + f * kSbBytes;
            bf16x8 bh[6], bl[6];
#pragma unroll
            for (int j = 0; j < 6; ++j) {
                bh[j] = *reinterpret_cast<const bf16x8 *>(src + 16 * j);
                if constexpr (XT == kDtypeF32)
                    bl[j] = *reinterpret_cast<const bf16x8 *>(src + plane_bytes + 16 * j);
            }
            mfma_pairs2<XT>(pairs, bh, bl, acc0, acc1);
        }
    }

    // ---- 4. per group: sum the wg partial tiles, one element per thread ----
    red[wave * 64 + lane] = acc0 + acc1;
    __syncthreads();
    const float *redf = reinterpret_cast<const float *>(red);
    for (int t = tid; t < G * 256; t += 64 * W) {
        const int gg = t >> 8;
        const int e = t & 255;
        const int64_t n0g = (static_cast<int64_t>(blockIdx.x) * G + gg) * 16;
        float v = redf[(gg * wg) * 256 + e];
        for (int pp = 1; pp < wg; ++pp) v += redf[(gg * wg + pp) * 256 + e];
        const int le = e >> 2;  // lane of the tile that held element e
        const int m = le & 15;
        const int64_t n = n0g + 4 * (le >> 4) + (e & 3);
        if (m < M && n < N) {
            if constexpr (XT == kDtypeI8) {
                int32_t *cp = static_cast<int32_t *>(c) + static_cast<int64_t>(m) * N + n;
                int32_t y = static_cast<int32_t>(v);
                if (beta != 0.0f) y += *cp;
                *cp = y;
            } else {
                float *cp = static_cast<float *>(c) + static_cast<int64_t>(m) * N + n;
                float y = alpha * v;
                if (beta != 0.0f) y = y + beta * *cp;
                if (bias != nullptr) y = y + bias[n];
                *cp = y;
            }
        }
    }
}

// ---------------------------------------------------------------------------------
// gemv_stream_kernel: for M * K too large to stage, activations come straight from
// global memory, fetched one sub-block ahead and issued before the weight prefetch
// (so waiting for them never drains the weight loads).  The KS waves of a workgroup
// split K round-robin; each activation fragment serves its G 16-row groups.  kStage
// (bf16, kAligned): the activations of a sub-block are loaded as pieces and become
// fragments through the wave's LDS region (load_x_pieces).
template <int XT, int G, bool kAligned, int KS, bool kStage, bool kDeep = false,
          bool kSplit = false>
__global__ __launch_bounds__(64 * KS) void gemv_stream_kernel(const void *__restrict__ x,
                                                          const uint8_t *__restrict__ w,
                                                          void *__restrict__ c, int M, int64_t N,
                                                          int64_t K, int64_t L, float alpha,
                                                          float beta,
                                                          const float *__restrict__ bias) {
    static_assert(!kStage || ((XT == kDtypeBF16 || XT == kDtypeI8 || kSplit) && kAligned),
                  "pieces are aligned bf16, int8 widened to bf16 as they are staged, or "
                  "float32 split into two columns");
    static_assert(!kDeep || kStage, "two sub-blocks in flight: the staged form only");
    static_assert(!kSplit || (XT == kDtypeF32 && kStage && !kDeep),
                  "planes as columns: float32, staged");
    // a piece: 16 bytes of one token's activations, 8 bf16, 16 int8 or 4 float32 values
    // (the int8 launch also needs K % 16 == 0 and a 16-byte aligned x; float32, K % 4 ==
    // 0).  kSplit (float32, up to 8 tokens): token t's piece becomes 4 bf16 of its hi plane
    // in staging row 2 t and 4 of its lo plane in row 2 t + 1, so the B operand's 16
    // columns are 8 tokens' two planes and one MFMA serves both.
    constexpr int kVals = XT == kDtypeI8 ? 16 : (kSplit ? 4 : 8);
    constexpr int kPieces = 4 * kTrits / kVals;        // per token and sub-block: 24, 12, 48
    constexpr int kTok = kSplit ? 8 : 16;              // tokens with pieces
    constexpr int kLanePieces = kTok * kPieces / 64;   // per lane: 6 or 3
    constexpr int kElemB = XT == kDtypeI8 ? 1 : (kSplit ? 4 : 2);
    constexpr int XM = kSplit ? kDtypeBF16 : XT;       // the MFMA's operand type
    __shared__ __attribute__((aligned(16))) uint8_t lut[kLutBytes];
    __shared__ __attribute__((aligned(16))) floatx4 red[KS * G * 64];
    __shared__ __attribute__((aligned(16))) uint8_t xst[kStage ? KS * kXStageBytes : 16];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int r = lane & 15;
    const int q = lane >> 4;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * (16 * G);
    const int64_t S = (L + 3) / 4;

    const bool xvalid = r < M;
    const int64_t xrow = static_cast<int64_t>(r) * K;
    bf16x8 bh[6], bl[6], nh[6], nl[6];
    u32x4 xp[6];
    uint8_t *xs = xst + wave * kXStageBytes;
    // load_x_pieces and stage_x_pieces written out here: the compiler schedules this
    // form's piece loads earlier among the MFMAs (llama.gate M = 16 12.35 us against 12.94)
    auto load_pieces = [&](int64_t sb) {
#pragma unroll
        for (int i = 0; i < kLanePieces; ++i) {
            const int P = 64 * i + lane;
            const int t = P / kPieces;
            const int64_t k = sb * (4 * kTrits) + kVals * (P - kPieces * t);
            const bool ok = t < M && sb < S && k < K;
            const uint8_t *src = ok ? static_cast<const uint8_t *>(x) + (t * K + k) * kElemB
                                    : reinterpret_cast<const uint8_t *>(kZeroBlock);
            xp[i] = *reinterpret_cast<const u32x4 *>(src);
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < kLanePieces; ++i) {
            const int P = 64 * i + lane;
            const int t = P / kPieces;
            if constexpr (kSplit) {
                // 4 float32 -> 4 bf16 of the hi plane (row 2 t) and 4 of the lo plane
                uint8_t *dst = xs + 2 * t * kXStagePitch + 8 * (P - kPieces * t);
                uint32_t h[2], l[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const float f0 = __uint_as_float(xp[i][2 * e]);
                    const float f1 = __uint_as_float(xp[i][2 * e + 1]);
                    const __bf16 h0 = static_cast<__bf16>(f0), h1 = static_cast<__bf16>(f1);
                    const __bf16 l0 = static_cast<__bf16>(f0 - static_cast<float>(h0));
                    const __bf16 l1 = static_cast<__bf16>(f1 - static_cast<float>(h1));
                    h[e] = __builtin_bit_cast(uint16_t, h0) |
                           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h1)) << 16);
                    l[e] = __builtin_bit_cast(uint16_t, l0) |
                           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, l1)) << 16);
                }
                *reinterpret_cast<uint2 *>(dst) = make_uint2(h[0], h[1]);
                *reinterpret_cast<uint2 *>(dst + kXStagePitch) = make_uint2(l[0], l[1]);
                continue;
            }
            uint8_t *dst = xs + t * kXStagePitch + 16 * (kVals / 8) * (P - kPieces * t);
            if constexpr (XT == kDtypeI8) {
                // 16 int8 -> 16 bf16 (exact: |v| <= 128 needs 8 significant bits)
                uint32_t h[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t wd = xp[i][e / 2];
                    const int sh = 16 * (e % 2);
                    const float f0 = static_cast<float>(static_cast<int8_t>((wd >> sh) & 0xFFu));
                    const float f1 =
                        static_cast<float>(static_cast<int8_t>((wd >> (sh + 8)) & 0xFFu));
                    h[e] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xFFFF0000u);
                }
                *reinterpret_cast<u32x4 *>(dst) = u32x4{h[0], h[1], h[2], h[3]};
                *reinterpret_cast<u32x4 *>(dst + 16) = u32x4{h[4], h[5], h[6], h[7]};
            } else {
                *reinterpret_cast<u32x4 *>(dst) = xp[i];
            }
        }
#pragma unroll
        for (int j = 0; j < 6; ++j)
            bh[j] = *reinterpret_cast<const bf16x8 *>(xs + r * kXStagePitch + 96 * q + 16 * j);
    };
    int64_t s = wave;
    if constexpr (kDeep) {
        // Two sub-blocks in flight.  Iteration i (sub-block s_i = wave + i KS): issue the
        // pieces of s_{i+2} into slot i % 2 (whose pieces of s_i were staged the iteration
        // before), run the MFMAs of s_i with the weights in slot i % 2 (loaded two
        // iterations ago), load the weights of s_{i+2} into that slot, then stage the
        // pieces of s_{i+1} (issued an iteration ago): every load has two iterations to
        // land, and no register of a load in flight is copied.  Two iterations per pass
        // keep the slots static.  (Fencing the loads at the top of the iteration with
        // sched_barrier measured slower: llama.down M = 8 12.6 -> 13.2 us.)
        floatx4 acc[G];
#pragma unroll
        for (int g = 0; g < G; ++g) acc[g] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 6; ++j) bl[j] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
        u32x4 xa[6], xb[6];
        u32x4 wa[G], wb[G];
        auto pieces_to = [&](int64_t sb, u32x4 (&dst)[6]) {
            load_pieces(sb);
#pragma unroll
            for (int i = 0; i < kLanePieces; ++i) dst[i] = xp[i];
        };
        auto stage_from = [&](const u32x4 (&src)[6]) {
#pragma unroll
            for (int i = 0; i < kLanePieces; ++i) xp[i] = src[i];
            stage();
        };
        auto weights_to = [&](int64_t sb, u32x4 (&dst)[G]) {
#pragma unroll
            for (int g = 0; g < G; ++g) dst[g] = load_limb(w, n0 + 16 * g + r, 4 * sb + q, N, L, L);
        };
        pieces_to(s, xa);
        weights_to(s, wa);
        pieces_to(s + KS, xb);
        weights_to(s + KS, wb);
        lut_init(lut, tid, 64 * KS);
        stage_from(xa);
        auto iter = [&](int64_t si, u32x4 (&xs_now)[6], u32x4 (&xs_next)[6], u32x4 (&wn)[G]) {
            pieces_to(si + 2 * KS, xs_now);
#pragma unroll
            for (int g = 0; g < G; ++g) acc[g] = mfma_limb<XM>(lut, wn[g], bh, bl, acc[g]);
            weights_to(si + 2 * KS, wn);
            stage_from(xs_next);
        };
        for (; s < S; s += 2 * KS) {
            iter(s, xa, xb, wa);
            if (s + KS >= S) break;
            iter(s + KS, xb, xa, wb);
        }
        reduce_store<XT, G, KS, kSplit>(acc, red, wave, lane, M, N, n0, c, alpha, beta, bias);
        return;
    }
    if constexpr (kStage) {
        load_pieces(s);
#pragma unroll
        for (int j = 0; j < 6; ++j) bl[j] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
    } else {
#pragma unroll
        for (int j = 0; j < 6; ++j)
            load_x8<XT, kAligned>(x, xrow, (4 * s + q) * kTrits + 8 * j, K,
                                  xvalid && (4 * s + q) < L, bh[j], bl[j]);
    }
    u32x4 wcur[G];
#pragma unroll
    for (int g = 0; g < G; ++g) wcur[g] = load_limb(w, n0 + 16 * g + r, 4 * s + q, N, L, L);
    lut_init(lut, tid, 64 * KS);
    if constexpr (kStage) stage();

    floatx4 acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = floatx4{0.f, 0.f, 0.f, 0.f};

    for (; s < S; s += KS) {
        const int64_t sn = s + KS;
        if constexpr (kStage) {
            load_pieces(sn);
        } else {
#pragma unroll
            for (int j = 0; j < 6; ++j)
                load_x8<XT, kAligned>(x, xrow, (4 * sn + q) * kTrits + 8 * j, K,
                                      xvalid && sn < S && (4 * sn + q) < L, nh[j], nl[j]);
        }
        u32x4 wnext[G];
#pragma unroll
        for (int g = 0; g < G; ++g) wnext[g] = load_limb(w, n0 + 16 * g + r, 4 * sn + q, N, L, L);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            acc[g] = mfma_limb<XM>(lut, wcur[g], bh, bl, acc[g]);
            wcur[g] = wnext[g];
        }
        if constexpr (kStage) {
            stage();
        } else {
#pragma unroll
            for (int j = 0; j < 6; ++j) {
                bh[j] = nh[j];
                bl[j] = nl[j];
            }
        }
    }
    reduce_store<XT, G, KS, kSplit>(acc, red, wave, lane, M, N, n0, c, alpha, beta, bias);
}

// ---------------------------------------------------------------------------------
// gemv_tile_kernel: 5..16 tokens fill the 16 columns of every MFMA tile, so one load of
// 16 rows x 4 limbs (16 bytes per lane) yields a whole 16 x 16 block of partial sums,
// and the activations it meets -- 16 tokens x 192 trits, six 16-byte fragments per
// lane -- are the same for every 16-row group.  So a wave owns one 4-limb sub-block of
// K for its whole life: that sub-block's activations are loaded once, stay in
// registers as the B operand, and R row groups stream through them (6 KB of activation
// reads per wave against R KB of weights, where the stream kernel above reads them
// again for every one or two row groups).
//
// Workgroup (row block b, split p): R row groups (16R rows) x NW consecutive
// sub-blocks, wave w taking sub-block p * NW + w.  Each load is a new row group, so it
// gets its own accumulator; the loads run four in flight, each slot refilled as soon
// as it is decoded, the table reads of load t + 1 issued before the MFMAs of load t
// (the column-strip kernel's pipeline).  At the end the NW partial tiles of each row
// group are summed through LDS in wave order.  With one split the workgroup applies
// alpha, beta and bias and stores C; with P > 1 splits it stores its raw sums to the
// caller's workspace (one M x N row-major matrix per split) and gemv_split_sum_kernel
// adds the splits in split order.  Every sum has a fixed order.
//
// Lane (r, q): A = limb 4 * sb + q of row 16 t + r of the block (load t); B = the
// activations of token r for the same limb (zeros for r >= M or past K).  A limb past L
// reads zeros (outside the buffer range), which decode to finite trits and meet zero
// activations; rows past N read zeros and are not stored.  Waves whose sub-block is
// past the last one (the last split of a K that is not a multiple of NW sub-blocks)
// load nothing and contribute zero tiles.
template <int XT, int NW, int R>
__global__ __launch_bounds__(64 * NW) void gemv_tile_kernel(
    const void *__restrict__ x, const uint8_t *__restrict__ w, void *__restrict__ c, int M,
    int64_t N, int64_t K, int L, int nsb, int nb, int x_aligned, float alpha, float beta,
    const float *__restrict__ bias, float *__restrict__ part) {
    constexpr int D = R < kDepth ? R : kDepth;
    // aligned bf16 activations are staged through the wave's LDS region (load_x_pieces);
    // the regions are dead past the start barrier, and the reduction reuses the space
    constexpr int kRedBytes = NW * R * 64 * 16;
    constexpr int kStageBytes = XT == kDtypeBF16 ? NW * kXStageBytes : 0;
    __shared__ __attribute__((aligned(16))) uint8_t lut[kLutBytes];
    __shared__ __attribute__((aligned(16)))
    uint8_t smem[kStageBytes > kRedBytes ? kStageBytes : kRedBytes];
    floatx4 *red = reinterpret_cast<floatx4 *>(smem);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15;
    const int q = lane >> 4;
    const int b = static_cast<int>(blockIdx.x % static_cast<unsigned>(nb));
    const int p = static_cast<int>(blockIdx.x / static_cast<unsigned>(nb));
    const int64_t row0 = static_cast<int64_t>(b) * 16 * R;
    const int sb = p * NW + wave;  // wave-uniform
    const bool active = sb < nsb;
    const int limb = 4 * sb + q;
    const bool in_row = active && limb < L;

    floatx4 acc[R];
#pragma unroll
    for (int t = 0; t < R; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};

    // Weights through a buffer based at the block's first row: rows past N read zeros.
    const int64_t remain = (N - row0) * L * kTrytes;
    const int nrec = remain < 0x7FFFFFFF ? static_cast<int>(remain) : 0x7FFFFFFF;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(w + row0 * L * kTrytes), 0, nrec, 0x00020000);
    const uint32_t row_bytes = static_cast<uint32_t>(L) * kTrytes;
    const uint32_t lane_off =
        static_cast<uint32_t>(r) * row_bytes + static_cast<uint32_t>(limb) * kTrytes;
    auto fetch = [&](int t) -> u32x4 {
        const uint32_t off =
            in_row ? lane_off + 16u * static_cast<uint32_t>(t) * row_bytes : kOobOffset;
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
    };

    XRaw xr[6];
    u32x4 xp[6];
    u32x4 ring[D];  // load t lives in ring[t % D]
    if (active) {
        // B: the activations of token r for the lane's limb, issued before the weights
        const bool bvalid = r < M && in_row;
        const int64_t xrow = static_cast<int64_t>(r < M ? r : 0) * K;
        const int64_t kb = static_cast<int64_t>(limb) * kTrits;
        if (XT == kDtypeBF16 && x_aligned) {
            load_x_pieces(x, M, K, sb, nsb, lane, xp);
        } else if (x_aligned) {
#pragma unroll
            for (int j = 0; j < 6; ++j) xr[j] = load_x8_raw<XT, true>(x, xrow, kb + 8 * j, K, bvalid);
        } else {
#pragma unroll
            for (int j = 0; j < 6; ++j) xr[j] = load_x8_raw<XT, false>(x, xrow, kb + 8 * j, K, bvalid);
        }
#pragma unroll
        for (int t = 0; t < D; ++t) ring[t] = fetch(t);
    }
    lut_fill(lut, tid, 64 * NW);
    if constexpr (XT == kDtypeBF16) {
        if (active && x_aligned) {
            // the barrier's wait for LDS operations ends every wave's fragment reads
            // before any wave writes the reduction into the same space
            u32x4 frag[6];
            stage_x_pieces(smem + wave * kXStageBytes, lane, xp, frag);
#pragma unroll
            for (int j = 0; j < 6; ++j) xr[j].a = frag[j];
        }
    }
    __syncthreads();

    if (active) {
        bf16x8 bh[6], bl[6];
#pragma unroll
        for (int j = 0; j < 6; ++j) cvt_x8<XT>(xr[j], bh[j], bl[j]);
        uint32_t cur[24], nxt[24];
#pragma unroll
        for (int d = 0; d < 4; ++d) decode_dword(lut, ring[0][d], cur + 6 * d);
        __builtin_amdgcn_sched_barrier(0);
        if (D < R) ring[0] = fetch(D);
#pragma unroll
        for (int t = 0; t < R; ++t) {
            if (t + 1 < R) {
#pragma unroll
                for (int d = 0; d < 4; ++d) decode_dword(lut, ring[(t + 1) % D][d], nxt + 6 * d);
                __builtin_amdgcn_sched_barrier(0);
                if (t + 1 + D < R) ring[(t + 1) % D] = fetch(t + 1 + D);
            }
            acc[t] = mfma_pairs<XT>(cur, bh, bl, acc[t]);
#pragma unroll
            for (int e = 0; e < 24; ++e) cur[e] = nxt[e];
        }
    }

    // ---- per row group: the NW partial tiles summed in wave order ----
#pragma unroll
    for (int t = 0; t < R; ++t) red[(wave * R + t) * 64 + lane] = acc[t];
    __syncthreads();
    for (int e = tid; e < R * 64; e += 64 * NW) {
        const int t = e >> 6;
        const int l = e & 63;
        floatx4 v = red[t * 64 + l];
#pragma unroll
        for (int ww = 1; ww < NW; ++ww) v += red[(ww * R + t) * 64 + l];
        const int64_t n0 = row0 + 16 * t;
        if (part == nullptr) {
            store_tile<XT>(v, l, M, N, n0, c, alpha, beta, bias);
        } else {
            // lane l of the tile holds rows n0 + 4 (l / 16) + i of token l % 16
            const int m = l & 15;
            if (m >= M) continue;
            const int64_t nb4 = n0 + 4 * (l >> 4);
            float *dst = part + (static_cast<int64_t>(p) * M + m) * N + nb4;
            if (nb4 + 3 < N && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
                *reinterpret_cast<float4 *>(dst) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (nb4 + i < N) dst[i] = v[i];
            }
        }
    }
}

// C from the P split partials of gemv_tile_kernel (M x N row-major each, raw sums):
// summed in split order, then alpha, beta and bias as store_tile applies them.  For
// int8 activations every partial and every sum is an integer below 2^24 in magnitude
// (K <= 131071), so the float sums are exact and convert to int32 exactly.
template <int XT>
__global__ __launch_bounds__(256) void gemv_split_sum_kernel(
    const float *__restrict__ part, void *__restrict__ c, int M, int64_t N, int P, float alpha,
    float beta, const float *__restrict__ bias) {
    const int64_t total = static_cast<int64_t>(M) * N;
    const int64_t quads = (N + 3) / 4;   // four consecutive outputs of one row per thread
    const bool vec = N % 4 == 0;         // then every quad is 16-byte aligned (part, C)
    for (int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; g < M * quads;
         g += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t m = g / quads;
        const int64_t n0 = (g - m * quads) * 4;
        const int64_t base = m * N + n0;
        const int cnt = N - n0 < 4 ? static_cast<int>(N - n0) : 4;
        float v[4];
        if (vec) {
            // four partials loaded at a time (all in flight), then added in split order
            auto ld = [&](int sp) {
                return *reinterpret_cast<const float4 *>(part + sp * total + base);
            };
            float4 a = ld(0);
            int sp = 1;
            for (; sp + 4 <= P; sp += 4) {
                const float4 b[4] = {ld(sp), ld(sp + 1), ld(sp + 2), ld(sp + 3)};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    a.x += b[j].x;
                    a.y += b[j].y;
                    a.z += b[j].z;
                    a.w += b[j].w;
                }
            }
            for (; sp < P; ++sp) {
                const float4 b = ld(sp);
                a.x += b.x;
                a.y += b.y;
                a.z += b.z;
                a.w += b.w;
            }
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        } else {
            for (int i = 0; i < cnt; ++i) {
                float t = part[base + i];
                for (int sp = 1; sp < P; ++sp) t += part[sp * total + base + i];
                v[i] = t;
            }
        }
        for (int i = 0; i < cnt; ++i) {
            if constexpr (XT == kDtypeI8) {
                int32_t *cp = static_cast<int32_t *>(c) + base + i;
                int32_t y = static_cast<int32_t>(v[i]);
                if (beta != 0.0f) y += *cp;
                *cp = y;
            } else {
                float *cp = static_cast<float *>(c) + base + i;
                float y = alpha * v[i];
                if (beta != 0.0f) y = y + beta * *cp;
                if (bias != nullptr) y = y + bias[n0 + i];
                *cp = y;
            }
        }
    }
}

// The tile kernel's plan for a shape: NW waves (sub-blocks) per workgroup, P splits of K,
// R row groups per workgroup -- four, fewer where the grid would not give every CU a
// workgroup (a plan sweep on the config-3/4 shapes at 16 tokens: eight waves and four
// row groups were best or within 5 % of best on each).  P depends on K alone, so the
// order of every sum is a function of the shape.
struct TilePlan {
    int nw, r, p;
    int64_t nb;
};
TilePlan gemv_tile_plan(int64_t n, int64_t k) {
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t nsb = (L + 3) / 4;
    TilePlan t;
    t.nw = nsb <= 4 ? 4 : 8;
    t.p = static_cast<int>((nsb + t.nw - 1) / t.nw);
    const int64_t groups = (n + 15) / 16;
    const int64_t cus = cu_count();
    t.r = 4;
    while (t.r > 1 && (groups + t.r - 1) / t.r * t.p < cus) t.r /= 2;
    t.nb = (groups + t.r - 1) / t.r;
    return t;
}

// Whether the tile kernel takes this call, and the workspace its splits need.  Its time
// hardly depends on M, and its K splits end in a second launch (about 3 us on top of the
// main kernel at 16 tokens); measured against the stream / wave kernels with fragment
// loads it is faster for 9..16 tokens over a long K (>= 32 sub-blocks) and at most 8192
// rows -- 14336 -> 4096 at 16 tokens 22.5 -> 17.6 us, 8192 -> 3072 13.7 -> 10.1 us --
// and slower on the wide and short-K config-3/4 shapes, which keep those kernels.  bf16
// activations with K % 8 == 0 and 16-byte aligned x take the stream kernel with staged
// pieces instead (launch_gemv_tile declines them).
bool gemv_tile_fits(int m, int64_t n, int64_t k) {
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t nsb = (L + 3) / 4;
    // buffer offsets within a block (16 R rows, R <= 4) stay below 2^31; grid and
    // split indices fit the kernel's ints
    return m >= 9 && m <= 16 && n > 0 && n <= 8192 && nsb >= 32 &&
           int64_t{64} * L * kTrytes < 0x7FFFFFFF && (n + 15) / 16 * nsb < (int64_t{1} << 30);
}

int64_t gemv_tile_workspace_bytes(int m, int64_t n, int64_t k) {
    if (!gemv_tile_fits(m, n, k)) return 0;
    const TilePlan t = gemv_tile_plan(n, k);
    return t.p > 1 ? int64_t{4} * t.p * m * n : 0;
}

template <int XT, int NW, int R>
hipError_t launch_tile_r(const TilePlan &t, const void *x, const uint8_t *w, void *c, int m,
                         int64_t n, int64_t k, bool aligned, float alpha, float beta,
                         const float *bias, float *part, hipStream_t s) {
    const int L = static_cast<int>((k + kTrits - 1) / kTrits);
    const int nsb = (L + 3) / 4;
    gemv_tile_kernel<XT, NW, R><<<dim3(static_cast<unsigned>(t.nb * t.p)), dim3(64 * NW), 0, s>>>(
        x, w, c, m, n, k, L, nsb, static_cast<int>(t.nb), aligned ? 1 : 0, alpha, beta, bias,
        t.p > 1 ? part : nullptr);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || t.p == 1) return e;
    const int64_t quads = static_cast<int64_t>(m) * ((n + 3) / 4);
    const int64_t blocks = std::min<int64_t>((quads + 255) / 256, 4 * cu_count());
    gemv_split_sum_kernel<XT><<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(
        part, c, m, n, t.p, alpha, beta, bias);
    return hipGetLastError();
}

template <int XT, int NW>
hipError_t launch_tile_nw(const TilePlan &t, const void *x, const uint8_t *w, void *c, int m,
                          int64_t n, int64_t k, bool aligned, float alpha, float beta,
                          const float *bias, float *part, hipStream_t s) {
    switch (t.r) {
        case 4: return launch_tile_r<XT, NW, 4>(t, x, w, c, m, n, k, aligned, alpha, beta, bias, part, s);
        case 2: return launch_tile_r<XT, NW, 2>(t, x, w, c, m, n, k, aligned, alpha, beta, bias, part, s);
        default: return launch_tile_r<XT, NW, 1>(t, x, w, c, m, n, k, aligned, alpha, beta, bias, part, s);
    }
}

// Runs the tile kernel when the shape fits and the workspace holds its splits;
// *handled is false otherwise (the caller then takes the wave / stream kernels).
template <int XT>
hipError_t launch_gemv_tile(bool *handled, const void *x, const uint8_t *w, void *c, int m,
                            int64_t n, int64_t k, float alpha, float beta, const float *bias,
                            void *ws, int64_t ws_bytes, hipStream_t s) {
    *handled = false;
    if (!gemv_tile_fits(m, n, k)) return hipSuccess;
    const TilePlan t = gemv_tile_plan(n, k);
    if (t.p > 1 && (ws == nullptr || ws_bytes < int64_t{4} * t.p * m * n)) return hipSuccess;
    constexpr int64_t kElem = XT == kDtypeF32 ? 4 : (XT == kDtypeBF16 ? 2 : 1);
    const bool aligned =
        (k % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % (kElem == 1 ? 8 : 16) == 0);
    // aligned bf16: the stream kernel with staged activation pieces, one launch, is faster
    // (llama.down M = 16 13.2 us against 14.4 with the split sum; phi3.down 7.9 against 9.4)
    if (XT == kDtypeBF16 && aligned) return hipSuccess;
    // int8 at 5+ tokens with 16-value pieces: the same staged stream kernel
    if (XT == kDtypeI8 && m >= 8 && k % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0)
        return hipSuccess;
    *handled = true;
    float *part = static_cast<float *>(ws);
    if (t.nw == 4)
        return launch_tile_nw<XT, 4>(t, x, w, c, m, n, k, aligned, alpha, beta, bias, part, s);
    return launch_tile_nw<XT, 8>(t, x, w, c, m, n, k, aligned, alpha, beta, bias, part, s);
}

template <int XT, int G, bool kAligned, int KS>
hipError_t launch_stream(const void *x, const uint8_t *w, void *c, int m, int64_t n, int64_t k,
                         int64_t L, float alpha, float beta, const float *bias, hipStream_t s) {
    const int64_t blocks = (n + 16 * G - 1) / (16 * G);
    // Staged pieces for one row group per workgroup or 8+ tokens (llama.down M = 8
    // 12.95 -> 11.43 us, phi3.down M = 8 8.26 -> 7.36, llama.gate M = 16 12.94 -> 12.26);
    // at two row groups and fewer tokens the direct fragment loads, which then touch only
    // M token rows, measured faster (llama.gate M = 5 9.53 against 10.66 staged).
    if constexpr (XT == kDtypeBF16 && kAligned) {
        if (G == 1 || m >= 8) {
            gemv_stream_kernel<XT, G, kAligned, KS, true><<<dim3(blocks), dim3(64 * KS), 0, s>>>(
                x, w, c, m, n, k, L, alpha, beta, bias);
            return hipGetLastError();
        }
    }
    if constexpr (XT == kDtypeI8 && kAligned) {
        // int8, 5+ tokens: the same staging, the values widened to bf16 (16-value pieces).
        // One row group per workgroup (<= 4096 rows) keeps two sub-blocks in flight: with
        // three pieces per lane the second slot is cheap (llama.down M = 8 14.5 -> 12.6 us,
        // M = 16 14.5 -> 13.1, 3072 -> 3072 5.5 -> 5.4; the wider, two- and four-group
        // shapes measured slower, 10.1 -> 11.7 on llama.gate, as did bf16, whose six
        // pieces per lane double the slot: llama.down M = 16 13.2 -> 13.4)
        if (m >= 5 && k % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0) {
            if constexpr (G == 1)
                gemv_stream_kernel<XT, G, kAligned, KS, true, true>
                    <<<dim3(blocks), dim3(64 * KS), 0, s>>>(x, w, c, m, n, k, L, alpha, beta, bias);
            else
                gemv_stream_kernel<XT, G, kAligned, KS, true>
                    <<<dim3(blocks), dim3(64 * KS), 0, s>>>(x, w, c, m, n, k, L, alpha, beta, bias);
            return hipGetLastError();
        }
    }
    gemv_stream_kernel<XT, G, kAligned, KS, false><<<dim3(blocks), dim3(64 * KS), 0, s>>>(
        x, w, c, m, n, k, L, alpha, beta, bias);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// gemv_stream2_kernel: 17..48 tokens (49..64 as two launches) of bf16 (K % 8 == 0) or int8
// (K % 16 == 0) activations at a 16-byte aligned x: the staged stream kernel with NB = 2 or
// 3 16-token column blocks: each weight limb is decoded once and meets every block's B
// fragments (six MFMAs each), so the weights stream once for all the tokens.  Staging, the fixed-order reduction and the stores as gemv_stream_kernel, per
// block (block b holds tokens 16 b .. 16 b + 15).  A separate kernel, not a template
// parameter of the other: the 8..16-token code generation stays as tuned.
template <int G, int KS, int NB, int XT>
__global__ __launch_bounds__(64 * KS) void gemv_stream2_kernel(const void *__restrict__ x,
                                                           const uint8_t *__restrict__ w,
                                                           void *__restrict__ c, int M,
                                                           int64_t N, int64_t K, int64_t L,
                                                           float alpha, float beta,
                                                           const float *__restrict__ bias) {
    static_assert(NB == 2 || NB == 3, "two or three column blocks");
    static_assert(XT == kDtypeBF16 || XT == kDtypeI8, "bf16, or int8 widened to bf16 in LDS");
    // A piece is 16 bytes of one token's activations: 8 bf16 or 16 int8 values (int8 is
    // widened to bf16 as it is staged, so the LDS layout and the fragment reads are the
    // same; the fp32 sums of integers stay exact under the ABI's K <= 131071).
    constexpr int kVals = XT == kDtypeI8 ? 16 : 8;        // values per piece
    constexpr int kPieces = 4 * kTrits / kVals;           // pieces per token and sub-block
    constexpr int kLanePieces = 16 * kPieces / 64;        // per lane and block: 6 or 3
    constexpr int kElem = XT == kDtypeI8 ? 1 : 2;
    // NB = 3: each wave's partial tiles go into its own staging region (its last fragment
    // reads come before them in the wave's LDS order), so eight waves fit in 154 KB
    constexpr bool kAlias = NB >= 3;
    static_assert(!kAlias || G * NB * 64 * 16 <= NB * kXStageBytes, "partials fit the region");
    __shared__ __attribute__((aligned(16))) uint8_t lut[kLutBytes];
    __shared__ __attribute__((aligned(16))) floatx4 red_own[kAlias ? 1 : KS * G * NB * 64];
    __shared__ __attribute__((aligned(16))) uint8_t xst[KS * NB * kXStageBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // partial tile (wave ww, row group g, block b)
    auto red_at = [&](int ww, int g, int b) -> floatx4 & {
        if constexpr (kAlias)
            return reinterpret_cast<floatx4 *>(xst)[ww * (NB * kXStageBytes / 16) + (g * NB + b) * 64 + lane];
        else return red_own[((ww * G + g) * NB + b) * 64 + lane];
    };
    const int wave = tid >> 6;
    const int r = lane & 15;
    const int q = lane >> 4;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * (16 * G);
    const int64_t S = (L + 3) / 4;

    bf16x8 bh[NB][6], bl[6];
    u32x4 xp[kLanePieces * NB];
    uint8_t *xs = xst + wave * NB * kXStageBytes;
#pragma unroll
    for (int j = 0; j < 6; ++j) bl[j] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
    auto load_pieces = [&](int64_t sb) {
#pragma unroll
        for (int i = 0; i < kLanePieces * NB; ++i) {
            const int P = 64 * i + lane;
            const int t = P / kPieces;
            const int64_t k = sb * (4 * kTrits) + kVals * (P - kPieces * t);
            const bool ok = t < M && sb < S && k < K;
            const uint8_t *src = ok ? static_cast<const uint8_t *>(x) + (t * K + k) * kElem
                                    : reinterpret_cast<const uint8_t *>(kZeroBlock);
            xp[i] = *reinterpret_cast<const u32x4 *>(src);
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < kLanePieces * NB; ++i) {
            const int P = 64 * i + lane;
            const int t = P / kPieces;
            uint8_t *dst = xs + t * kXStagePitch + 16 * (kVals / 8) * (P - kPieces * t);
            if constexpr (XT == kDtypeI8) {
                // 16 int8 -> 16 bf16 (exact: |v| <= 128 needs 8 significant bits)
                uint32_t h[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t wd = xp[i][e / 2];
                    const int sh = 16 * (e % 2);
                    const float f0 = static_cast<float>(static_cast<int8_t>((wd >> sh) & 0xFFu));
                    const float f1 =
                        static_cast<float>(static_cast<int8_t>((wd >> (sh + 8)) & 0xFFu));
                    h[e] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xFFFF0000u);
                }
                *reinterpret_cast<u32x4 *>(dst) = u32x4{h[0], h[1], h[2], h[3]};
                *reinterpret_cast<u32x4 *>(dst + 16) = u32x4{h[4], h[5], h[6], h[7]};
            } else {
                *reinterpret_cast<u32x4 *>(dst) = xp[i];
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int j = 0; j < 6; ++j)
                bh[b][j] = *reinterpret_cast<const bf16x8 *>(
                    xs + (16 * b + r) * kXStagePitch + 96 * q + 16 * j);
    };
    int64_t s = wave;
    load_pieces(s);
    u32x4 wcur[G];
#pragma unroll
    for (int g = 0; g < G; ++g) wcur[g] = load_limb(w, n0 + 16 * g + r, 4 * s + q, N, L, L);
    lut_init(lut, tid, 64 * KS);
    stage();

    floatx4 acc[G][NB];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[g][b] = floatx4{0.f, 0.f, 0.f, 0.f};

    for (; s < S; s += KS) {
        const int64_t sn = s + KS;
        load_pieces(sn);
        u32x4 wnext[G];
#pragma unroll
        for (int g = 0; g < G; ++g) wnext[g] = load_limb(w, n0 + 16 * g + r, 4 * sn + q, N, L, L);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            uint32_t pairs[24];
#pragma unroll
            for (int d = 0; d < 4; ++d) decode_dword(lut, wcur[g][d], pairs + 6 * d);
#pragma unroll
            for (int b = 0; b < NB; ++b)
                acc[g][b] = mfma_pairs<kDtypeBF16>(pairs, bh[b], bl, acc[g][b]);
            wcur[g] = wnext[g];
        }
        stage();
    }

    // per (row group, block): the KS partial tiles summed in wave order
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int b = 0; b < NB; ++b) red_at(wave, g, b) = acc[g][b];
    __syncthreads();
    for (int e = wave; e < G * NB; e += KS) {
        const int g = e / NB;
        const int b = e % NB;
        floatx4 v = red_at(0, g, b);
#pragma unroll
        for (int ww = 1; ww < KS; ++ww) v += red_at(ww, g, b);
        store_tile<XT>(v, lane, M - 16 * b, N, n0 + 16 * g,
                               static_cast<float *>(c) + static_cast<int64_t>(16 * b) * N, alpha,
                               beta, bias);
    }
}

// Rows per workgroup and waves splitting K for the stream kernel.  Aligned bf16 at 8..16
// tokens: the rule at the top of the function.  Otherwise (a sweep of 1, 2, 4, 8 row
// groups x 4, 8, 16 waves on the config-3/4 decode shapes at 8 and 16 tokens, fragment
// loads):
// at most 4096 rows take one row group per workgroup -- the grid then covers the CUs --
// with eight waves over >= 32 sub-blocks (llama.down M = 8 15.7 -> 13.0 us, phi3.down
// M = 16 13.3 -> 11.3 us) and four below (phi3.o M = 16 6.9 -> 6.0 us); 9..16 tokens
// over >= 9216 rows share each activation fragment between four row groups (llama.gate
// M = 16 14.4 -> 13.0 us); up to 8 tokens over a long K (>= 40 sub-blocks) split it
// over eight waves; else two row groups, four waves.
template <int XT, bool kAligned>
hipError_t launch_stream_shape(const void *x, const uint8_t *w, void *c, int m, int64_t n,
                               int64_t k, int64_t L, float alpha, float beta, const float *bias,
                               hipStream_t s) {
    const int64_t nsb = (L + 3) / 4;
    // int8 with K % 16 == 0 and a 16-byte aligned x stages its pieces like bf16
    bool staged = false;
    if constexpr (XT == kDtypeBF16 && kAligned) staged = true;
    if constexpr (XT == kDtypeI8 && kAligned)
        staged = k % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    if (staged) {
        // 8..16 tokens, staged pieces (their cost no longer grows with the tokens): eight
        // waves, the row groups per workgroup by width -- a sweep of 1, 2, 4 groups x 4, 8,
        // 16 waves at 5, 8, 9, 12 and 16 tokens: llama.gate M = 16 12.3 -> 10.1 us, phi3.qkv
        // 9.8 -> 7.5, phi3.gate_up 10.7 -> 8.4, phi3.o 5.9 -> 4.9, 4096 -> 6144 8.6 -> 7.2,
        // phi3.qkv M = 8 8.3 -> 7.5; at 5 tokens the fragment loads stay faster
        if (m >= 8) {
            if (n <= 4096)
                return launch_stream<XT, 1, kAligned, 8>(x, w, c, m, n, k, L, alpha, beta, bias, s);
            if (n < 9216)
                return launch_stream<XT, 2, kAligned, 8>(x, w, c, m, n, k, L, alpha, beta, bias, s);
            return launch_stream<XT, 4, kAligned, 8>(x, w, c, m, n, k, L, alpha, beta, bias, s);
        }
    }
    if (n <= 4096) {
        if (nsb >= 32)
            return launch_stream<XT, 1, kAligned, 8>(x, w, c, m, n, k, L, alpha, beta, bias, s);
        return launch_stream<XT, 1, kAligned, 4>(x, w, c, m, n, k, L, alpha, beta, bias, s);
    }
    if (m > 8 && n >= 9216)
        return launch_stream<XT, 4, kAligned, 4>(x, w, c, m, n, k, L, alpha, beta, bias, s);
    if (m <= 8 && nsb >= 40)
        return launch_stream<XT, 2, kAligned, 8>(x, w, c, m, n, k, L, alpha, beta, bias, s);
    return launch_stream<XT, 2, kAligned, 4>(x, w, c, m, n, k, L, alpha, beta, bias, s);
}

// Dynamic LDS of the wave kernel: 160 KiB per CU less its static reduction tile.
constexpr size_t kMaxWaveLds = 160 * 1024 - 16 * 64 * 16 - kLutBytes;

struct WaveArgs {
    const void *x;
    const uint8_t *w;
    void *c;
    int m;
    int64_t n, k;
    int L, nsb, wg, nsbw_max;
    uint32_t magic;
    bool aligned;
    size_t lds;
    float alpha, beta;
    const float *bias;
    hipStream_t s;
};

template <int XT, int W, int SU, int R>
hipError_t launch_wave(const WaveArgs &a) {
    auto fn = reinterpret_cast<const void *>(&gemv_wave_kernel<XT, W, SU, R>);
    static size_t raised = 64 * 1024;  // dynamic LDS above 64 KiB needs an opt-in
    if (a.lds > raised) {
        const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 static_cast<int>(kMaxWaveLds));
        if (e != hipSuccess) return e;
        raised = kMaxWaveLds;
    }
    const int G = W / a.wg;
    const int64_t groups = (a.n + 15) / 16;
    gemv_wave_kernel<XT, W, SU, R><<<dim3((groups + G - 1) / G), dim3(64 * W), a.lds, a.s>>>(
        a.x, a.w, a.c, a.m, a.n, a.k, a.L, a.nsb, a.wg, a.nsbw_max, a.magic, a.aligned ? 1 : 0,
        a.alpha, a.beta, a.bias);
    return hipGetLastError();
}

// Run length R: every value for bf16 activations (the decode case); 4 / 8 / 12 for
// fp32 and int8, whose spare loads matter less next to their staging cost.
template <int XT, int W, int SU, int R = kMaxRun>
hipError_t launch_wave_r(int run, const WaveArgs &a) {
    if constexpr (R <= 1) {
        return launch_wave<XT, W, SU, 1>(a);
    } else if constexpr (XT != kDtypeBF16 && R % 4 != 0) {
        return launch_wave_r<XT, W, SU, R - 1>(run, a);
    } else {
        const int lower = XT == kDtypeBF16 ? R - 1 : R - 4;
        if (run > lower || (XT != kDtypeBF16 && R == 4)) return launch_wave<XT, W, SU, R>(a);
        return launch_wave_r<XT, W, SU, R - 1>(run, a);
    }
}

template <int XT, int W>
hipError_t launch_wave_su(int su, int run, const WaveArgs &a) {
    if (su <= 4) return launch_wave_r<XT, W, 4>(run, a);
    return launch_wave_r<XT, W, 8>(run, a);
}

// Waves in flight the wave kernel aims for before it splits K finer.
constexpr int64_t kTargetWaves = 1024;

// float32 at 5..8 tokens (K % 4 == 0, 16-byte aligned x): the staged stream kernel with
// each token's hi and lo planes as two of the 16 B columns, row groups per workgroup as for
// bf16 at 8+ tokens.  Against the wave / stream kernels' second MFMA per operand (same
// box): 8 tokens 14336 -> 4096 26.65 -> 15.91 us, 4096 -> 14336 17.30 -> 10.96, 3072 ->
// 16384 14.31 -> 9.03, 3072 -> 3072 7.75 -> 6.07; 5 tokens 22.98 -> 15.93, 14.10 ->
// 10.90, 18.19 -> 9.06.  At 3 and 4 tokens the strip kernel stays faster (14336 -> 4096
// 11.41 / 13.98 against 15.97 / 15.98 this way).
hipError_t launch_stream_split(const void *x, const uint8_t *w, void *c, int m, int64_t n,
                               int64_t k, int64_t L, float alpha, float beta, const float *bias,
                               hipStream_t s) {
    auto go = [&](auto gc) {
        constexpr int G = decltype(gc)::value;
        const int64_t blocks = (n + 16 * G - 1) / (16 * G);
        gemv_stream_kernel<kDtypeF32, G, true, 8, true, false, true>
            <<<dim3(static_cast<unsigned>(blocks)), dim3(64 * 8), 0, s>>>(x, w, c, m, n, k, L,
                                                                        alpha, beta, bias);
        return hipGetLastError();
    };
    if (n <= 4096) return go(std::integral_constant<int, 1>());
    if (n < 9216) return go(std::integral_constant<int, 2>());
    return go(std::integral_constant<int, 4>());
}

bool stream_split_fits(const void *x, int m, int64_t k) {
    return m >= 5 && m <= 8 && k % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
}

template <int XT>
hipError_t launch_gemv_x(const void *x, const uint8_t *w, void *c, int m, int64_t n, int64_t k,
                         float alpha, float beta, const float *bias, hipStream_t s) {
    if constexpr (XT == kDtypeF32) {
        if (stream_split_fits(x, m, k))
            return launch_stream_split(x, w, c, m, n, k, (k + kTrits - 1) / kTrits, alpha, beta,
                                       bias, s);
    }
    using LY = WaveLayout<XT>;
    const int elem = LY::kElem;
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t groups = (n + 15) / 16;
    const int64_t nsb = (L + 3) / 4;
    const bool aligned8 = (k % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % (8 * elem) == 0);
    // longest run per wave: the run's loads and its activation loads all in flight
    const int64_t max_run = std::min<int64_t>(
        kMaxRun, (64 * kMaxChunksPerLane) / (static_cast<int64_t>(m) * LY::kChunksPerSb));
    // waves per group: the fewest that fit the run, then more while the grid is
    // small and every wave keeps at least two sub-blocks
    int wg = 1;
    while (wg <= 8 && max_run > 0 && nsb > max_run * wg) wg *= 2;
    // bf16 over many rows takes the stream kernel: 8+ tokens over >= 9216 rows (3072 ->
    // 16384 at M = 8: 10.5 -> 8.7 us; even at 3072 -> 9216), 5+ over >= 14336 (4096 ->
    // 14336 at M = 5: 11.2 -> 9.6 us; 3072 -> 9216 at M = 5 stays faster staged)
    // ... and 8+ tokens with aligned bf16 activations, staged (see launch_stream_shape)
    // int8 from 5 tokens (K % 16 == 0, aligned x) takes the staged stream kernel: against
    // the wave kernel at 5..7 tokens 3072 -> 9216 12.25 / 10.49 / 11.35 -> 9.08 / 9.05 /
    // 9.18 us, 8192 -> 3072 10.28 / 10.96 / 11.64 -> 8.18 / 8.16 / 8.18, 14336 -> 4096 13.3
    // -> 12.4 (3072 -> 3072 at 5 tokens 5.57 -> 5.78)
    const bool stage_i8 = XT == kDtypeI8 && m >= 5 && k % 16 == 0 &&
                          reinterpret_cast<uintptr_t>(x) % 16 == 0;
    const bool wide = (XT == kDtypeBF16 && ((m >= 8 && n >= 9216) || (m >= 5 && n >= 14336) ||
                                            (m >= 8 && aligned8))) ||
                      stage_i8;
    if (L > 0 && max_run > 0 && wg <= 8 && !wide) {
        while (wg < 8 && groups * wg < kTargetWaves && nsb >= 4 * wg) wg *= 2;
        const int W = wg < 4 ? 4 : wg;
        const int nsbw_max = static_cast<int>((nsb + wg - 1) / wg);
        const size_t lds =
            static_cast<size_t>(W) * wave_lds_bytes(m, nsbw_max, LY::kPlanes);
        const int cpr = nsbw_max * LY::kChunksPerSb;
        const int su = (m * cpr + 63) / 64;
        if (lds <= kMaxWaveLds && su <= kMaxChunksPerLane) {
            WaveArgs a;
            a.x = x;
            a.w = w;
            a.c = c;
            a.m = m;
            a.n = n;
            a.k = k;
            a.L = static_cast<int>(L);
            a.nsb = static_cast<int>(nsb);
            a.wg = wg;
            a.nsbw_max = nsbw_max;
            a.magic = static_cast<uint32_t>((uint64_t{1} << 32) / cpr + 1);
            a.aligned = (k % LY::kChunkVals == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
            a.lds = lds;
            a.alpha = alpha;
            a.beta = beta;
            a.bias = bias;
            a.s = s;
            if (W == 4) return launch_wave_su<XT, 4>(su, nsbw_max, a);
            return launch_wave_su<XT, 8>(su, nsbw_max, a);
        }
    }
    if (aligned8) return launch_stream_shape<XT, true>(x, w, c, m, n, k, L, alpha, beta, bias, s);
    return launch_stream_shape<XT, false>(x, w, c, m, n, k, L, alpha, beta, bias, s);
}

}  // namespace

// 17..48 tokens (64 with K <= 8192, bf16 32 from K = 12288: gemv_column_blocks_max_tokens)
// with aligned bf16 activations (called by the K3 launcher, which owns M > 16): the
// column-block stream kernel, no workspace.  17..32
// tokens, two blocks: row groups per workgroup and waves from a sweep of 1, 2, 4 groups x
// 4, 8 waves at 17, 24 and 32 tokens on the config-3/4 shapes, against the eight-wave GEMM
// kernel with its K split: at 32 tokens llama.qkv 15.8 -> 9.9 us, 4096 -> 4096 13.9 ->
// 8.7, gate_up 35.1 -> 28.7, llama.down 28.0 -> 19.6, phi3.o 15.2 -> 7.4, phi3.gate_up
// 20.7 -> 13.2. 33..48 tokens, three blocks, eight waves (four measured slower: one wave
// per SIMD): at 48 tokens llama.gate 31.7 -> 26.6 us, llama.down 34.4 -> 28.3, llama.qkv
// 20.0 -> 13.6, phi3.qkv 23.8 -> 20.1, phi3.o 19.1 -> 10.4, phi3.down 24.9 -> 17.0,
// phi3.gate_up 28.2 -> 21.3.  49..64 tokens: two launches, tokens [0, 32) and [32, M)
// (four blocks in one launch were slower than the GEMM kernel on the long-K and widest
// shapes: each workgroup then reads 64 tokens' activations); at 64 tokens llama.gate 33.3
// -> 30.2 us, llama.qkv 21.3 -> 19.5, phi3.qkv 26.0 -> 23.2, phi3.o 20.2 -> 14.1,
// phi3.down 26.0 -> 23.4, phi3.gate_up 30.9 -> 24.4; K > 8192 keeps the GEMM kernel
// (llama.down 34.6 -> 36.1 at 49 tokens).  Results are bit-identical to the GEMM kernel's
// on integer activations.  *handled is false for other shapes.
hipError_t launch_gemv_column_blocks(bool *handled, const void *x, int x_dtype,
                                     const uint8_t *w, void *c, int m, int64_t n, int64_t k,
                                     float alpha, float beta, const float *bias, hipStream_t s) {
    *handled = false;
    if (!gemv_column_blocks_fits(x, x_dtype, m, n, k)) return hipSuccess;
    if (m > 48) {
        // tokens [32, m): x advances 32 rows of K values (16-byte aligned by the K rule), C
        // 32 rows of N four-byte values
        const int64_t elem = x_dtype == kDtypeI8 ? 1 : 2;
        bool h = false;
        const hipError_t e =
            launch_gemv_column_blocks(&h, x, x_dtype, w, c, 32, n, k, alpha, beta, bias, s);
        if (e != hipSuccess) return e;
        *handled = true;
        return launch_gemv_column_blocks(&h, static_cast<const uint8_t *>(x) + 32 * k * elem,
                                         x_dtype, w, static_cast<float *>(c) + 32 * n, m - 32,
                                         n, k, alpha, beta, bias, s);
    }
    const int64_t L = (k + kTrits - 1) / kTrits;
    *handled = true;
    auto go = [&](auto xc, auto gc, auto kc, auto nbc) {
        constexpr int XT = decltype(xc)::value;
        constexpr int G = decltype(gc)::value, KS = decltype(kc)::value;
        constexpr int NB = decltype(nbc)::value;
        const int64_t blocks = (n + 16 * G - 1) / (16 * G);
        gemv_stream2_kernel<G, KS, NB, XT><<<dim3(static_cast<unsigned>(blocks)), dim3(64 * KS),
                                             0, s>>>(x, w, c, m, n, k, L, alpha, beta, bias);
        return hipGetLastError();
    };
    auto shape = [&](auto xc) {
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        using I3 = std::integral_constant<int, 3>;
        using I4 = std::integral_constant<int, 4>;
        using I8 = std::integral_constant<int, 8>;
        if (m > 32) return n <= 4096 ? go(xc, I1(), I8(), I3()) : go(xc, I2(), I8(), I3());
        if (n <= 4096) return go(xc, I1(), I8(), I2());
        if (n < 9216) return go(xc, I2(), I8(), I2());
        return go(xc, I2(), I4(), I2());
    };
    if (x_dtype == kDtypeI8) return shape(std::integral_constant<int, kDtypeI8>());
    return shape(std::integral_constant<int, kDtypeBF16>());
}

int64_t gemv_column_blocks_max_tokens(int64_t k, int x_dtype) {
    // 64 up to K = 8192 (49..64 as two launches), else 48; bf16 32 from K = 12288: over the
    // longest K the eight-wave kernel's four-limb, 128-row form is faster at 33..48 bf16
    // tokens (14336 -> 4096 at 33 / 48 tokens 26.5 / 27.6 -> 25.0 / 25.0 us, 14336 -> 8192
    // 33.9 / 34.9 -> 29.6 / 31.3) while over 11008 it is not (20.9 / 21.1 -> 23.2 / 23.6),
    // nor at 17..32 tokens (14336 -> 4096 at 32 19.1 against 22.6), nor for int8, whose
    // column blocks stage a third of the bytes (14336 -> 4096 at 48 29.2 us against 37.4 at
    // 49 in the eight-wave kernel)
    if (k <= 8192) return 64;
    return x_dtype == kDtypeBF16 && k >= 12288 ? 32 : 48;
}

bool gemv_column_blocks_fits(const void *x, int x_dtype, int64_t m, int64_t n, int64_t k) {
    // 16-byte pieces of whole 8-value (bf16) or 16-value (int8) chunks; block offsets
    // (16 rows x N) and grid in range
    const int64_t chunk = x_dtype == kDtypeI8 ? 16 : 8;
    return (x_dtype == kDtypeBF16 || x_dtype == kDtypeI8) && m >= 17 &&
           m <= gemv_column_blocks_max_tokens(k, x_dtype) && n > 0 && k > 0 && k % chunk == 0 &&
           reinterpret_cast<uintptr_t>(x) % 16 == 0 && (n + 15) / 16 < (int64_t(1) << 31) &&
           k < (int64_t(1) << 31);
}

int64_t gemv_workspace_bytes(int64_t m, int64_t n, int64_t k, int x_dtype) {
    if (m < 5 || m > 16 || n <= 0 || k <= 0) return 0;
    // bf16 with K % 8 == 0 runs the staged stream kernel in one launch instead
    if (x_dtype == kDtypeBF16 && k % 8 == 0) return 0;
    if (x_dtype == kDtypeI8 && m >= 5 && k % 16 == 0) return 0;   // the same, 16-value pieces
    return gemv_tile_workspace_bytes(static_cast<int>(m), n, k);   // float32 partials
}

hipError_t launch_gemv(const void *x, int x_dtype, const uint8_t *w, void *c, int m, int64_t n,
                       int64_t k, float alpha, float beta, const float *bias, hipStream_t s,
                       void *ws, int64_t ws_bytes) {
    if (m == 0 || n == 0) return hipSuccess;
    bool handled = false;
    hipError_t e = launch_gemv_strip(&handled, x, x_dtype, w, c, m, n, k, alpha, beta, bias, s);
    if (handled || e != hipSuccess) return e;
    switch (x_dtype) {
        case kDtypeBF16:
            e = launch_gemv_tile<kDtypeBF16>(&handled, x, w, c, m, n, k, alpha, beta, bias, ws,
                                             ws_bytes, s);
            break;
        case kDtypeF32:
            e = launch_gemv_tile<kDtypeF32>(&handled, x, w, c, m, n, k, alpha, beta, bias, ws,
                                            ws_bytes, s);
            break;
        default:
            e = launch_gemv_tile<kDtypeI8>(&handled, x, w, c, m, n, k, alpha, beta, bias, ws,
                                           ws_bytes, s);
            break;
    }
    if (handled || e != hipSuccess) return e;
    switch (x_dtype) {
        case kDtypeBF16: return launch_gemv_x<kDtypeBF16>(x, w, c, m, n, k, alpha, beta, bias, s);
        case kDtypeF32: return launch_gemv_x<kDtypeF32>(x, w, c, m, n, k, alpha, beta, bias, s);
        default: return launch_gemv_x<kDtypeI8>(x, w, c, m, n, k, alpha, beta, bias, s);
    }
}

}  // namespace t81hip

// t81lib_amd/csrc/gemv_strip.hip -- K2 for M <= 4 tokens (bf16 and int8 up to 8 over wide,
// short-K shapes): column strips, activations fixed in registers, wide contiguous weight
// loads.
//
//   C[m, n] = alpha * sum_k X[m, k] * T[n, k] + beta * C[m, n] + bias[n]
//
// The limbs of a row are cut into ranges of 4*S consecutive limbs (S = 16 or 8 for one
// token, 8 for two, 4 for up to four, 2 for up to eight).  A workgroup owns H = R * RPI
// consecutive rows
// (RPI = 16 / S); wave w of it streams range w of all of them (a column "strip"), so the activations
// a lane needs never change: they are loaded once, as the B operand of
// v_mfma_f32_16x16x32_bf16, and stay in registers.  One load instruction covers RPI
// rows x 4*S limbs, i.e. RPI contiguous runs of 64*S bytes (1 KB, 2 x 512 B or 4 x 256 B),
// where a 16-rows x 64 B pattern splits every load into 16 pieces.
//
// Lane (i, q) (i = lane % 16, q = lane / 16) of load t supplies A row i, k-slots of
// quarter q: with a = i / S and s = i % S it holds limb l0 + q*S + s of row
// row0 + t*RPI + a.  Lane (j, q) of B holds the activations of token j / S for limb
// l0 + q*S + j % S.  An MFMA sums over the quarters, D[i][j] = sum_q A(i, q) . B(j, q),
// and A(i, q) meets the activations of its own limb exactly when j % S == i % S: that
// entry is row a's partial sum over the limbs l0 + q*S + s (q = 0..3) for token j / S.
// The other entries mix limbs and are never read.  Each load has its own accumulator
// (started at zero); lane (j, q) holds D[4q + e][j] for e < 4 and keeps element j % 4,
// which for S in {4, 8, 16} is the one matched entry it holds, if any; for S = 2 it keeps
// elements j % 2 and j % 2 + 2, its two matched entries (rows 2q and 2q + 1).  The MFMA
// count per weight byte is the same for every M <= RPI; tokens past M have zero
// activations.
//
// The weights are decoded in padded order (each tryte -> bf16 t0, t1, t2, 0 through
// one 8-byte table read), eight MFMAs per limb; the activations carry a zero in every
// fourth slot to match.  Limbs past L read nothing (their loads point past the buffer
// range and return zeros, which decode to finite trits) and meet zero activations;
// rows past N read zeros and are never stored.
//
// At the end each wave writes its kept values to LDS and every output sums its S
// sub-sums per range over the ranges in a fixed order: no atomics, deterministic results.
#include <algorithm>

#include "gemv_common.hpp"
#include "t81_device.hpp"
#include "t81_kernels.hpp"

namespace t81hip {

namespace {

constexpr int kStripMaxWaves = 8;    // waves per workgroup (2 per SIMD: 256 registers each)
// Weight loads in flight per wave.  Every wave issues its loads at once, the memory
// system returns them in no particular order and a wave consumes them in order:
// four in flight (refilled as each is decoded) keeps the early ones early, where
// eight (all of a strip) made a wave's first decode wait for half of the launch's
// traffic and its last one start after all of it.
constexpr int kStripDepth = 4;
constexpr uint32_t kStripOob = 0x80000000u;

// Padded-order decode of one dword (4 trytes) through the E table: eight dwords, each
// pair a finished half of an MFMA operand (bf16 t0 | t1 << 16, t2 | 0 << 16).
__device__ __forceinline__ void strip_decode(const uint8_t *lds, uint32_t w, uint32_t *out) {
    const uint32_t w8 = w << 3;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const uint32_t a = (w8 >> (8 * b)) & 0xFFu;
        const uint2 e = *reinterpret_cast<const uint2 *>(lds + kLutE + a);
        out[2 * b] = e.x;
        out[2 * b + 1] = e.y;
    }
}

// Natural-order bf16 activations (48 values) -> the eight padded operands:
// operand o = (x[6o], x[6o+1], x[6o+2], 0, x[6o+3], x[6o+4], x[6o+5], 0).
__device__ __forceinline__ void strip_pad(const bf16x8 *nat, bf16x8 *out) {
    uint32_t d[24];
#pragma unroll
    for (int j = 0; j < 6; ++j) {
        const u32x4 v = __builtin_bit_cast(u32x4, nat[j]);
        d[4 * j] = v[0];
        d[4 * j + 1] = v[1];
        d[4 * j + 2] = v[2];
        d[4 * j + 3] = v[3];
    }
#pragma unroll
    for (int o = 0; o < 8; ++o) {
        const u32x4 q = {d[3 * o], d[3 * o + 1] & 0xFFFFu,
                         __builtin_amdgcn_alignbit(d[3 * o + 2], d[3 * o + 1], 16),
                         d[3 * o + 2] >> 16};
        out[o] = __builtin_bit_cast(bf16x8, q);
    }
}

// acc += A x B over the NOPS operands of one limb (eight padded or six natural-order;
// fp32: hi and lo planes).
template <int XT, int NOPS>
__device__ __forceinline__ floatx4 strip_mfma(const uint32_t *pairs, const bf16x8 *bh,
                                              const bf16x8 *bl) {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int o = 0; o < NOPS; ++o) {
        const u32x4 araw = {pairs[4 * o], pairs[4 * o + 1], pairs[4 * o + 2], pairs[4 * o + 3]};
        const bf16x8 a = __builtin_bit_cast(bf16x8, araw);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bh[o], acc, 0, 0, 0);
        if constexpr (XT == kDtypeF32)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl[o], acc, 0, 0, 0);
    }
    return acc;
}

// Element j % 4 of a finished accumulator (lane j = lane % 16).
__device__ __forceinline__ float strip_keep(floatx4 v, int j) {
    const float lo = (j & 1) ? v[1] : v[0];
    const float hi = (j & 1) ? v[3] : v[2];
    return (j & 2) ? hi : lo;
}
// S = 2: elements j % 2 and j % 2 + 2 (rows 4q + j % 2 and 4q + j % 2 + 2).
__device__ __forceinline__ float strip_keep2(floatx4 v, int j, int kp) {
    return (j & 1) ? (kp ? v[3] : v[1]) : (kp ? v[2] : v[0]);
}

// S: sub-positions per quarter (range = 4*S limbs, S in {2, 4, 8, 16}); NW: waves, one range
// each at a time; R: loads per range, i.e. R * (16 / S) rows per workgroup.  kNt: weight
// loads carry the non-temporal hint (see launch_strip_x).  DEPTH: loads in flight per
// wave (kStripDepth, three for the short natural-order strips).  kNat: limbs
// decoded in natural trit order (E and F tables, six MFMAs per limb) instead of padded
// order (E table only, eight MFMAs) -- fewer MFMAs for two ORs per dword; the launch uses
// it for one token over one 64-limb range or up to three 32-limb ranges, where it
// measured faster (4096 x 14336: 7.03 -> 6.95 us; 3072 x 9216: 5.36 -> 5.09 us).
//
// kStageB (bf16, aligned x; waves that stream more than one range): the B operand of a
// range is loaded as consecutive 16-byte pieces of each token's values (piece p = 64 i +
// lane: token p / (24 S), limb (p % (24 S)) / 6 of the range, values 8 (p % 6) ..) and
// reaches the lanes through the wave's own LDS region (64 slots of 112 bytes, one per
// (token, limb), so the fragment reads of 16 lanes fall on distinct banks).  Loaded as
// fragments, each 16-lane pass touches 16 limbs 96 bytes apart.  Measured at four tokens:
// 14336 -> 4096 9.38 -> 8.57 us, 8192 -> 3072 6.27 -> 6.01 us; slower where every wave
// streams one range (4096 -> 14336 at one token 6.45 -> 8.73 us: the LDS round trip then
// sits at the start of every wave's critical path).
//
// kSplit (float32, M <= 2): the hi and lo bf16 planes of each token are two B token
// columns (2 m: hi, 2 m + 1: lo) instead of a second MFMA per operand, so one MFMA
// serves both planes; each output adds its token's two columns at the end.  The launch
// takes S = 8 for one token and 4 for two, as bf16 takes for two and four tokens.
template <int XT, int S, int NW, int R, bool kNat = false, bool kNt = false,
          int DEPTH = kStripDepth, bool kStageB = false, bool kSplit = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void gemv_strip_kernel(
    const void *__restrict__ x, const uint8_t *__restrict__ w, void *__restrict__ c, int M,
    int64_t N, int64_t K, int L, int nranges, int x_aligned, float alpha, float beta,
    const float *__restrict__ bias) {
    static_assert(S == 2 || S == 4 || S == 8 || S == 16,
                  "matched entries per lane: one for S >= 4, two for S = 2");
    static_assert(!kStageB || (XT == kDtypeBF16 && !kNat), "staged B: bf16, padded order");
    static_assert(!kSplit || (XT == kDtypeF32 && S <= 8 && !kStageB),
                  "planes as token columns: float32, two columns per token");
    // the MFMA's operand type: one bf16 plane (bf16, int8, float32 planes as columns)
    constexpr int XM = kSplit ? kDtypeBF16 : XT;
    constexpr int RPI = 16 / S;  // rows per load (and tokens per MFMA)
    constexpr int H = R * RPI;   // rows per workgroup
    constexpr int D = R < DEPTH ? R : DEPTH;
    __shared__ __attribute__((aligned(16))) uint8_t lut[kLutBytes];
    constexpr int KP = S == 2 ? 2 : 1;   // matched entries a lane keeps per load
    __shared__ float red[NW][R][KP][64];
    constexpr int kSlot = 112;
    __shared__ __attribute__((aligned(16))) uint8_t xst[kStageB ? NW * 64 * kSlot : 16];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 15;
    const int q = lane >> 4;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * H;

    // Weights: a buffer based at the workgroup's first row; rows past N read zeros.
    const int64_t remain = (N - row0) * L * kTrytes;
    const int nrec = remain < 0x7FFFFFFF ? static_cast<int>(remain) : 0x7FFFFFFF;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(w + row0 * L * kTrytes), 0, nrec, 0x00020000);
    const uint32_t row_bytes = static_cast<uint32_t>(L) * kTrytes;
    const int sub = q * S + i % S;  // the lane's limb within a range, for A and for B

    auto publish_lut = [&]() {
        lut_fill(lut, tid, 64 * NW);
        __syncthreads();
    };

    float kept[R][KP];
#pragma unroll
    for (int t = 0; t < R; ++t)
#pragma unroll
        for (int kp = 0; kp < KP; ++kp) kept[t][kp] = 0.0f;
    auto keep = [&](int t, floatx4 v) {
        if constexpr (S == 2) {
            kept[t][0] += strip_keep2(v, i, 0);
            kept[t][1] += strip_keep2(v, i, 1);
        } else {
            kept[t][0] += strip_keep(v, i);
        }
    };

    bool first = true;
    for (int rg = wave; rg < nranges; rg += NW) {
        const int limb = rg * 4 * S + sub;
        const bool in_row = limb < L;
        // ---- B: activations of token i / S for the lane's limb (kSplit: column i / S is
        // plane (i / S) % 2 of token i / S / 2) ----
        const int mb = kSplit ? (i / S) >> 1 : i / S;
        const bool bvalid = mb < M && in_row;
        const int64_t xrow = static_cast<int64_t>(mb < M ? mb : 0) * K;
        const int64_t kb = static_cast<int64_t>(limb) * kTrits;
        XRaw xr[6];
        u32x4 xp[6];
        if constexpr (kStageB) {
#pragma unroll
            for (int ii = 0; ii < 6; ++ii) {
                const int p = 64 * ii + lane;
                const int tk = p / (24 * S);
                const int pp = p - tk * (24 * S);
                const int64_t v =
                    (static_cast<int64_t>(rg) * 4 * S + pp / 6) * kTrits + 8 * (pp % 6);
                const bool ok = tk < M && v < K;
                const uint8_t *src = ok ? static_cast<const uint8_t *>(x) + (tk * K + v) * 2
                                        : reinterpret_cast<const uint8_t *>(kZeroBlock);
                xp[ii] = *reinterpret_cast<const u32x4 *>(src);
            }
        } else if (x_aligned) {
#pragma unroll
            for (int j = 0; j < 6; ++j)
                xr[j] = load_x8_raw<XT, true>(x, xrow, kb + 8 * j, K, bvalid);
        } else {
#pragma unroll
            for (int j = 0; j < 6; ++j)
                xr[j] = load_x8_raw<XT, false>(x, xrow, kb + 8 * j, K, bvalid);
        }

        // ---- A: load t = the lane's limb of row t * RPI + i / S ----
        const uint32_t lane_off = in_row ? static_cast<uint32_t>(i / S) * row_bytes +
                                               static_cast<uint32_t>(limb) * kTrytes
                                         : kStripOob;
        auto fetch = [&](int t) -> u32x4 {
            const uint32_t off = in_row ? lane_off + static_cast<uint32_t>(t * RPI) * row_bytes
                                        : kStripOob;
            return __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, kNt ? kCpolNt : 0));
        };
        u32x4 ring[D];  // load t lives in ring[t % D]
#pragma unroll
        for (int t = 0; t < D; ++t) ring[t] = fetch(t);

        if (first) {
            publish_lut();
            first = false;
        }

        if constexpr (kStageB) {
            // the wave's own region: its LDS operations complete in order, so the next
            // range's writes come after these reads without a barrier
            uint8_t *xs = xst + wave * 64 * kSlot;
#pragma unroll
            for (int ii = 0; ii < 6; ++ii) {
                const int p = 64 * ii + lane;
                const int tk = p / (24 * S);
                const int pp = p - tk * (24 * S);
                *reinterpret_cast<u32x4 *>(xs + (tk * 4 * S + pp / 6) * kSlot + 16 * (pp % 6)) =
                    xp[ii];
            }
            const int slot = (i / S) * 4 * S + sub;
#pragma unroll
            for (int j = 0; j < 6; ++j)
                xr[j].a = *reinterpret_cast<const u32x4 *>(xs + slot * kSlot + 16 * j);
        }
        constexpr int kOps = kNat ? 6 : 8;  // MFMA operands per limb
        bf16x8 nh[6], nl[6], bh[kOps], bl[kOps];
#pragma unroll
        for (int j = 0; j < 6; ++j) cvt_x8<XT>(xr[j], nh[j], nl[j]);
        if constexpr (kSplit) {
            // the lane's column carries one plane
            const bool lo_col = ((i / S) & 1) != 0;
#pragma unroll
            for (int j = 0; j < 6; ++j) nh[j] = lo_col ? nl[j] : nh[j];
        }
        if constexpr (kNat) {
#pragma unroll
            for (int j = 0; j < 6; ++j) {
                bh[j] = nh[j];
                bl[j] = nl[j];
            }
        } else {
            strip_pad(nh, bh);
            if constexpr (XM == kDtypeF32) strip_pad(nl, bl);
        }
        auto decode = [&](uint32_t wd, uint32_t *out) {
            if constexpr (kNat) decode_dword(lut, wd, out);
            else strip_decode(lut, wd, out);
        };

        // Software-pipelined: the table reads of load t + 1 are issued before the
        // MFMAs of load t; a ring slot is refilled as soon as it is decoded.  The
        // accumulator of load t is read one load later, when its MFMAs are done.
        uint32_t cur[4 * kOps], nxt[4 * kOps];
#pragma unroll
        for (int d = 0; d < 4; ++d) decode(ring[0][d], cur + kOps * d);
        __builtin_amdgcn_sched_barrier(0);
        if (D < R) ring[0] = fetch(D);
        floatx4 prev = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < R; ++t) {
            if (t + 1 < R) {
#pragma unroll
                for (int d = 0; d < 4; ++d) decode(ring[(t + 1) % D][d], nxt + kOps * d);
                __builtin_amdgcn_sched_barrier(0);
                if (t + 1 + D < R) ring[(t + 1) % D] = fetch(t + 1 + D);
            }
            const floatx4 acc = strip_mfma<XM, kOps>(cur, bh, bl);
            if (t > 0) keep(t - 1, prev);
            prev = acc;
#pragma unroll
            for (int e = 0; e < 4 * kOps; ++e) cur[e] = nxt[e];
        }
        keep(R - 1, prev);
    }
    if (first) publish_lut();  // a wave with no range still takes part in the barriers

    // ---- kept values to LDS; each output sums S sub-sums per wave, waves in order ----
#pragma unroll
    for (int t = 0; t < R; ++t)
#pragma unroll
        for (int kp = 0; kp < KP; ++kp) red[wave][t][kp][lane] = kept[t][kp];
    __syncthreads();

    const int nw_used = nranges < NW ? nranges : NW;
    for (int e = tid; e < H * RPI; e += 64 * NW) {
        const int r = e / RPI;  // row within the workgroup: load r / RPI, A row group r % RPI
        const int m = e % RPI;
        const int t = r / RPI;
        const int ra = r % RPI;
        const int64_t n = row0 + r;
        if (m >= M || n >= N) continue;
        float val = 0.0f;
        for (int ww = 0; ww < nw_used; ++ww) {
#pragma unroll
            for (int ss = 0; ss < S; ++ss) {
                // entry D[ra*S + ss][m*S + ss] sits in lane (m*S + ss) + 16 * ((ra*S + ss) / 4)
                // (S = 2: lane j's two kept entries are rows 4q + j % 2 (kp 0) and
                // 4q + j % 2 + 2 (kp 1), i.e. kp = ra % 2)
                const int kp = S == 2 ? (ra & 1) : 0;
                if constexpr (kSplit) {
                    // token m's hi column 2 m and lo column 2 m + 1
                    val += red[ww][t][kp][2 * m * S + ss + 16 * ((ra * S + ss) >> 2)];
                    val += red[ww][t][kp][(2 * m + 1) * S + ss + 16 * ((ra * S + ss) >> 2)];
                } else {
                    val += red[ww][t][kp][m * S + ss + 16 * ((ra * S + ss) >> 2)];
                }
            }
        }
        if constexpr (XT == kDtypeI8) {
            int32_t *cp = static_cast<int32_t *>(c) + static_cast<int64_t>(m) * N + n;
            int32_t y = static_cast<int32_t>(val);
            if (beta != 0.0f) y += *cp;
            *cp = y;
        } else {
            float *cp = static_cast<float *>(c) + static_cast<int64_t>(m) * N + n;
            float y = alpha * val;
            if (beta != 0.0f) y = y + beta * *cp;
            if (bias != nullptr) y = y + bias[n];
            *cp = y;
        }
    }
}

struct StripArgs {
    const void *x;
    const uint8_t *w;
    void *c;
    int m;
    int64_t n, k;
    int L, nranges;
    bool aligned;
    float alpha, beta;
    const float *bias;
    hipStream_t s;
};

template <int XT, int S, int NW, int R, bool kNat = false, bool kNt = false,
          int DEPTH = kStripDepth, bool kStageB = false, bool kSplit = false>
hipError_t launch_strip(const StripArgs &a) {
    constexpr int H = R * (16 / S);
    const int64_t blocks = (a.n + H - 1) / H;
    gemv_strip_kernel<XT, S, NW, R, kNat, kNt, DEPTH, kStageB, kSplit>
        <<<dim3(static_cast<unsigned>(blocks)), dim3(64 * NW), 0, a.s>>>(
            a.x, a.w, a.c, a.m, a.n, a.k, a.L, a.nranges, a.aligned ? 1 : 0, a.alpha, a.beta,
            a.bias);
    return hipGetLastError();
}

template <int XT, int S, int R, bool kNt = false, bool kStageB = false, bool kSplit = false>
hipError_t launch_strip_nw(int nw, const StripArgs &a) {
    constexpr int D = kStripDepth;
    if constexpr (kSplit) {
        switch (nw) {
            case 1: return launch_strip<XT, S, 1, R, false, kNt, D, false, true>(a);
            case 2: return launch_strip<XT, S, 2, R, false, kNt, D, false, true>(a);
            case 3: return launch_strip<XT, S, 3, R, false, kNt, D, false, true>(a);
            case 4: return launch_strip<XT, S, 4, R, false, kNt, D, false, true>(a);
            case 5: return launch_strip<XT, S, 5, R, false, kNt, D, false, true>(a);
            case 6: return launch_strip<XT, S, 6, R, false, kNt, D, false, true>(a);
            case 7: return launch_strip<XT, S, 7, R, false, kNt, D, false, true>(a);
            default: return launch_strip<XT, S, 8, R, false, kNt, D, false, true>(a);
        }
    }
    if constexpr (kStageB) {
        // staged B runs only where waves stream several ranges: five waves or more
        switch (nw) {
            case 5: return launch_strip<XT, S, 5, R, false, kNt, D, true>(a);
            case 6: return launch_strip<XT, S, 6, R, false, kNt, D, true>(a);
            case 7: return launch_strip<XT, S, 7, R, false, kNt, D, true>(a);
            default: return launch_strip<XT, S, 8, R, false, kNt, D, true>(a);
        }
    }
    switch (nw) {
        case 1: return launch_strip<XT, S, 1, R, false, kNt>(a);
        case 2: return launch_strip<XT, S, 2, R, false, kNt>(a);
        case 3: return launch_strip<XT, S, 3, R, false, kNt>(a);
        case 4: return launch_strip<XT, S, 4, R, false, kNt>(a);
        case 5: return launch_strip<XT, S, 5, R, false, kNt>(a);
        case 6: return launch_strip<XT, S, 6, R, false, kNt>(a);
        case 7: return launch_strip<XT, S, 7, R, false, kNt>(a);
        default: return launch_strip<XT, S, 8, R, false, kNt>(a);
    }
}

// Natural-order launches (bf16, one token, at most three ranges).  Strips of at most
// seven loads keep three of them in flight, not four: 4096 -> 14336 (seven loads)
// 6.69 -> 6.45 us, 3072 -> 9216 (four) 4.94 -> 4.69 us; eight loads (3072 -> 16384)
// measured 1 % slower with three.
template <int S, int R, bool kNt, int XT = kDtypeBF16, bool kSplit = false>
hipError_t launch_strip_nat_nw(int nw, const StripArgs &a) {
    constexpr int kD = R <= 7 ? 3 : kStripDepth;
    switch (nw) {
        case 1: return launch_strip<XT, S, 1, R, true, kNt, kD, false, kSplit>(a);
        case 2: return launch_strip<XT, S, 2, R, true, kNt, kD, false, kSplit>(a);
        default: return launch_strip<XT, S, 3, R, true, kNt, kD, false, kSplit>(a);
    }
}
template <int S, bool kNt, int XT = kDtypeBF16, bool kSplit = false>
hipError_t launch_strip_nat(int nw, int r, const StripArgs &a) {
    if (r == 14) return launch_strip_nat_nw<S, 14, kNt, XT, kSplit>(nw, a);
    if (r == 7) return launch_strip_nat_nw<S, 7, kNt, XT, kSplit>(nw, a);
    if (r >= 16) return launch_strip_nat_nw<S, 16, kNt, XT, kSplit>(nw, a);
    if (r >= 8) return launch_strip_nat_nw<S, 8, kNt, XT, kSplit>(nw, a);
    return launch_strip_nat_nw<S, 4, kNt, XT, kSplit>(nw, a);
}

template <int XT, int S, bool kNt = false, bool kStageB = false, bool kSplit = false>
hipError_t launch_strip_nr(int nw, int r, const StripArgs &a) {
    if constexpr (XT == kDtypeBF16 || kSplit) {
        if (r == 14) return launch_strip_nw<XT, S, 14, kNt, kStageB, kSplit>(nw, a);
        if (r == 7) return launch_strip_nw<XT, S, 7, kNt, kStageB, kSplit>(nw, a);
    }
    if (r >= 16) return launch_strip_nw<XT, S, 16, kNt, kStageB, kSplit>(nw, a);
    if (r >= 8) return launch_strip_nw<XT, S, 8, kNt, kStageB, kSplit>(nw, a);
    return launch_strip_nw<XT, S, 4, kNt, kStageB, kSplit>(nw, a);
}

// The weight loads of bf16 launches over at least this many packed bytes carry the
// non-temporal hint.  Measured on the config-3 / config-4 decode shapes (rotating weight
// copies, so every call streams from HBM): 4096 -> 14336, 14336 -> 4096, 3072 -> 9216 and
// 3072 -> 16384 take 2-5 % less time at one token (2-5 % at four on the two largest);
// 8192 -> 3072 (8.4 MB) takes 3-5 % more.
constexpr int64_t kStripNtMinBytes = int64_t{9} << 20;

// Fewer waves than this leave SIMDs idle: shorter strips are then worth their extra
// activation reads.
constexpr int64_t kStripMinWaves = 1200;

template <int XT>
hipError_t launch_strip_x(bool *handled, const void *x, const uint8_t *w, void *c, int m,
                          int64_t n, int64_t k, float alpha, float beta, const float *bias,
                          hipStream_t s) {
    *handled = false;
    const int64_t L = (k + kTrits - 1) / kTrits;
    if (m < 1 || m > 8 || n <= 0 || L <= 0) return hipSuccess;
    // bf16 at 5..8 tokens over >= 12288 rows and K <= 4096: S = 2 (8 rows x 8 limbs per
    // load, two kept entries per lane).  Against the stream kernel, same box: 4096 -> 14336
    // at 5 / 6 / 8 tokens 9.40 / 9.52 / 9.57 -> 8.68 / 8.74 / 8.83 us, 3072 -> 16384 7.88 /
    // 8.05 / 8.00 -> 6.29 / 6.31 / 6.70; even on 3072 -> 9216 (6.81 / 7.00 / 7.42 -> 6.70 /
    // 7.10 / 7.61); slower over a long K, where every wave streams several ranges (14336
    // -> 4096 11.24 -> 12.99 / 13.11 / 13.48, 8192 -> 3072 7.38 -> 8.74), and on 3072 ->
    // 3072.
    // int8 the same (4096 -> 14336 at 5 / 8 tokens 16.48 / 9.92 -> 8.65 / 8.65 us, 3072 ->
    // 16384 12.52 / 8.25 -> 6.34 / 6.50)
    if (m > 4 && !((XT == kDtypeBF16 || XT == kDtypeI8) && n >= 12288 && k <= 4096))
        return hipSuccess;
    // float32 at one or two tokens: hi and lo planes as B token columns (kSplit), so the
    // launch is shaped as bf16 at mc = 2 m tokens.  Against a second MFMA per operand
    // (same box): one token 4096 -> 14336 10.03 -> 7.39 us, 14336 -> 4096 10.63 -> 9.44,
    // 3072 -> 9216 6.45 -> 5.66, 3072 -> 16384 7.25 -> 6.25, but 8192 -> 3072 6.72 -> 8.77
    // and 3072 -> 3072 4.10 -> 4.43, so one token takes it from 4096 rows; two tokens
    // everywhere (4096 -> 14336 9.34 -> 7.85, 8192 -> 3072 9.71 -> 7.19, 3072 -> 3072 4.70
    // -> 3.99).
    // (three and four tokens, as S = 2, on the wide short-K shapes the S = 2 form takes:
    // 4096 -> 14336 at 3 / 4 tokens 9.54 / 10.26 -> 9.15 / 9.33 us, 3072 -> 16384 8.01 /
    // 8.92 -> 6.53 / 6.70; elsewhere slower, 14336 -> 4096 11.46 -> 14.09)
    const bool wide_short = n >= 12288 && k <= 4096;
    const bool split = XT == kDtypeF32 &&
                       (m == 2 || (m == 1 && n >= 4096) || (m <= 4 && wide_short));
    const int mc = split ? 2 * m : m;
    // S = 16 (one row x 64 limbs per load) for one token when it pads the row no more
    // than S = 8 does; S = 8 (2 rows x 32 limbs) up to 2 tokens; S = 4 up to 4.
    const int64_t pad16 = (L + 63) / 64 * 64;
    const int64_t pad8 = (L + 31) / 32 * 32;
    const int S = mc == 1 && pad16 <= pad8 ? 16 : (mc <= 2 ? 8 : (mc <= 4 ? 4 : 2));
    // buffer offsets within a workgroup's rows must stay below 2^31
    constexpr int64_t kElem = XT == kDtypeF32 ? 4 : (XT == kDtypeBF16 ? 2 : 1);
    if (64 * L * kTrytes >= 0x7FFFFFFF) return hipSuccess;
    const int64_t nranges = (L + 4 * S - 1) / (4 * S);
    // ranges per wave, then as few waves as that allows (balanced: 10 ranges -> 5 x 2)
    const int64_t per_wave = (nranges + kStripMaxWaves - 1) / kStripMaxWaves;
    const int nw = static_cast<int>((nranges + per_wave - 1) / per_wave);
    StripArgs a;
    a.x = x;
    a.w = w;
    a.c = c;
    a.m = m;
    a.n = n;
    a.k = k;
    a.L = static_cast<int>(L);
    a.nranges = static_cast<int>(nranges);
    a.aligned = (k % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % (kElem == 1 ? 8 : 16) == 0);
    a.alpha = alpha;
    a.beta = beta;
    a.bias = bias;
    a.s = s;
    *handled = true;
    // Loads per strip R: a wave reads 4*S*M*48 activations per range against R KB of
    // weights, so R starts at the first of 8, 16 that keeps that ratio (bf16 bytes) at
    // or below 0.4; then it halves, down to 4, while the launch has fewer than 1200
    // waves (longer strips also lengthen the compute tail after the last load).
    const double x_ratio8 = 4.0 * S * mc * kTrits * 2 / (8 * 1024.0);
    int r = x_ratio8 <= 0.4 ? 8 : 16;
    auto waves = [&](int rr) { return (n + rr * (16 / S) - 1) / (rr * (16 / S)) * nw; };
    while (r > 4 && waves(r) < kStripMinWaves) r /= 2;
    // bf16 (the decode case): one load fewer per strip when that evens out the
    // workgroups per CU, the busiest CU then streaming fewer rows (4096 x 14336:
    // 896 workgroups, 3.5 per CU, become 1024, 4 per CU, 7.3 -> 7.1 us).
    if ((XT == kDtypeBF16 || split) && (r == 8 || r == 16)) {
        const int64_t cus = cu_count();
        auto busiest = [&](int rr) {
            const int64_t blocks = (n + rr * (16 / S) - 1) / (rr * (16 / S));
            return (blocks + cus - 1) / cus * rr;
        };
        if (busiest(r - r / 8) < busiest(r)) r -= r / 8;
    }
    if constexpr (XT == kDtypeF32) {
        if (split) {
            // as bf16 at mc = 2 or 4 tokens: padded order, S = 8 / 4, the same hint
            const bool nt = n * L * kTrytes >= kStripNtMinBytes;
            if (S == 8)
                return nt ? launch_strip_nr<XT, 8, true, false, true>(nw, r, a)
                          : launch_strip_nr<XT, 8, false, false, true>(nw, r, a);
            if (S == 2)
                return nt ? launch_strip_nr<XT, 2, true, false, true>(nw, r, a)
                          : launch_strip_nr<XT, 2, false, false, true>(nw, r, a);
            return nt ? launch_strip_nr<XT, 4, true, false, true>(nw, r, a)
                      : launch_strip_nr<XT, 4, false, false, true>(nw, r, a);
        }
    }
    if constexpr (XT == kDtypeBF16) {
        const bool nt = n * L * kTrytes >= kStripNtMinBytes;
        if (m == 1 && ((S == 8 && nranges <= 3) || (S == 16 && nranges == 1))) {
            if (nt)
                return S == 16 ? launch_strip_nat<16, true>(nw, r, a)
                               : launch_strip_nat<8, true>(nw, r, a);
            return S == 16 ? launch_strip_nat<16, false>(nw, r, a)
                           : launch_strip_nat<8, false>(nw, r, a);
        }
        // staged B where waves stream several ranges (see gemv_strip_kernel); two to eight
        // tokens (S = 8, 4, 2)
        if (a.aligned && per_wave > 1 && S != 16) {
            if (S == 2)
                return nt ? launch_strip_nr<XT, 2, true, true>(nw, r, a)
                          : launch_strip_nr<XT, 2, false, true>(nw, r, a);
            if (nt)
                return S == 8 ? launch_strip_nr<XT, 8, true, true>(nw, r, a)
                              : launch_strip_nr<XT, 4, true, true>(nw, r, a);
            return S == 8 ? launch_strip_nr<XT, 8, false, true>(nw, r, a)
                          : launch_strip_nr<XT, 4, false, true>(nw, r, a);
        }
        if (nt) {
            switch (S) {
                case 16: return launch_strip_nr<XT, 16, true>(nw, r, a);
                case 8: return launch_strip_nr<XT, 8, true>(nw, r, a);
                case 4: return launch_strip_nr<XT, 4, true>(nw, r, a);
                default: return launch_strip_nr<XT, 2, true>(nw, r, a);
            }
        }
        if (S == 2) return launch_strip_nr<XT, 2>(nw, r, a);
    }
    switch (S) {
        case 16: return launch_strip_nr<XT, 16>(nw, r, a);
        case 8: return launch_strip_nr<XT, 8>(nw, r, a);
        case 4: return launch_strip_nr<XT, 4>(nw, r, a);
        default: return launch_strip_nr<XT, 2>(nw, r, a);
    }
}

}  // namespace

hipError_t launch_gemv_strip(bool *handled, const void *x, int x_dtype, const uint8_t *w,
                             void *c, int m, int64_t n, int64_t k, float alpha, float beta,
                             const float *bias, hipStream_t s) {
    switch (x_dtype) {
        case kDtypeBF16:
            return launch_strip_x<kDtypeBF16>(handled, x, w, c, m, n, k, alpha, beta, bias, s);
        case kDtypeF32:
            return launch_strip_x<kDtypeF32>(handled, x, w, c, m, n, k, alpha, beta, bias, s);
        default:
            return launch_strip_x<kDtypeI8>(handled, x, w, c, m, n, k, alpha, beta, bias, s);
    }
}

}  // namespace t81hip

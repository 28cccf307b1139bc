// t81lib_amd/csrc/gemv_diag.hip -- K2 for M <= 2 tokens: activations held in registers.
//
//   C[m, n] = alpha * sum_k X[m, k] * T[n, k] + beta * C[m, n] + bias[n]
//
// Same work split as gemv_wave_kernel (a wave streams a run of nsbw 4-limb
// sub-blocks of one 16-row group; the runs of a group are summed through LDS), but
// the B operand of the MFMA never moves.  v_mfma_f32_16x16x32_bf16 computes
// D = A B with column j of D depending only on column j of B; the kernel loads,
// once per wave, B-column j = (slot s, token m) with j = s * T + m: lane (j, q)
// holds the activations of token m for limb q of the run's sub-block s.  Slot f's
// six MFMAs (A = its decoded weights) go into their own accumulator acc[f], whose
// column f * T + m is then exactly sum_k T[row, k] * X[m, k] over that sub-block;
// the other columns are never read.  The trits are decoded in padded order (see
// decode_dword_padded): eight MFMAs per limb instead of six, but one table read and
// one bitfield extract per byte is the whole decode.  At the end each lane (j, q) picks acc[j / T]
// (a select over compile-time indices), and row-wise DPP shifts add the slots up,
// leaving token m's sums in lane 16 - T + m.  Per sub-block the work is then only
// the weight decode (16 table lookups) and eight MFMAs: no activation traffic at all.
//
// T = M (1 or 2), so a run holds at most 16 / T sub-blocks; R, the
// run length, is a template constant so every wave issues the same number of
// weight loads (exact s_waitcnt counts); a wave with nsbw < R points its spare
// loads past the buffer's range, where they return zeros without touching memory.
#include <algorithm>

#include "gemv_common.hpp"
#include "t81_device.hpp"
#include "t81_kernels.hpp"

namespace t81hip {

namespace {

constexpr int kDiagDepth = 4;          // weight loads in flight per wave
constexpr int kDiagMaxWaves = 8;       // waves per workgroup (W) at most
constexpr uint32_t kDiagOob = 0x80000000u;

// Decode in "padded" order: every tryte becomes four bf16 k-slots (t0, t1, t2, 0)
// through the E table alone (E[u] = {bf16(t0) | bf16(t1) << 16, bf16(t2)}), so one
// ds_read_b64 per byte lands a finished half of an MFMA operand: no shifts, ORs or
// moves to assemble.  A limb is 16 trytes = 64 k-slots = eight MFMAs; the
// activation operands carry a zero in every fourth slot to match.
__device__ __forceinline__ void decode_dword_padded(const uint8_t *lds, uint32_t w,
                                                    uint32_t *out) {
    const uint32_t w8 = w << 3;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const uint32_t a = (w8 >> (8 * b)) & 0xFFu;
        const uint2 e = *reinterpret_cast<const uint2 *>(lds + kLutE + a);
        out[2 * b] = e.x;
        out[2 * b + 1] = e.y;
    }
}

// Natural-order bf16 activations (24 dwords = 48 values) -> the eight padded operands:
// operand o = (x[6o], x[6o+1], x[6o+2], 0, x[6o+3], x[6o+4], x[6o+5], 0).
__device__ __forceinline__ void pad_operands(const bf16x8 *nat, bf16x8 *out) {
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

// acc0/acc1 += A x B over the eight padded operands of one limb (fp32: hi and lo
// planes), even operands into acc0 and odd ones into acc1: two independent MFMA
// chains of four instead of one of eight.
template <int XT>
__device__ __forceinline__ void mfma_padded(const uint32_t *pairs, const bf16x8 *bh,
                                            const bf16x8 *bl, floatx4 &acc0, floatx4 &acc1) {
#pragma unroll
    for (int o = 0; o < 8; ++o) {
        const u32x4 araw = {pairs[4 * o], pairs[4 * o + 1], pairs[4 * o + 2], pairs[4 * o + 3]};
        const bf16x8 a = __builtin_bit_cast(bf16x8, araw);
        floatx4 &acc = (o & 1) ? acc1 : acc0;
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bh[o], acc, 0, 0, 0);
        if constexpr (XT == kDtypeF32)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl[o], acc, 0, 0, 0);
    }
}

// v += v of lane (lane - S) in the same 16-lane row; lanes below S add 0.
template <int S>
__device__ __forceinline__ void add_row_shr(floatx4 &v) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int moved =
            __builtin_amdgcn_update_dpp(0, __float_as_int(v[t]), 0x110 + S, 0xF, 0xF, true);
        v[t] += __int_as_float(moved);
    }
}

// At least 2 waves per SIMD (<= 256 registers each): the launch rarely has more than
// 2048 waves, and left alone the compiler sometimes trades occupancy for registers.
template <int XT, int W, int T, int R>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2))) void gemv_diag_kernel(
    const void *__restrict__ x, const uint8_t *__restrict__ w, void *__restrict__ c, int M,
    int64_t N, int64_t K, int L, int nsb, int wg, int x_aligned, float alpha, float beta,
    const float *__restrict__ bias) {
    static_assert(R * T <= 16, "a run's slots must fit in the 16 columns");
    __shared__ __attribute__((aligned(16))) uint8_t lut[kLutBytes];
    __shared__ float red[W][T][16];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15;  // A: weight row of the group; B: column (slot, token)
    const int q = lane >> 4;    // limb of the sub-block
    const int G = W / wg;
    const int g = wave / wg;
    const int p = wave - g * wg;
    const int64_t group = static_cast<int64_t>(blockIdx.x) * G + g;
    const int64_t groups = (N + 15) / 16;
    const int64_t n0 = group * 16;
    const int s0 = (p * nsb) / wg;
    const int nsbw = group < groups ? ((p + 1) * nsb) / wg - s0 : 0;

    // ---- 1. B operands: column col = slot sl * T + token m, limb q ----
    const int sl = col / T;
    const int m = col % T;
    const bool xvalid = sl < nsbw && m < M;
    const int64_t kq = static_cast<int64_t>(4 * (s0 + sl) + q) * kTrits;
    const int64_t xrow = static_cast<int64_t>(m < M ? m : 0) * K;
    XRaw xr[6];
    if (x_aligned) {
#pragma unroll
        for (int j = 0; j < 6; ++j) xr[j] = load_x8_raw<XT, true>(x, xrow, kq + 8 * j, K, xvalid);
    } else {
#pragma unroll
        for (int j = 0; j < 6; ++j) xr[j] = load_x8_raw<XT, false>(x, xrow, kq + 8 * j, K, xvalid);
    }

    // ---- 2. weights: buffer based at the group's first row, rows past N read zeros ----
    const int64_t remain = group < groups ? (N - n0) * L * kTrytes : 0;
    const int nrec = remain < 0x7FFFFFFF ? static_cast<int>(remain) : 0x7FFFFFFF;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(group < groups ? w + n0 * L * kTrytes : w), 0, nrec, 0x00020000);
    const uint32_t lane_base = static_cast<uint32_t>((col * L + 4 * s0 + q) * kTrytes);
    auto fetch = [&](int f) -> u32x4 {
        const uint32_t off = f < nsbw ? lane_base + 64u * static_cast<uint32_t>(f) : kDiagOob;
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
    };
    constexpr int D = R < kDiagDepth ? R : kDiagDepth;
    u32x4 ring[D];  // sub-block f lives in ring[f % D]
#pragma unroll
    for (int i = 0; i < D; ++i) ring[i] = fetch(i);

    // ---- 3. decode tables (shared, fixed address: lookups need no base add) ----
    lut_fill(lut, tid, 64 * W);
    __syncthreads();

    bf16x8 nh[6], nl[6], bh[8], bl[8];
#pragma unroll
    for (int j = 0; j < 6; ++j) cvt_x8<XT>(xr[j], nh[j], nl[j]);
    pad_operands(nh, bh);
    if constexpr (XT == kDtypeF32) pad_operands(nl, bl);

    // ---- 4. stream: one accumulator per sub-block ----
    floatx4 acc[R][2];
#pragma unroll
    for (int f = 0; f < R; ++f) acc[f][0] = acc[f][1] = floatx4{0.f, 0.f, 0.f, 0.f};
    // Straight-line code, no branch per slot, software-pipelined: the table lookups of
    // sub-block f + 1 are issued before the MFMAs of sub-block f, so their latency hides
    // behind the MFMAs.  Slots past nsbw run on zeros (their loads are out of range) and
    // their B columns are zero, so acc[f] for f >= nsbw only ever holds 0 in the one
    // column that is read.
    uint32_t cur[32], nxt[32];
#pragma unroll
    for (int d = 0; d < 4; ++d) decode_dword_padded(lut, ring[0][d], cur + 8 * d);
    __builtin_amdgcn_sched_barrier(0);
    if (D < R) ring[0] = fetch(D);
#pragma unroll
    for (int f = 0; f < R; ++f) {
        if (f + 1 < R) {
#pragma unroll
            for (int d = 0; d < 4; ++d)
                decode_dword_padded(lut, ring[(f + 1) % D][d], nxt + 8 * d);
            // the refill reuses the slot's registers once they are decoded
            __builtin_amdgcn_sched_barrier(0);
            if (f + 1 + D < R) ring[(f + 1) % D] = fetch(f + 1 + D);
        }
        mfma_padded<XT>(cur, bh, bl, acc[f][0], acc[f][1]);
#pragma unroll
        for (int i = 0; i < 32; ++i) cur[i] = nxt[i];
    }

    // ---- 5. lane (col, q) keeps column col of acc[col / T], then the slots are summed ----
    floatx4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int f = 0; f < R; ++f)
        if (sl == f) v = acc[f][0] + acc[f][1];
    // row_shr:s (DPP) brings lane col - s of the same 16-lane row (0 past the row start)
    add_row_shr<8>(v);
    if constexpr (T <= 4) add_row_shr<4>(v);
    if constexpr (T <= 2) add_row_shr<2>(v);
    if constexpr (T <= 1) add_row_shr<1>(v);
    // token m's partial sums (rows 4q .. 4q+3 of the group) are now in lane 16 - T + m
    if (col >= 16 - T) {
#pragma unroll
        for (int t = 0; t < 4; ++t) red[wave][col - (16 - T)][4 * q + t] = v[t];
    }
    __syncthreads();

    // ---- 6. per group: the wg runs in wave order, one output per thread ----
    const float *redf = &red[0][0][0];
    for (int e = tid; e < G * T * 16; e += 64 * W) {
        const int gg = e / (T * 16);
        const int mm = (e / 16) % T;
        const int row = e % 16;
        float val = 0.0f;
        for (int pp = 0; pp < wg; ++pp) val += redf[((gg * wg + pp) * T + mm) * 16 + row];
        const int64_t n = (static_cast<int64_t>(blockIdx.x) * G + gg) * 16 + row;
        if (mm < M && n < N) {
            if constexpr (XT == kDtypeI8) {
                int32_t *cp = static_cast<int32_t *>(c) + static_cast<int64_t>(mm) * N + n;
                int32_t y = static_cast<int32_t>(val);
                if (beta != 0.0f) y += *cp;
                *cp = y;
            } else {
                float *cp = static_cast<float *>(c) + static_cast<int64_t>(mm) * N + n;
                float y = alpha * val;
                if (beta != 0.0f) y = y + beta * *cp;
                if (bias != nullptr) y = y + bias[n];
                *cp = y;
            }
        }
    }
}

struct DiagArgs {
    const void *x;
    const uint8_t *w;
    void *c;
    int m;
    int64_t n, k;
    int L, nsb, wg;
    bool aligned;
    float alpha, beta;
    const float *bias;
    hipStream_t s;
};

template <int XT, int W, int T, int R>
hipError_t launch_diag(const DiagArgs &a) {
    const int G = W / a.wg;
    const int64_t groups = (a.n + 15) / 16;
    gemv_diag_kernel<XT, W, T, R><<<dim3((groups + G - 1) / G), dim3(64 * W), 0, a.s>>>(
        a.x, a.w, a.c, a.m, a.n, a.k, a.L, a.nsb, a.wg, a.aligned ? 1 : 0, a.alpha, a.beta,
        a.bias);
    return hipGetLastError();
}

// Run length R: every value for bf16 activations (the decode case); multiples of 4
// for fp32 and int8.
template <int XT, int W, int T, int R = 16 / T>
hipError_t launch_diag_r(int run, const DiagArgs &a) {
    if constexpr (R <= 1) {
        return launch_diag<XT, W, T, 1>(a);
    } else if constexpr (XT != kDtypeBF16 && R % 4 != 0) {
        return launch_diag_r<XT, W, T, R - 1>(run, a);
    } else {
        const int lower = XT == kDtypeBF16 ? R - 1 : R - 4;
        if (run > lower || (XT != kDtypeBF16 && R == 4)) return launch_diag<XT, W, T, R>(a);
        return launch_diag_r<XT, W, T, R - 1>(run, a);
    }
}

template <int XT, int W>
hipError_t launch_diag_t(int t, int run, const DiagArgs &a) {
    if (t == 1) return launch_diag_r<XT, W, 1>(run, a);
    return launch_diag_r<XT, W, 2>(run, a);
}

// Waves in flight the kernel aims for before it splits K finer.
constexpr int64_t kDiagTargetWaves = 1024;

template <int XT>
hipError_t launch_diag_x(bool *handled, const void *x, const uint8_t *w, void *c, int m,
                         int64_t n, int64_t k, float alpha, float beta, const float *bias,
                         hipStream_t s) {
    *handled = false;
    const int64_t L = (k + kTrits - 1) / kTrits;
    // M = 3, 4 (T = 4, runs of at most 4 sub-blocks) measured slower than gemv_wave_kernel
    if (m < 1 || m > 2 || L <= 0 || L > (1 << 22)) return hipSuccess;
    const int T = m;  // 1 or 2
    const int64_t max_run = 16 / T;
    const int64_t groups = (n + 15) / 16;
    const int64_t nsb = (L + 3) / 4;
    int wg = 1;
    while (wg <= kDiagMaxWaves && nsb > max_run * wg) wg *= 2;
    if (wg > kDiagMaxWaves) return hipSuccess;
    while (wg < kDiagMaxWaves && groups * wg < kDiagTargetWaves && nsb >= 4 * wg) wg *= 2;
    const int W = wg < 4 ? 4 : wg;
    DiagArgs a;
    a.x = x;
    a.w = w;
    a.c = c;
    a.m = m;
    a.n = n;
    a.k = k;
    a.L = static_cast<int>(L);
    a.nsb = static_cast<int>(nsb);
    a.wg = wg;
    constexpr int elem = XT == kDtypeF32 ? 4 : (XT == kDtypeBF16 ? 2 : 1);
    a.aligned = (k % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % (elem == 1 ? 8 : 16) == 0);
    a.alpha = alpha;
    a.beta = beta;
    a.bias = bias;
    a.s = s;
    const int run = static_cast<int>((nsb + wg - 1) / wg);
    *handled = true;
    if (W == 4) return launch_diag_t<XT, 4>(T, run, a);
    return launch_diag_t<XT, 8>(T, run, a);
}

}  // namespace

hipError_t launch_gemv_diag(bool *handled, const void *x, int x_dtype, const uint8_t *w, void *c,
                            int m, int64_t n, int64_t k, float alpha, float beta,
                            const float *bias, hipStream_t s) {
    switch (x_dtype) {
        case kDtypeBF16:
            return launch_diag_x<kDtypeBF16>(handled, x, w, c, m, n, k, alpha, beta, bias, s);
        case kDtypeF32:
            return launch_diag_x<kDtypeF32>(handled, x, w, c, m, n, k, alpha, beta, bias, s);
        default:
            return launch_diag_x<kDtypeI8>(handled, x, w, c, m, n, k, alpha, beta, bias, s);
    }
}

}  // namespace t81hip

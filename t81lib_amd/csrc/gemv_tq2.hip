// t81lib_amd/csrc/gemv_tq2.hip -- decode-shaped matmul straight from GGUF TQ2_0 weights.
//
//   C[m, n] = alpha * sum_k X[m, k] * W[n, k] + beta * C[m, n] + bias[n],
//   W[n, 256 b + e] = d[n, b] * (digit(n, b, e) - 1)
//
// TQ2_0 (llama.cpp ggml block_tq2_0, written by t81/gguf.py:601-615): a row of K
// weights is B = ceil(K / 256) blocks of 66 bytes, 64 bytes of 2-bit digits (byte
// a*32 + c holds elements a*128 + s*32 + c at bits 2s) and the half scale d.  At
// 2.06 bits per weight it streams 23 % fewer bytes than the 16-byte limb layout.
//
// Same column-strip organisation as gemv_strip.hip: a workgroup owns H = R * 16 / S
// rows, wave w streams blocks [w*S, w*S + S) of every row ("range"), and a load t
// covers 16 / S rows x S blocks.  Lane (i, q) holds piece q (qs bytes 16q .. 16q+15,
// 64 digits) of block l0 + i % S of row row0 + t*16/S + i / S: the four quarter-lanes
// of an A row hold the four pieces of one block, so the matched MFMA entries
// D[i][j] (j % S == i % S, token j / S) are whole-block dot products.  Lane (j, q)
// keeps element j % 4 (its one matched entry, if any) times that block's scale.
// The B operand (the activations of token j / S for piece q of block l0 + j % S, in
// the order the digits decode) is loaded once per range and stays in registers.
//
// Blocks are 66 bytes, so a piece is only 2-byte aligned: each lane reads the five
// aligned dwords that cover it and funnel-shifts by 16 bits when needed.  Bytes
// decode through a 2 KB LDS table (byte -> four bf16 values digit - 1), eight
// MFMAs (v_mfma_f32_16x16x32_bf16) per piece with no padding slots.  Blocks past B
// read zeros (out-of-range offsets) and meet zero activations and a zero scale;
// rows past N read zeros and are not stored.  Partial sums go through LDS and every
// output sums its S sub-sums per range over the ranges in a fixed order.
#include <hip/hip_fp16.h>

#include <algorithm>

#include "gemv_common.hpp"
#include "t81_device.hpp"
#include "t81_kernels.hpp"

namespace t81hip {

namespace {

constexpr int kTq2Bytes = 66;
constexpr int kTq2MaxWaves = 8;
// Loads in flight per wave, refilled as each is decoded: three for one or two tokens
// (S = 8), four above (llama.gate M = 1 6.99 -> 6.84 us with three; M = 4 7.90 -> 8.08).
// The non-temporal hint that helps the limb strip kernel measured 6.99 -> 7.91 us here
// (each piece's 4-byte tail load re-reads the line that the next piece's load streams).
template <int S>
constexpr int tq2_depth() { return S == 8 ? 3 : 4; }
constexpr uint32_t kTq2Oob = 0x80000000u;
constexpr int kTq2LutWords = 512;  // 256 entries x 8 bytes

// entry[b] = { bf16(q0 - 1) | bf16(q1 - 1) << 16, bf16(q2 - 1) | bf16(q3 - 1) << 16 },
// q_s = (b >> 2s) & 3 (a digit of 3 decodes to 2, as the reference's dequantizer does).
__device__ __forceinline__ uint32_t tq2_bf16_of_digit(uint32_t q) {
    return q == 0 ? 0xBF80u : (q == 1 ? 0u : (q == 2 ? 0x3F80u : 0x4000u));
}

__device__ __forceinline__ void tq2_lut_fill(uint32_t *lut, int tid, int nthreads) {
    for (int w = tid; w < kTq2LutWords; w += nthreads) {
        const uint32_t b = static_cast<uint32_t>(w >> 1);
        const int s = 2 * (w & 1);
        lut[w] = tq2_bf16_of_digit((b >> (2 * s)) & 3u) |
                 (tq2_bf16_of_digit((b >> (2 * s + 2)) & 3u) << 16);
    }
}

// One piece (16 bytes) -> 32 dwords: for byte u, dwords 2u, 2u+1 = the four decoded digits.
__device__ __forceinline__ void tq2_decode(const uint8_t *lut, const uint32_t *p, uint32_t *out) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint32_t a = (b == 0 ? (p[k] << 3) : (p[k] >> (8 * b - 3))) & 0x7F8u;
            const uint2 e = *reinterpret_cast<const uint2 *>(lut + a);
            out[8 * k + 2 * b] = e.x;
            out[8 * k + 2 * b + 1] = e.y;
        }
    }
}

template <int XT>
__device__ __forceinline__ floatx4 tq2_mfma(const uint32_t *pairs, const bf16x8 *bh,
                                            const bf16x8 *bl) {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int o = 0; o < 8; ++o) {
        const u32x4 araw = {pairs[4 * o], pairs[4 * o + 1], pairs[4 * o + 2], pairs[4 * o + 3]};
        const bf16x8 a = __builtin_bit_cast(bf16x8, araw);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bh[o], acc, 0, 0, 0);
        if constexpr (XT == kDtypeF32)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl[o], acc, 0, 0, 0);
    }
    return acc;
}

__device__ __forceinline__ float tq2_keep(floatx4 v, int j) {
    const float lo = (j & 1) ? v[1] : v[0];
    const float hi = (j & 1) ? v[3] : v[2];
    return (j & 2) ? hi : lo;
}

// Activation operands for one piece: element of slot (byte u, digit s) is
// k0 + s * 32 + u (k0 = 256 * block + (q / 2) * 128 + (q % 2) * 16); operand o holds
// bytes 2o and 2o + 1, four digits each.  v16[s] = the 16 values k0 + s*32 + [0, 16).
__device__ __forceinline__ void tq2_operands(const bf16x8 (&v16)[4][2], bf16x8 *out) {
    auto half = [&](int s, int u) -> uint32_t {
        const u32x4 w = __builtin_bit_cast(u32x4, v16[s][u >> 3]);
        const uint32_t d = w[(u & 7) >> 1];
        return (u & 1) ? (d >> 16) : (d & 0xFFFFu);
    };
#pragma unroll
    for (int o = 0; o < 8; ++o) {
        const int u0 = 2 * o, u1 = 2 * o + 1;
        const u32x4 q = {half(0, u0) | (half(1, u0) << 16), half(2, u0) | (half(3, u0) << 16),
                         half(0, u1) | (half(1, u1) << 16), half(2, u1) | (half(3, u1) << 16)};
        out[o] = __builtin_bit_cast(bf16x8, q);
    }
}

template <int XT, int S, int NW, int R>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void gemv_tq2_kernel(
    const void *__restrict__ x, const uint8_t *__restrict__ w, float *__restrict__ c, int M,
    int64_t N, int64_t K, int B, int nranges, int x_aligned, float alpha, float beta,
    const float *__restrict__ bias) {
    static_assert(S == 4 || S == 8, "one matched entry per lane");
    constexpr int RPI = 16 / S;
    constexpr int H = R * RPI;
    constexpr int D = R < tq2_depth<S>() ? R : tq2_depth<S>();
    __shared__ __attribute__((aligned(16))) uint32_t lut[kTq2LutWords];
    __shared__ float red[NW][R][64];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 15;
    const int q = lane >> 4;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * H;
    const uint32_t row_bytes = static_cast<uint32_t>(B) * kTq2Bytes;

    const int64_t remain = (N - row0) * row_bytes;
    const int nrec = remain < 0x7FFFFFFF ? static_cast<int>(remain) : 0x7FFFFFFF;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(w + row0 * row_bytes), 0, nrec, 0x00020000);

    float kept[R];
#pragma unroll
    for (int t = 0; t < R; ++t) kept[t] = 0.0f;

    bool first = true;
    for (int rg = wave; rg < nranges; rg += NW) {
        const int l0 = rg * S;
        // ---- B: token i / S, block l0 + i % S, piece q ----
        const int mb = i / S;
        const int bb = l0 + i % S;
        const bool bvalid = mb < M && bb < B;
        const int64_t xrow = static_cast<int64_t>(mb < M ? mb : 0) * K;
        const int64_t k0 = static_cast<int64_t>(bb) * 256 + (q >> 1) * 128 + (q & 1) * 16;
        XRaw xr[4][2];
        if (x_aligned) {
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    xr[s][h] = load_x8_raw<XT, true>(x, xrow, k0 + 32 * s + 8 * h, K, bvalid);
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    xr[s][h] = load_x8_raw<XT, false>(x, xrow, k0 + 32 * s + 8 * h, K, bvalid);
        }

        // ---- A: piece q of block l0 + i % S of row t * RPI + i / S; scale of the kept entry ----
        const bool ablk = l0 + i % S < B;
        const uint32_t piece_off = static_cast<uint32_t>(i / S) * row_bytes +
                                   static_cast<uint32_t>(l0 + i % S) * kTq2Bytes + 16u * q;
        // the kept entry of lane (j = i, q): row (4q + i % 4) / S, block l0 + i % S
        const uint32_t scale_off = static_cast<uint32_t>((4 * q + (i & 3)) / S) * row_bytes +
                                   static_cast<uint32_t>(l0 + i % S) * kTq2Bytes + 64u;
        struct Load {
            u32x4 a;
            uint32_t b;
            uint32_t d;
        };
        auto fetch = [&](int t) -> Load {
            const uint32_t row_add = static_cast<uint32_t>(t * RPI) * row_bytes;
            const uint32_t off = ablk ? ((piece_off + row_add) & ~3u) : kTq2Oob;
            const uint32_t soff = ablk ? scale_off + row_add : kTq2Oob;
            Load ld;
            ld.a = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
            ld.b = __builtin_amdgcn_raw_buffer_load_b32(rsrc, off + 16u, 0, 0);
            ld.d = __builtin_amdgcn_raw_buffer_load_b16(rsrc, soff, 0, 0);
            return ld;
        };
        // pieces start 2 bytes into a dword when block (row * B + block) is odd
        const uint32_t shift = (piece_off & 2u) * 8u;  // RPI * row_bytes % 4 == 0: fixed per lane
        auto piece = [&](const Load &ld, uint32_t *p) {
            p[0] = __builtin_amdgcn_alignbit(ld.a[1], ld.a[0], shift);
            p[1] = __builtin_amdgcn_alignbit(ld.a[2], ld.a[1], shift);
            p[2] = __builtin_amdgcn_alignbit(ld.a[3], ld.a[2], shift);
            p[3] = __builtin_amdgcn_alignbit(ld.b, ld.a[3], shift);
        };
        Load ring[D];
#pragma unroll
        for (int t = 0; t < D; ++t) ring[t] = fetch(t);

        if (first) {
            tq2_lut_fill(lut, tid, 64 * NW);
            __syncthreads();
            first = false;
        }

        bf16x8 v16h[4][2], v16l[4][2], bh[8], bl[8];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int h = 0; h < 2; ++h) cvt_x8<XT>(xr[s][h], v16h[s][h], v16l[s][h]);
        tq2_operands(v16h, bh);
        if constexpr (XT == kDtypeF32) tq2_operands(v16l, bl);

        const uint8_t *lutb = reinterpret_cast<const uint8_t *>(lut);
        uint32_t cur[32], nxt[32], p[4];
        float dcur = 0.0f, dnxt = 0.0f;
        piece(ring[0], p);
        tq2_decode(lutb, p, cur);
        dcur = __half2float(__ushort_as_half(static_cast<uint16_t>(ring[0].d)));
        __builtin_amdgcn_sched_barrier(0);
        if (D < R) ring[0] = fetch(D);
        floatx4 prev = {0.f, 0.f, 0.f, 0.f};
        float dprev = 0.0f;
#pragma unroll
        for (int t = 0; t < R; ++t) {
            if (t + 1 < R) {
                piece(ring[(t + 1) % D], p);
                tq2_decode(lutb, p, nxt);
                dnxt = __half2float(__ushort_as_half(static_cast<uint16_t>(ring[(t + 1) % D].d)));
                __builtin_amdgcn_sched_barrier(0);
                if (t + 1 + D < R) ring[(t + 1) % D] = fetch(t + 1 + D);
            }
            const floatx4 acc = tq2_mfma<XT>(cur, bh, bl);
            if (t > 0) kept[t - 1] += dprev * tq2_keep(prev, i);
            prev = acc;
            dprev = dcur;
            dcur = dnxt;
#pragma unroll
            for (int e = 0; e < 32; ++e) cur[e] = nxt[e];
        }
        kept[R - 1] += dprev * tq2_keep(prev, i);
    }
    if (first) {
        tq2_lut_fill(lut, tid, 64 * NW);
        __syncthreads();
    }

#pragma unroll
    for (int t = 0; t < R; ++t) red[wave][t][lane] = kept[t];
    __syncthreads();

    const int nw_used = nranges < NW ? nranges : NW;
    for (int e = tid; e < H * RPI; e += 64 * NW) {
        const int r = e / RPI;
        const int m = e % RPI;
        const int t = r / RPI;
        const int ra = r % RPI;
        const int64_t n = row0 + r;
        if (m >= M || n >= N) continue;
        float val = 0.0f;
        for (int ww = 0; ww < nw_used; ++ww) {
#pragma unroll
            for (int ss = 0; ss < S; ++ss) val += red[ww][t][m * S + ss + 16 * ((ra * S + ss) >> 2)];
        }
        float *cp = c + static_cast<int64_t>(m) * N + n;
        float y = alpha * val;
        if (beta != 0.0f) y = y + beta * *cp;
        if (bias != nullptr) y = y + bias[n];
        *cp = y;
    }
}

struct Tq2Args {
    const void *x;
    const uint8_t *w;
    float *c;
    int m;
    int64_t n, k;
    int B, nranges;
    bool aligned;
    float alpha, beta;
    const float *bias;
    hipStream_t s;
};

template <int XT, int S, int NW, int R>
hipError_t launch_tq2(const Tq2Args &a) {
    constexpr int H = R * (16 / S);
    const int64_t blocks = (a.n + H - 1) / H;
    gemv_tq2_kernel<XT, S, NW, R><<<dim3(static_cast<unsigned>(blocks)), dim3(64 * NW), 0, a.s>>>(
        a.x, a.w, a.c, a.m, a.n, a.k, a.B, a.nranges, a.aligned ? 1 : 0, a.alpha, a.beta, a.bias);
    return hipGetLastError();
}

template <int XT, int S, int R>
hipError_t launch_tq2_nw(int nw, const Tq2Args &a) {
    switch (nw) {
        case 1: return launch_tq2<XT, S, 1, R>(a);
        case 2: return launch_tq2<XT, S, 2, R>(a);
        case 3: return launch_tq2<XT, S, 3, R>(a);
        case 4: return launch_tq2<XT, S, 4, R>(a);
        case 5: return launch_tq2<XT, S, 5, R>(a);
        case 6: return launch_tq2<XT, S, 6, R>(a);
        case 7: return launch_tq2<XT, S, 7, R>(a);
        default: return launch_tq2<XT, S, 8, R>(a);
    }
}

// Eight block loads per strip, or seven when that lowers the busiest CU's share of
// the workgroups (4096 -> 14336: 896 workgroups, 3.5 per CU, become 1024, 4 per CU).
template <int XT, int S>
hipError_t launch_tq2_r(int nw, const Tq2Args &a) {
    const int64_t cus = cu_count();
    auto busiest = [&](int64_t r) {
        const int64_t blocks = (a.n + r * (16 / S) - 1) / (r * (16 / S));
        return (blocks + cus - 1) / cus * r;
    };
    if (busiest(7) < busiest(8)) return launch_tq2_nw<XT, S, 7>(nw, a);
    return launch_tq2_nw<XT, S, 8>(nw, a);
}

// One launch for up to four tokens.
template <int XT>
hipError_t launch_tq2_group(const void *x, const uint8_t *w, float *c, int m, int64_t n, int64_t k,
                            float alpha, float beta, const float *bias, hipStream_t s) {
    const int64_t B = (k + 255) / 256;
    const int S = m <= 2 ? 8 : 4;
    const int64_t nranges = (B + S - 1) / S;
    const int64_t per_wave = std::max<int64_t>(1, (nranges + kTq2MaxWaves - 1) / kTq2MaxWaves);
    const int nw = static_cast<int>(std::max<int64_t>(1, (nranges + per_wave - 1) / per_wave));
    Tq2Args a;
    a.x = x;
    a.w = w;
    a.c = c;
    a.m = m;
    a.n = n;
    a.k = k;
    a.B = static_cast<int>(B);
    a.nranges = static_cast<int>(nranges);
    constexpr int kElem = XT == kDtypeF32 ? 4 : (XT == kDtypeBF16 ? 2 : 1);
    a.aligned = (k % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % (kElem == 1 ? 8 : 16) == 0);
    a.alpha = alpha;
    a.beta = beta;
    a.bias = bias;
    a.s = s;
    if (S == 8) return launch_tq2_r<XT, 8>(nw, a);
    return launch_tq2_r<XT, 4>(nw, a);
}

template <int XT>
hipError_t launch_tq2_x(const void *x, const uint8_t *w, float *c, int64_t m, int64_t n, int64_t k,
                        float alpha, float beta, const float *bias, hipStream_t s) {
    constexpr int64_t kElem = XT == kDtypeF32 ? 4 : (XT == kDtypeBF16 ? 2 : 1);
    // tokens in groups of four; each group writes its own rows of C
    for (int64_t m0 = 0; m0 < m; m0 += 4) {
        const int mg = static_cast<int>(std::min<int64_t>(4, m - m0));
        const void *xg = static_cast<const uint8_t *>(x) + m0 * k * kElem;
        const hipError_t e =
            launch_tq2_group<XT>(xg, w, c + m0 * n, mg, n, k, alpha, beta, bias, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

bool tq2_matmul_fits(int64_t n, int64_t k) {
    const int64_t row_bytes = (k + 255) / 256 * kTq2Bytes;
    return row_bytes >= 0 && 32 * row_bytes < 0x7FFFFFFF && n < (int64_t{1} << 40);
}

hipError_t launch_tq2_matmul(const void *x, int x_dtype, const uint8_t *w, float *c, int64_t m,
                             int64_t n, int64_t k, float alpha, float beta, const float *bias,
                             hipStream_t s) {
    if (m == 0 || n == 0) return hipSuccess;
    switch (x_dtype) {
        case kDtypeBF16: return launch_tq2_x<kDtypeBF16>(x, w, c, m, n, k, alpha, beta, bias, s);
        case kDtypeF32: return launch_tq2_x<kDtypeF32>(x, w, c, m, n, k, alpha, beta, bias, s);
        default: return launch_tq2_x<kDtypeI8>(x, w, c, m, n, k, alpha, beta, bias, s);
    }
}

}  // namespace t81hip

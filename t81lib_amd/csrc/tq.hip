// t81lib_amd/csrc/tq.hip -- GGUF ternary block codecs: TQ1_0 and TQ2_0 (llama.cpp's
// ggml block_tq1_0 / block_tq2_0, 256 weights per block), as the reference writes and
// reads them in t81/gguf.py:518-663 and 1020-1069.
//
// One wavefront per block.  Quantize: d = max |v| over the block (NaN if any value is
// NaN), inv_d = 0 if d == 0 else 1 / d, trit of v * inv_d (threshold form
// |v| >= thr -> sign, else round half away from zero clipped to [-1, 1]), digit
// q = trit + 1; the scale is stored as IEEE half (round to nearest even).
//  TQ2_0 (66 B): byte a*32 + c holds the digits of elements a*128 + s*32 + c at
//   bits 2s (a < 2, s < 4, c < 32); then the half scale.
//  TQ1_0 (54 B): bytes 0..31 hold base-3 numbers of 5 digits (first weighted 81)
//   over elements i*32 + c, bytes 32..47 over 160 + i*16 + c, bytes 48..51 four
//   digits weighted 81, 27, 9, 3 over 240 + i*4 + c; a number v < 243 is stored as
//   (v * 256 + 242) / 243, so digit n reads back as ((uint8)(byte * 3^n) * 3) >> 8.
// All float arithmetic is float32 with separate roundings (no contraction), as numpy
// evaluates it.  Rows are zero-padded to whole blocks.  Dequantize writes with the
// non-temporal hint (every output byte is written once); whole-block rows into an
// aligned output as one float4 per lane.
#include <hip/hip_fp16.h>

#include "t81_device.hpp"
#include "t81_kernels.hpp"

#pragma clang fp contract(off)

namespace t81hip {

namespace {

constexpr int kQK = 256;
constexpr int kTq1 = 34;
constexpr int kTq2 = 35;

__host__ __device__ constexpr int tq_bytes(int quant) { return quant == kTq1 ? 54 : 66; }

__device__ __forceinline__ int tq_trit(float v, int use_thr, float thr) {
    if (use_thr) {
        if (!(fabsf(v) >= thr)) return 0;
        return v > 0.0f ? 1 : (v < 0.0f ? -1 : 0);
    }
    if (v != v) return 0;
    float r = v >= 0.0f ? floorf(v + 0.5f) : ceilf(v - 0.5f);
    r = r > 1.0f ? 1.0f : (r < -1.0f ? -1.0f : r);
    return static_cast<int>(r);
}

// Max over the wavefront (lane values >= 0 or NaN-free by construction).
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// Whole blocks of a 16-byte aligned matrix (cols a multiple of 256): lane l reads values
// 4 l .. 4 l + 3 of its wavefront's block with one non-temporal float4 (each value is read
// once), takes the block max from those, turns them into digits (trit + 1) and writes the
// four digits to the wavefront's 256-byte LDS slot; each lane then gathers the digits its
// output byte packs, in the layouts described at the top.  The slot is private to the
// wavefront, whose LDS operations complete in order, so no barrier is needed.
// (8192 x 3072: TQ1_0 63.5 -> 26.1 us, TQ2_0 57.7 -> 24.3 against tq_quantize_kernel.)
template <int Q>
__global__ __launch_bounds__(256) void tq_quantize_vec_kernel(const float *__restrict__ src,
                                                              uint8_t *__restrict__ dst,
                                                              int64_t blocks, float thr,
                                                              int use_thr) {
    __shared__ uint32_t slots[4][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t blk = static_cast<int64_t>(blockIdx.x) * 4 + wave;
    if (blk >= blocks) return;  // whole wavefront
    const floatx4 x =
        __builtin_nontemporal_load(reinterpret_cast<const floatx4 *>(src + blk * kQK) + lane);
    float mx = 0.0f;
    bool nan = false;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const float a = fabsf(x[u]);
        nan |= a != a;
        mx = fmaxf(mx, a);
    }
    mx = wave_max(mx);
    const float d = __builtin_amdgcn_ballot_w64(nan) != 0 ? __builtin_nanf("") : mx;
    const float inv_d = d == 0.0f ? 0.0f : 1.0f / d;
    uint32_t dig = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u)
        dig |= static_cast<uint32_t>(tq_trit(x[u] * inv_d, use_thr, thr) + 1) << (8 * u);
    slots[wave][lane] = dig;
    __builtin_amdgcn_wave_barrier();
    const uint8_t *sd = reinterpret_cast<const uint8_t *>(slots[wave]);
    uint8_t *out = dst + blk * tq_bytes(Q);
    if constexpr (Q == kTq2) {
        const int a = lane >> 5;
        const int c = lane & 31;
        uint32_t b = 0;
#pragma unroll
        for (int s = 0; s < 4; ++s) b |= static_cast<uint32_t>(sd[a * 128 + s * 32 + c]) << (2 * s);
        out[lane] = static_cast<uint8_t>(b);
    } else {
        if (lane < 52) {
            int first, stride, ndig;
            if (lane < 32) {
                first = lane, stride = 32, ndig = 5;
            } else if (lane < 48) {
                first = 160 + (lane - 32), stride = 16, ndig = 5;
            } else {
                first = 240 + (lane - 48), stride = 4, ndig = 4;
            }
            uint32_t v = 0;
#pragma unroll
            for (int i = 0; i < 5; ++i)
                if (i < ndig) v = v * 3 + sd[first + i * stride];
            if (ndig == 4) v *= 3;  // four digits weighted 81, 27, 9, 3
            out[lane] = static_cast<uint8_t>((v * 256u + 242u) / 243u);
        }
    }
    if (lane == 0) {
        const uint16_t h = __half_as_ushort(__float2half_rn(d));
        out[tq_bytes(Q) - 2] = static_cast<uint8_t>(h & 0xFFu);
        out[tq_bytes(Q) - 1] = static_cast<uint8_t>(h >> 8);
    }
}

template <int Q>
__global__ __launch_bounds__(256) void tq_quantize_kernel(const float *__restrict__ src,
                                                          uint8_t *__restrict__ dst,
                                                          int64_t rows, int64_t cols,
                                                          int64_t nb, float thr, int use_thr) {
    const int lane = threadIdx.x & 63;
    const int64_t blk =
        static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (blk >= rows * nb) return;  // whole wavefront
    const int64_t r = blk / nb;
    const int64_t col0 = (blk - r * nb) * kQK;
    const float *row = src + r * cols;
    auto at = [&](int j) -> float {
        const int64_t col = col0 + j;
        return col < cols ? row[col] : 0.0f;
    };

    float mx = 0.0f;
    bool nan = false;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const float a = fabsf(at(lane + 64 * u));
        nan |= a != a;
        mx = fmaxf(mx, a);
    }
    mx = wave_max(mx);
    const float d = __builtin_amdgcn_ballot_w64(nan) != 0 ? __builtin_nanf("") : mx;
    const float inv_d = d == 0.0f ? 0.0f : 1.0f / d;

    uint8_t *out = dst + blk * tq_bytes(Q);
    if constexpr (Q == kTq2) {
        const int a = lane >> 5;
        const int c = lane & 31;
        uint32_t b = 0;
#pragma unroll
        for (int s = 0; s < 4; ++s)
            b |= static_cast<uint32_t>(tq_trit(at(a * 128 + s * 32 + c) * inv_d, use_thr, thr) + 1)
                 << (2 * s);
        out[lane] = static_cast<uint8_t>(b);
    } else {
        if (lane < 52) {
            int first, stride, ndig;
            if (lane < 32) {
                first = lane, stride = 32, ndig = 5;
            } else if (lane < 48) {
                first = 160 + (lane - 32), stride = 16, ndig = 5;
            } else {
                first = 240 + (lane - 48), stride = 4, ndig = 4;
            }
            uint32_t v = 0;
#pragma unroll
            for (int i = 0; i < 5; ++i)
                if (i < ndig)
                    v = v * 3 + static_cast<uint32_t>(
                                    tq_trit(at(first + i * stride) * inv_d, use_thr, thr) + 1);
            if (ndig == 4) v *= 3;  // four digits weighted 81, 27, 9, 3
            out[lane] = static_cast<uint8_t>((v * 256u + 242u) / 243u);
        }
    }
    if (lane == 0) {
        const uint16_t h = __half_as_ushort(__float2half_rn(d));
        out[tq_bytes(Q) - 2] = static_cast<uint8_t>(h & 0xFFu);
        out[tq_bytes(Q) - 1] = static_cast<uint8_t>(h >> 8);
    }
}

template <int Q>
__global__ __launch_bounds__(256) void tq_dequantize_kernel(const uint8_t *__restrict__ src,
                                                            float *__restrict__ dst,
                                                            int64_t rows, int64_t cols,
                                                            int64_t nb) {
    const int lane = threadIdx.x & 63;
    const int64_t blk =
        static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (blk >= rows * nb) return;
    const int64_t r = blk / nb;
    const int64_t col0 = (blk - r * nb) * kQK;
    const uint8_t *in = src + blk * tq_bytes(Q);
    const uint16_t h = static_cast<uint16_t>(in[tq_bytes(Q) - 2] | (in[tq_bytes(Q) - 1] << 8));
    const float d = __half2float(__ushort_as_half(h));
    float *row = dst + r * cols;
    auto put = [&](int j, int digit) {
        const int64_t col = col0 + j;
        if (col < cols) __builtin_nontemporal_store(d * static_cast<float>(digit - 1), row + col);
    };
    if constexpr (Q == kTq2) {
        const uint32_t b = in[lane];
        const int a = lane >> 5;
        const int c = lane & 31;
#pragma unroll
        for (int s = 0; s < 4; ++s) put(a * 128 + s * 32 + c, static_cast<int>((b >> (2 * s)) & 3u));
    } else if (lane < 52) {
        const uint32_t b = in[lane];
        int first, stride, ndig;
        if (lane < 32) {
            first = lane, stride = 32, ndig = 5;
        } else if (lane < 48) {
            first = 160 + (lane - 32), stride = 16, ndig = 5;
        } else {
            first = 240 + (lane - 48), stride = 4, ndig = 4;
        }
        uint32_t p = 1;
#pragma unroll
        for (int n = 0; n < 5; ++n) {
            if (n < ndig) {
                const uint32_t q = (b * p) & 0xFFu;
                put(first + n * stride, static_cast<int>((q * 3u) >> 8));
            }
            p *= 3;
        }
    }
}

// Whole blocks (cols a multiple of 256) into a 16-byte aligned output, where block b's
// weights are outputs 256 b .. 256 b + 255: lane l writes weights 4 l .. 4 l + 3 with one
// non-temporal float4.  Those four share a digit position: TQ2_0 bits 2s of four
// consecutive bytes; TQ1_0 digit n of four consecutive bytes (n = e / 32 below 160,
// (e - 160) / 16 below 240, (e - 240) / 4 after, e = 4 l).
template <int Q>
__global__ __launch_bounds__(256) void tq_dequantize_vec_kernel(const uint8_t *__restrict__ src,
                                                                float *__restrict__ dst,
                                                                int64_t blocks) {
    const int lane = threadIdx.x & 63;
    const int64_t blk =
        static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (blk >= blocks) return;
    const uint8_t *in = src + blk * tq_bytes(Q);
    const uint16_t h = static_cast<uint16_t>(in[tq_bytes(Q) - 2] | (in[tq_bytes(Q) - 1] << 8));
    const float d = __half2float(__ushort_as_half(h));
    const int e = 4 * lane;
    int digit[4];
    if constexpr (Q == kTq2) {
        const int base = (e >> 7) * 32 + (e & 31);
        const int sh = 2 * ((e >> 5) & 3);
#pragma unroll
        for (int j = 0; j < 4; ++j) digit[j] = (in[base + j] >> sh) & 3;
    } else {
        int base, n;
        if (e < 160) {
            base = e & 31, n = e >> 5;
        } else if (e < 240) {
            base = 32 + ((e - 160) & 15), n = (e - 160) >> 4;
        } else {
            base = 48, n = (e - 240) >> 2;
        }
        uint32_t p = 1;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < n) p *= 3;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t q = (static_cast<uint32_t>(in[base + j]) * p) & 0xFFu;
            digit[j] = static_cast<int>((q * 3u) >> 8);
        }
    }
    floatx4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = d * static_cast<float>(digit[j] - 1);
    __builtin_nontemporal_store(o, reinterpret_cast<floatx4 *>(dst + blk * kQK + e));
}

}  // namespace

hipError_t launch_tq_quantize(const float *src, uint8_t *dst, int64_t rows, int64_t cols,
                              float thr, int use_thr, int quant, hipStream_t s) {
    const int64_t nb = (cols + kQK - 1) / kQK;
    const int64_t blocks = rows * nb;
    if (blocks == 0) return hipSuccess;
    const dim3 grid(static_cast<unsigned>((blocks + 3) / 4));
    if (cols % kQK == 0 && (reinterpret_cast<uintptr_t>(src) & 15u) == 0) {
        if (quant == kTq2)
            tq_quantize_vec_kernel<kTq2><<<grid, 256, 0, s>>>(src, dst, blocks, thr, use_thr);
        else
            tq_quantize_vec_kernel<kTq1><<<grid, 256, 0, s>>>(src, dst, blocks, thr, use_thr);
    } else if (quant == kTq2)
        tq_quantize_kernel<kTq2><<<grid, 256, 0, s>>>(src, dst, rows, cols, nb, thr, use_thr);
    else
        tq_quantize_kernel<kTq1><<<grid, 256, 0, s>>>(src, dst, rows, cols, nb, thr, use_thr);
    return hipGetLastError();
}

hipError_t launch_tq_dequantize(const uint8_t *src, float *dst, int64_t rows, int64_t cols,
                                int quant, hipStream_t s) {
    const int64_t nb = (cols + kQK - 1) / kQK;
    const int64_t blocks = rows * nb;
    if (blocks == 0) return hipSuccess;
    const dim3 grid(static_cast<unsigned>((blocks + 3) / 4));
    if (cols % kQK == 0 && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
        if (quant == kTq2)
            tq_dequantize_vec_kernel<kTq2><<<grid, 256, 0, s>>>(src, dst, blocks);
        else
            tq_dequantize_vec_kernel<kTq1><<<grid, 256, 0, s>>>(src, dst, blocks);
    } else if (quant == kTq2) {
        tq_dequantize_kernel<kTq2><<<grid, 256, 0, s>>>(src, dst, rows, cols, nb);
    } else {
        tq_dequantize_kernel<kTq1><<<grid, 256, 0, s>>>(src, dst, rows, cols, nb);
    }
    return hipGetLastError();
}

}  // namespace t81hip

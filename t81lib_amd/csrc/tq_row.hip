// t81lib_amd/csrc/tq_row.hip -- the reference's own TQ1_0 row codec
// (src/t81/core/gguf_quants.h:14-168) and the tensor payload its dequant_tq1_0 /
// dequant_tq2_0 bindings read (python/bindings.cpp:561-638).
//
// Word format: 8 trits per uint16, digit d = {+1: 0, 0: 1, -1: 2}, word = sum_i d_i 3^i
// with trit i of the word (values 8w + i of the row) as digit i; the words of a row of
// n values are ceil(n / 8), pad trits 0.  A row has one float scale: quantize uses
// the caller's scale when it is > 0, else max |v| of the row (NaN values never win the
// comparison), then trit(v * (1 / scale)) with |v| clamped to 1 (a NaN product clamps
// to +1, as std::fmin / std::fmax return the non-NaN operand) and the threshold
// clamped to [0, 0.9999]; decode gives trit * scale (all zeros when scale == 0).
//
// Tensor payload: groups of block_rows rows, each a little-endian IEEE half scale,
// 8 reserved bytes in the TQ2_0 variant, then the group's rows of words, byte-packed
// (the payload need not be aligned).  The writer here (no reference counterpart; the
// reference only reads such payloads) stores h = half(max |v| of the group) and
// quantizes each row with the scale float(h), as a caller of quantize_row_tq1_0
// would.
//
// All the kernels are bound by HBM: a word is 32 bytes of float32 on one side and
// 2 bytes on the other.  Quantize runs two lanes per word (float4 loads where the row is
// 16-byte aligned, rows of up to 8192 values held in registers and read once); both
// dequantize paths do too, with non-temporal float4 stores, when the row length is a
// multiple of 8 and the output 16-byte aligned, else one lane per word, consecutive lanes
// on consecutive words.
#include <hip/hip_runtime.h>

#include "t81_device.hpp"
#include "t81_kernels.hpp"

#pragma clang fp contract(off)

namespace t81hip {

namespace {

constexpr int kWordTrits = 8;

__device__ __forceinline__ int tq1r_trit(float v, float thr) {
    const float c = v != v ? 1.0f : (v > 1.0f ? 1.0f : (v < -1.0f ? -1.0f : v));
    if (c >= thr) return 1;
    if (c <= -thr) return -1;
    return 0;
}

__device__ __forceinline__ uint32_t tq1r_digit(int t) { return t > 0 ? 0u : (t < 0 ? 2u : 1u); }

// IEEE half bits -> float32 bits, exactly (subnormals normalised, NaN payload kept).
__host__ __device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1Fu) {
        bits = sign | 0x7F800000u | (m << 13);
    } else if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            // m * 2^-24: shift the leading one up to bit 10, one exponent step per shift
            int shift = 0;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                ++shift;
            }
            bits = sign | (static_cast<uint32_t>(113 - shift) << 23) | ((m & 0x3FFu) << 13);
        }
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    return __builtin_bit_cast(float, bits);
}

// Max of non-NaN |v| over the workgroup (kT threads, red[kT / 64]), from per-thread
// maxima >= 0.
template <int kT = 256>
__device__ __forceinline__ float block_max(float m, float *red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < kT / 64; ++w) r = red[w] > r ? red[w] : r;
    return r;
}

// Max of non-NaN |v| over this thread's values (thread t of kT takes every kT-th quad):
// float4 loads over the 16-byte aligned whole quads when the row starts aligned, single
// loads for the rest.
template <int kT = 256>
__device__ __forceinline__ float abs_max_strided(const float *v, int64_t n) {
    float m = 0.0f;
    int64_t head = 0;
    if ((reinterpret_cast<uintptr_t>(v) & 15u) == 0) {
        const int64_t quads = n >> 2;
        int64_t i = threadIdx.x;
        // four loads in flight per lane over long spans (the payload writer's scale
        // pass over 8192 x 3072 took 49.9 us with one, 30.9 with four)
        for (; i + 3 * kT < quads; i += 4 * kT) {
            floatx4 a[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                a[u] = *reinterpret_cast<const floatx4 *>(v + 4 * (i + kT * u));
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float b = fabsf(a[u][j]);
                    m = b > m ? b : m;
                }
        }
        for (; i < quads; i += kT) {
            const floatx4 a = *reinterpret_cast<const floatx4 *>(v + 4 * i);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float b = fabsf(a[j]);
                m = b > m ? b : m;
            }
        }
        head = quads << 2;
    }
    for (int64_t i = head + threadIdx.x; i < n; i += kT) {
        const float a = fabsf(v[i]);
        m = a > m ? a : m;
    }
    return m;
}

// The words of a row, two lanes per word: lane 2w + h turns values 8w + 4h .. 8w + 4h + 4
// (pad trits 0) into the half word sum_i d_i 3^i, and the even lane hands its half plus
// 81 times its neighbour's to store(w, word), so a wavefront reads 1 KiB of the row
// contiguously.  Both lanes of a pair run the same iterations (256 is even), so the
// partner is always live.
template <typename Store>
__device__ __forceinline__ void quantize_words(const float *v, int64_t n, int64_t words,
                                               float scale, float inv, float thr,
                                               Store store) {
    const bool vec = (reinterpret_cast<uintptr_t>(v) & 15u) == 0;
    for (int64_t q = threadIdx.x; q < 2 * words; q += 256) {
        const int64_t k0 = 4 * q;
        float x[4];
        if (vec && k0 + 4 <= n) {
            const floatx4 a = *reinterpret_cast<const floatx4 *>(v + k0);
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = a[i];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = k0 + i < n ? v[k0 + i] : 0.0f;
        }
        uint32_t half = 0;
#pragma unroll
        for (int i = 3; i >= 0; --i) {
            const int t = (k0 + i < n && scale > 0.0f) ? tq1r_trit(x[i] * inv, thr) : 0;
            half = half * 3u + tq1r_digit(t);
        }
        const uint32_t hi = __shfl_xor(half, 1, 64);
        if ((q & 1) == 0) store(q >> 1, half + 81u * hi);
    }
}

// Trit i (0..7) of a word's low 8 base-3 digits times scale.
__device__ __forceinline__ void decode_word(uint32_t word, float scale, float *out, int count) {
#pragma unroll
    for (int i = 0; i < kWordTrits; ++i) {
        const uint32_t d = word % 3u;
        word /= 3u;
        if (i < count) {
            const float t = d == 0 ? 1.0f : (d == 2 ? -1.0f : 0.0f);
            out[i] = scale == 0.0f ? 0.0f : t * scale;
        }
    }
}

// One workgroup per row: the scale (caller's when > 0, else the row's max |v|), then
// the row's words.
__global__ __launch_bounds__(256) void tq1r_quantize_rows_kernel(
    const float *__restrict__ values, int64_t n, float thr, const float *__restrict__ scales_in,
    float *__restrict__ scales_out, uint16_t *__restrict__ dst) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const float *v = values + row * n;
    float scale = scales_in != nullptr ? scales_in[row] : 0.0f;
    if (!(scale > 0.0f)) scale = block_max(abs_max_strided(v, n), red);
    if (scales_out != nullptr && threadIdx.x == 0) scales_out[row] = scale;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    const int64_t words = (n + kWordTrits - 1) / kWordTrits;
    uint16_t *out = dst + row * words;
    quantize_words(v, n, words, scale, inv, thr, [out](int64_t w, uint32_t word) {
        out[w] = static_cast<uint16_t>(word);
    });
}

// Rows of n <= 1024 R values, n a multiple of 4 and the matrix 16-byte aligned: the row
// is read once, R float4 per lane (quad q = lane + 256 j), and quantized from registers;
// lane q and lane q ^ 1 hold the two halves of word q >> 1 at every j.
template <int R>
__global__ __launch_bounds__(256) void tq1r_quantize_rows_reg_kernel(
    const float *__restrict__ values, int64_t n, float thr, const float *__restrict__ scales_in,
    float *__restrict__ scales_out, uint16_t *__restrict__ dst) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const float *v = values + row * n;
    const int quads = static_cast<int>(n >> 2);
    floatx4 x[R];
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int q = threadIdx.x + 256 * j;
        // non-temporal: the row is read once (8192 x 3072: 24.8 -> 23.9 us in an A/B)
        x[j] = q < quads ? __builtin_nontemporal_load(reinterpret_cast<const floatx4 *>(v + 4 * q))
                         : floatx4{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = fabsf(x[j][i]);
            m = a > m ? a : m;
        }
    }
    float scale = scales_in != nullptr ? scales_in[row] : 0.0f;
    if (!(scale > 0.0f)) scale = block_max(m, red);
    if (scales_out != nullptr && threadIdx.x == 0) scales_out[row] = scale;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    const int words = static_cast<int>((n + kWordTrits - 1) / kWordTrits);
    uint16_t *out = dst + row * words;
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int q = threadIdx.x + 256 * j;
        if (q < 2 * words) {
            uint32_t half = 0;
#pragma unroll
            for (int i = 3; i >= 0; --i) {
                const int t = (4 * q + i < n && scale > 0.0f) ? tq1r_trit(x[j][i] * inv, thr) : 0;
                half = half * 3u + tq1r_digit(t);
            }
            const uint32_t hi = __shfl_xor(half, 1, 64);
            if ((q & 1) == 0) out[q >> 1] = static_cast<uint16_t>(half + 81u * hi);
        }
    }
}

__global__ __launch_bounds__(256) void tq1r_dequantize_rows_kernel(
    const uint16_t *__restrict__ src, int64_t rows, int64_t n, int64_t words,
    const float *__restrict__ scales, float *__restrict__ dst) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= rows * words) return;
    const int64_t row = idx / words;
    const int64_t w = idx - row * words;
    const int64_t k0 = w * kWordTrits;
    const int count = static_cast<int>(n - k0 < kWordTrits ? n - k0 : kWordTrits);
    float out[kWordTrits];
    decode_word(src[idx], scales[row], out, count);
    float *o = dst + row * n + k0;
#pragma unroll
    for (int i = 0; i < kWordTrits; ++i)
        if (i < count) o[i] = out[i];
}

// Rows whose length is a multiple of 8 into a 16-byte aligned output: the output is the
// flat run of all words' values, and thread t writes values 4t .. 4t + 4 (half t & 1 of
// word t >> 1) with one non-temporal float4 store, 1 KiB per wavefront contiguously (the
// non-temporal hint: 8192 x 3072 in 15.2 us against 26.8 with ordinary stores).
__global__ __launch_bounds__(256) void tq1r_dequantize_rows_vec_kernel(
    const uint16_t *__restrict__ src, int64_t total_words, int64_t words,
    const float *__restrict__ scales, float *__restrict__ dst) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t w = t >> 1;
    if (w >= total_words) return;
    const int64_t row = total_words <= 0xFFFFFFFFll
                            ? static_cast<int64_t>(static_cast<uint32_t>(w) /
                                                   static_cast<uint32_t>(words))
                            : w / words;
    const float scale = scales[row];
    uint32_t word = src[w];
    if (t & 1) word /= 81u;
    floatx4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t d = word % 3u;
        word /= 3u;
        const float tv = d == 0 ? 1.0f : (d == 2 ? -1.0f : 0.0f);
        o[i] = scale == 0.0f ? 0.0f : tv * scale;
    }
    __builtin_nontemporal_store(o, reinterpret_cast<floatx4 *>(dst + 4 * t));
}

struct PayloadLayout {
    int64_t group;      // rows per group (>= 1, at most max(rows, 1))
    int64_t header;     // 2 (+ 8 reserved bytes)
    int64_t row_bytes;  // 2 * words
    int64_t stride;     // bytes per whole group
};

__global__ __launch_bounds__(256) void tq1r_dequantize_payload_kernel(
    const uint8_t *__restrict__ payload, int64_t rows, int64_t n, int64_t words, PayloadLayout lay,
    float *__restrict__ dst) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= rows * words) return;
    const int64_t row = idx / words;
    const int64_t w = idx - row * words;
    const int64_t g = row / lay.group;
    const uint8_t *grp = payload + g * lay.stride;
    // the word's bytes are loaded with the scale's, ahead of the scale's conversion
    const uint8_t *p = grp + lay.header + (row - g * lay.group) * lay.row_bytes + 2 * w;
    const uint32_t word = static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8);
    const float scale = half_bits_to_float(static_cast<uint32_t>(grp[0]) |
                                           (static_cast<uint32_t>(grp[1]) << 8));
    const int64_t k0 = w * kWordTrits;
    const int count = static_cast<int>(n - k0 < kWordTrits ? n - k0 : kWordTrits);
    float out[kWordTrits];
    decode_word(word, scale, out, count);
    float *o = dst + row * n + k0;
#pragma unroll
    for (int i = 0; i < kWordTrits; ++i)
        if (i < count) o[i] = out[i];
}

// Rows whose length is a multiple of 8 into a 16-byte aligned output, as
// tq1r_dequantize_rows_vec_kernel.  A group's rows of words are contiguous in the payload
// (a row is exactly its words) and its rows contiguous in the output, so workgroup b takes
// chunk b % chunks of group b / chunks (a division of uniform values), and its thread t'
// decodes half t' & 1 of the group's word t' >> 1 into one non-temporal float4 at output
// 4 t' of the group -- no per-lane division.  kEven: the payload starts at an even
// address, so every word does (headers, rows and groups have even sizes) and is read with
// one 16-bit load.
template <bool kEven>
__global__ __launch_bounds__(256) void tq1r_dequantize_payload_vec_kernel(
    const uint8_t *__restrict__ payload, int64_t rows, int64_t n, int64_t words,
    uint32_t chunks, PayloadLayout lay, float *__restrict__ dst) {
    const uint32_t g = blockIdx.x / chunks;
    const int64_t q = static_cast<int64_t>(blockIdx.x - g * chunks) * 256 + threadIdx.x;
    const int64_t r0 = static_cast<int64_t>(g) * lay.group;
    const int64_t nr = rows - r0 < lay.group ? rows - r0 : lay.group;
    if (q >= 2 * nr * words) return;
    const uint8_t *grp = payload + g * lay.stride;
    // both loads ahead of the scale's conversion, whose branches would otherwise hold the
    // word's load behind the scale's (two memory latencies per wave; 8192 x 3072:
    // 20.0 -> 16.9 us)
    const uint8_t *p = grp + lay.header + 2 * (q >> 1);
    uint32_t word = kEven ? *reinterpret_cast<const uint16_t *>(p)
                          : static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8);
    const uint32_t hbits = kEven ? *reinterpret_cast<const uint16_t *>(grp)
                                 : static_cast<uint32_t>(grp[0]) |
                                       (static_cast<uint32_t>(grp[1]) << 8);
    if (q & 1) word /= 81u;
    const float scale = half_bits_to_float(hbits);
    floatx4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t d = word % 3u;
        word /= 3u;
        const float tv = d == 0 ? 1.0f : (d == 2 ? -1.0f : 0.0f);
        o[i] = scale == 0.0f ? 0.0f : tv * scale;
    }
    __builtin_nontemporal_store(o, reinterpret_cast<floatx4 *>(dst + r0 * n + 4 * q));
}

// One workgroup per group: h = half(max |v| over the group's rows, contiguous in the
// input), round to nearest even; the reserved bytes are zeroed.
// (1024 threads: one workgroup per group leaves a grid of rows / 32 workgroups; 256
// threads each took 30.9 us for 8192 x 3072.)
__global__ __launch_bounds__(1024) void tq1r_payload_scales_kernel(
    const float *__restrict__ values, int64_t rows, int64_t n, PayloadLayout lay,
    uint8_t *__restrict__ payload) {
    __shared__ float red[16];
    const int64_t g = blockIdx.x;
    const int64_t r0 = g * lay.group;
    const int64_t nr = rows - r0 < lay.group ? rows - r0 : lay.group;
    const float m = block_max<1024>(abs_max_strided<1024>(values + r0 * n, nr * n), red);
    uint8_t *grp = payload + g * lay.stride;
    if (threadIdx.x == 0) {
        const uint16_t h = __builtin_bit_cast(uint16_t, static_cast<_Float16>(m));
        grp[0] = static_cast<uint8_t>(h & 0xFFu);
        grp[1] = static_cast<uint8_t>(h >> 8);
    }
    if (threadIdx.x >= 2 && threadIdx.x < lay.header) grp[threadIdx.x] = 0;
}

// One workgroup per row, scale read back from its group's half: quantize_row_tq1_0
// with that scale (<= 0 falls back to the row's own max, as the reference does).
__global__ __launch_bounds__(256) void tq1r_payload_rows_kernel(
    const float *__restrict__ values, int64_t n, float thr, PayloadLayout lay,
    uint8_t *__restrict__ payload) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const int64_t g = row / lay.group;
    uint8_t *grp = payload + g * lay.stride;
    const float *v = values + row * n;
    float scale = half_bits_to_float(static_cast<uint32_t>(grp[0]) |
                                     (static_cast<uint32_t>(grp[1]) << 8));
    if (!(scale > 0.0f)) scale = block_max(abs_max_strided(v, n), red);
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    const int64_t words = (n + kWordTrits - 1) / kWordTrits;
    uint8_t *out = grp + lay.header + (row - g * lay.group) * lay.row_bytes;
    quantize_words(v, n, words, scale, inv, thr, [out](int64_t w, uint32_t word) {
        out[2 * w] = static_cast<uint8_t>(word & 0xFFu);
        out[2 * w + 1] = static_cast<uint8_t>(word >> 8);
    });
}

PayloadLayout layout(int64_t rows, int64_t n, int64_t block_rows, bool refinements) {
    PayloadLayout lay;
    const int64_t cap = rows > 1 ? rows : 1;
    lay.group = block_rows < 1 ? 1 : (block_rows > cap ? cap : block_rows);
    lay.header = refinements ? 10 : 2;
    lay.row_bytes = 2 * ((n + kWordTrits - 1) / kWordTrits);
    lay.stride = lay.header + lay.group * lay.row_bytes;
    return lay;
}

float clamp_threshold(float t) { return t < 0.0f ? 0.0f : (0.9999f < t ? 0.9999f : t); }

unsigned grid_of(int64_t threads) { return static_cast<unsigned>((threads + 255) / 256); }

}  // namespace

int64_t tq1r_payload_bytes(int64_t rows, int64_t n, int64_t block_rows, bool refinements) {
    if (rows <= 0) return 0;
    const PayloadLayout lay = layout(rows, n, block_rows, refinements);
    const int64_t groups = (rows + lay.group - 1) / lay.group;
    const int64_t last = rows - (groups - 1) * lay.group;
    return (groups - 1) * lay.stride + lay.header + last * lay.row_bytes;
}

int tq1r_payload_check(int64_t nbytes, int64_t rows, int64_t n, int64_t block_rows,
                       bool refinements) {
    if (rows <= 0 || nbytes >= tq1r_payload_bytes(rows, n, block_rows, refinements)) return 0;
    const PayloadLayout lay = layout(rows, n, block_rows, refinements);
    // every group before g0 ends at or before g0 * stride <= nbytes: the first failing
    // check of the binding's sequential walk lies in group g0 or the one after it
    const int64_t groups = (rows + lay.group - 1) / lay.group;
    int64_t g = nbytes / lay.stride;
    if (g > groups - 1) g = groups - 1;
    for (; g < groups; ++g) {
        const int64_t off = g * lay.stride;
        if (off + 2 > nbytes) return 1;
        if (refinements && off + 10 > nbytes) return 2;
        const int64_t nr = rows - g * lay.group < lay.group ? rows - g * lay.group : lay.group;
        if (off + lay.header + nr * lay.row_bytes > nbytes) return 3;
    }
    return 0;
}

hipError_t launch_tq1r_quantize_rows(const float *values, int64_t rows, int64_t n, float thr,
                                     const float *scales_in, float *scales_out, uint16_t *dst,
                                     hipStream_t s) {
    if (rows == 0 || n == 0) return hipSuccess;
    const dim3 grid(static_cast<unsigned>(rows));
    const float t = clamp_threshold(thr);
    if (n % 4 == 0 && n <= 8192 && (reinterpret_cast<uintptr_t>(values) & 15u) == 0) {
        if (n <= 1024)
            tq1r_quantize_rows_reg_kernel<1><<<grid, 256, 0, s>>>(values, n, t, scales_in,
                                                                  scales_out, dst);
        else if (n <= 2048)
            tq1r_quantize_rows_reg_kernel<2><<<grid, 256, 0, s>>>(values, n, t, scales_in,
                                                                  scales_out, dst);
        else if (n <= 4096)
            tq1r_quantize_rows_reg_kernel<4><<<grid, 256, 0, s>>>(values, n, t, scales_in,
                                                                  scales_out, dst);
        else
            tq1r_quantize_rows_reg_kernel<8><<<grid, 256, 0, s>>>(values, n, t, scales_in,
                                                                  scales_out, dst);
    } else {
        tq1r_quantize_rows_kernel<<<grid, 256, 0, s>>>(values, n, t, scales_in, scales_out, dst);
    }
    return hipGetLastError();
}

hipError_t launch_tq1r_dequantize_rows(const uint16_t *src, int64_t rows, int64_t n,
                                       const float *scales, float *dst, hipStream_t s) {
    const int64_t words = (n + kWordTrits - 1) / kWordTrits;
    if (rows * words == 0) return hipSuccess;
    if (n % kWordTrits == 0 && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0)
        tq1r_dequantize_rows_vec_kernel<<<grid_of(2 * rows * words), 256, 0, s>>>(
            src, rows * words, words, scales, dst);
    else
        tq1r_dequantize_rows_kernel<<<grid_of(rows * words), 256, 0, s>>>(src, rows, n, words,
                                                                           scales, dst);
    return hipGetLastError();
}

hipError_t launch_tq1r_dequantize_payload(const uint8_t *payload, int64_t rows, int64_t n,
                                          int64_t block_rows, bool refinements, float *dst,
                                          hipStream_t s) {
    const int64_t words = (n + kWordTrits - 1) / kWordTrits;
    if (rows * words == 0) return hipSuccess;
    const PayloadLayout lay = layout(rows, n, block_rows, refinements);
    const int64_t groups = (rows + lay.group - 1) / lay.group;
    const int64_t chunks = (2 * lay.group * words + 255) / 256;
    if (n % kWordTrits == 0 && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0 &&
        groups * chunks <= 0xFFFFFFFFll / 256) {
        const dim3 grid(static_cast<unsigned>(groups * chunks));
        if ((reinterpret_cast<uintptr_t>(payload) & 1u) == 0)
            tq1r_dequantize_payload_vec_kernel<true><<<grid, 256, 0, s>>>(
                payload, rows, n, words, static_cast<uint32_t>(chunks), lay, dst);
        else
            tq1r_dequantize_payload_vec_kernel<false><<<grid, 256, 0, s>>>(
                payload, rows, n, words, static_cast<uint32_t>(chunks), lay, dst);
    } else
        tq1r_dequantize_payload_kernel<<<grid_of(rows * words), 256, 0, s>>>(payload, rows, n,
                                                                              words, lay, dst);
    return hipGetLastError();
}

hipError_t launch_tq1r_quantize_payload(const float *values, int64_t rows, int64_t n,
                                        int64_t block_rows, bool refinements, float thr,
                                        uint8_t *payload, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    const PayloadLayout lay = layout(rows, n, block_rows, refinements);
    const int64_t groups = (rows + lay.group - 1) / lay.group;
    tq1r_payload_scales_kernel<<<dim3(static_cast<unsigned>(groups)), 1024, 0, s>>>(
        values, rows, n, lay, payload);
    if (n > 0)
        tq1r_payload_rows_kernel<<<dim3(static_cast<unsigned>(rows)), 256, 0, s>>>(
            values, n, clamp_threshold(thr), lay, payload);
    return hipGetLastError();
}

}  // namespace t81hip

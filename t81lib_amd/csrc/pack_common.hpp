// t81lib_amd/csrc/pack_common.hpp -- threshold quantization and 12-value packing shared by
// the packers (pack.hip) and the fused activation path of the limb GEMM (limb.hip).
#pragma once

#include "t81_device.hpp"

namespace t81hip {

// Quantize one value.  The reference clamps to [-1, 1] before comparing
// (python/bindings.cpp:406, t81/torch/__init__.py:46); for every threshold the
// host lets through (0 <= thr <= 1, or NaN) the clamp cannot change either
// comparison, so it is left out:  v > 1 gives c = 1 >= thr and v >= thr alike,
// v < -1 gives c = -1 <= -thr and v <= -thr alike, NaN fails all compares.
// torch form: "-1 wins" ordering of t81/torch/__init__.py:47-49.
__device__ __forceinline__ int quantize_one(float v, float thr, int torch_form) {
    const bool pos = v >= thr;
    const bool neg = v <= -thr;
    if (torch_form) return neg ? -1 : (pos ? 1 : 0);
    return pos ? 1 : (neg ? -1 : 0);
}

// Conversions of one stored element to float (bf16 is carried as uint16_t bits).
template <typename T>
__device__ __forceinline__ float from_bits16(uint32_t bits);
template <>
__device__ __forceinline__ float from_bits16<uint16_t>(uint32_t bits) {
    return __uint_as_float(bits << 16);
}
template <>
__device__ __forceinline__ float from_bits16<_Float16>(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

template <typename T>
__device__ __forceinline__ float load_as_float(const T *p) {
    if constexpr (sizeof(T) == 4) {
        return *p;
    } else {
        return from_bits16<T>(*reinterpret_cast<const uint16_t *>(p));
    }
}

// 12 consecutive values starting at src[c0], zero past `limit` columns, quantized
// and packed as 4 trytes (little-endian bytes) into one dword.
template <typename T, bool kVec>
__device__ __forceinline__ uint32_t pack12(const T *src, int64_t c0, int64_t limit, float thr,
                                           int torch_form) {
    float v[12];
    if (kVec && c0 + 12 <= limit) {
        if constexpr (sizeof(T) == 4) {
            const float4 *p = reinterpret_cast<const float4 *>(src + c0);
            const float4 x0 = p[0], x1 = p[1], x2 = p[2];
            v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
            v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
            v[8] = x2.x; v[9] = x2.y; v[10] = x2.z; v[11] = x2.w;
        } else {
            // 12 x 2 bytes = 24 bytes: one 16-byte and one 8-byte load (8-byte aligned)
            const uint2 *p = reinterpret_cast<const uint2 *>(src + c0);
            const uint2 a = p[0], b = p[1], c = p[2];
            const uint32_t h[6] = {a.x, a.y, b.x, b.y, c.x, c.y};
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                v[2 * i] = from_bits16<T>(h[i] & 0xFFFFu);
                v[2 * i + 1] = from_bits16<T>(h[i] >> 16);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 12; ++i) v[i] = (c0 + i < limit) ? load_as_float<T>(src + c0 + i) : 0.0f;
    }
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int t[3];
#pragma unroll
        for (int p = 0; p < 3; ++p) {
            const int64_t c = c0 + 3 * j + p;
            t[p] = (c < limit) ? quantize_one(v[3 * j + p], thr, torch_form) : 0;
        }
        const uint32_t tryte = static_cast<uint32_t>(13 + t[0] + 3 * t[1] + 9 * t[2]);
        word |= tryte << (8 * j);
    }
    return word;
}

}  // namespace t81hip

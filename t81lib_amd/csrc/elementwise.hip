// t81lib_amd/csrc/elementwise.hip -- the elementwise ops of the ROCm backend contract
// (include/t81/linalg/gemm_gpu.hpp:80-85, 233-249), float32, contiguous.
//
// Each reproduces the reference's CPU loop (src/linalg/gemm_dispatch.cpp:145-211)
// bit for bit: the same expression, evaluated left to right with every multiply
// and add rounded separately (no contraction -- the reference's CPU build has no
// FMA), the same NaN behaviour (a NaN condition is "!= 0", a NaN clamp input
// passes through).  HBM-bound: one 16-byte vector per thread per input where the
// pointers allow it (non-temporal from 1 Mi elements), grid-stride otherwise.
#include "t81_device.hpp"
#include "t81_kernels.hpp"

#pragma clang fp contract(off)

namespace t81hip {

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float where_one(float c, float x, float y) { return c != 0.0f ? x : y; }
__device__ __forceinline__ float clamp_one(float v, float lo, float hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}
__device__ __forceinline__ float lerp_one(float s, float e, float w) { return s + w * (e - s); }
__device__ __forceinline__ float addcmul_one(float in, float t1, float t2, float value) {
    return in + value * t1 * t2;
}

template <bool kNT>
__device__ __forceinline__ floatx4 load4(const float *p, int64_t i) {
    if constexpr (kNT) return __builtin_nontemporal_load(reinterpret_cast<const floatx4 *>(p) + i);
    else return reinterpret_cast<const floatx4 *>(p)[i];
}

// op: 0 where(a = cond, b = x, c = y); 1 clamp(a, p0 = lo, p1 = hi); 2 lerp(a = start,
// b = end, c = weight); 3 addcmul(a = input, b = t1, c = t2, p0 = value)
template <int OP>
__device__ __forceinline__ float apply(float a, float b, float c, float p0, float p1) {
    if constexpr (OP == 0) return where_one(a, b, c);
    else if constexpr (OP == 1) return clamp_one(a, p0, p1);
    else if constexpr (OP == 2) return lerp_one(a, b, c);
    else return addcmul_one(a, b, c, p0);
}

// kNT (large vector launches): non-temporal stores, and for the three-input ops
// non-temporal loads -- every byte is touched once.  32 Mi elements: clamp 45.7 -> 37.3 us
// (the loads too: 42.6), where / lerp / addcmul 92.5 -> 84.4 us (the stores alone: 90.8).
template <int OP, bool kVec, bool kNT = false>
__global__ __launch_bounds__(kThreads) void elementwise_kernel(const float *__restrict__ a,
                                                              const float *__restrict__ b,
                                                              const float *__restrict__ c,
                                                              float *__restrict__ out, int64_t n,
                                                              float p0, float p1) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if constexpr (kVec) {
        const int64_t n4 = n / 4;
        for (; i < n4; i += stride) {
            constexpr bool kNTLoad = kNT && OP != 1;
            const floatx4 va = load4<kNTLoad>(a, i);
            floatx4 vb = va, vc = va;
            if constexpr (OP != 1) {
                vb = load4<kNTLoad>(b, i);
                vc = load4<kNTLoad>(c, i);
            }
            floatx4 r;
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = apply<OP>(va[e], vb[e], vc[e], p0, p1);
            if constexpr (kNT)
                __builtin_nontemporal_store(r, reinterpret_cast<floatx4 *>(out) + i);
            else
                reinterpret_cast<floatx4 *>(out)[i] = r;
        }
        // tail of n % 4 elements
        i = 4 * n4 + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    }
    for (; i < n; i += stride) {
        const float va = a[i];
        const float vb = OP != 1 ? b[i] : 0.0f;
        const float vc = OP != 1 ? c[i] : 0.0f;
        out[i] = apply<OP>(va, vb, vc, p0, p1);
    }
}

template <int OP>
hipError_t launch_op(const float *a, const float *b, const float *c, float *out, int64_t n,
                     float p0, float p1, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    auto aligned = [](const void *p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    const bool vec = aligned(a) && aligned(b) && aligned(c) && aligned(out);
    const int64_t work = vec ? (n + 3) / 4 : n;
    int64_t blocks = (work + kThreads - 1) / kThreads;
    if (blocks > 65536) blocks = 65536;
    // the hint from 1 Mi elements (4 MiB per operand, an XCD's L2) up
    if (vec && n >= (int64_t{1} << 20))
        elementwise_kernel<OP, true, true><<<dim3(blocks), dim3(kThreads), 0, s>>>(a, b, c, out, n,
                                                                                  p0, p1);
    else if (vec)
        elementwise_kernel<OP, true><<<dim3(blocks), dim3(kThreads), 0, s>>>(a, b, c, out, n, p0, p1);
    else
        elementwise_kernel<OP, false><<<dim3(blocks), dim3(kThreads), 0, s>>>(a, b, c, out, n, p0, p1);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_where(const float *cond, const float *x, const float *y, float *out, int64_t n,
                        hipStream_t s) {
    return launch_op<0>(cond, x, y, out, n, 0.0f, 0.0f, s);
}

hipError_t launch_clamp(const float *in, float *out, int64_t n, float lo, float hi,
                        hipStream_t s) {
    return launch_op<1>(in, nullptr, nullptr, out, n, lo, hi, s);
}

hipError_t launch_lerp(const float *start, const float *end, const float *weight, float *out,
                       int64_t n, hipStream_t s) {
    return launch_op<2>(start, end, weight, out, n, 0.0f, 0.0f, s);
}

hipError_t launch_addcmul(const float *in, const float *t1, const float *t2, float value,
                          float *out, int64_t n, hipStream_t s) {
    return launch_op<3>(in, t1, t2, out, n, value, 0.0f, s);
}

}  // namespace t81hip

// t81lib_amd/csrc/floors.hip -- measurement kernels for bench.py (libt81_floors.so), not
// part of the t81lib path: a plain streaming read of a buffer, the floor that any kernel
// reading the same bytes in one launch can be compared with; and the VALU form of the
// one-token GEMV (t81_floor_gemv_valu), timed beside K2's matrix-core form.
//
// t81_floor_read: the buffer is cut into `blocks` contiguous spans of whole 16-byte words;
// each workgroup of 256 threads streams its span in rounds of U loads per thread, all U
// issued before any is used (consecutive threads, consecutive words: every load
// instruction reads 4 KB contiguously), XOR-folds them and writes one word per workgroup
// to out[blockIdx.x], so the loads cannot be optimised away.  U = unroll (1, 4 or 8):
// the bytes in flight per thread.  bytes must be a multiple of 16 and src 16-byte aligned.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "t81_device.hpp"

namespace {

template <int U>
__global__ __launch_bounds__(256) void read_floor_kernel(const uint4 *__restrict__ src,
                                                         int64_t words, int64_t span,
                                                         uint32_t *__restrict__ out) {
    const int64_t begin = static_cast<int64_t>(blockIdx.x) * span;
    const int64_t end = begin + span < words ? begin + span : words;
    uint4 acc = {0u, 0u, 0u, 0u};
    for (int64_t base = begin; base < end; base += 256 * U) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = base + 256 * u + threadIdx.x;
            v[u] = i < end ? src[i] : uint4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            acc.x ^= v[u].x;
            acc.y ^= v[u].y;
            acc.z ^= v[u].z;
            acc.w ^= v[u].w;
        }
    }
    uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
    for (int o = 32; o > 0; o >>= 1) r ^= __shfl_xor(r, o);
    __shared__ uint32_t red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = r;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

}  // namespace

// blocks workgroups, each streaming ceil(words / blocks) words with `unroll` loads per
// thread in flight (1, 4 or 8); out receives one word per workgroup.
extern "C" int t81_floor_read(const void *src, int64_t bytes, uint32_t *out, int blocks,
                              int unroll, void *stream) {
    if (src == nullptr || out == nullptr || bytes <= 0 || bytes % 16 != 0 || blocks <= 0 ||
        reinterpret_cast<uintptr_t>(src) % 16 != 0 || (unroll != 1 && unroll != 4 && unroll != 8))
        return -1;
    const int64_t words = bytes / 16;
    const int64_t span = (words + blocks - 1) / blocks;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const auto *p = static_cast<const uint4 *>(src);
    if (unroll == 8)
        read_floor_kernel<8><<<dim3(blocks), dim3(256), 0, s>>>(p, words, span, out);
    else if (unroll == 4)
        read_floor_kernel<4><<<dim3(blocks), dim3(256), 0, s>>>(p, words, span, out);
    else
        read_floor_kernel<1><<<dim3(blocks), dim3(256), 0, s>>>(p, words, span, out);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

namespace {

// ---- the VALU form of the one-token GEMV ----
// y[r] = sum_k x[k] * T[r, k] at one bf16 token with no matrix cores, as the decode path
// could be written with vector ALU products and a cross-lane reduction:
//  * lane l owns limbs l and l + 64 of every row (L <= 128 limbs) and keeps their 48
//    activations each as 24 bf16 pairs in registers for the whole launch;
//  * a wave streams rows gw, gw + G, ... (G waves in the grid), D rows at a time with all
//    their limb loads in flight: lane l reads 16 bytes of limb l (and of limb l + 64), so a
//    row is one or two contiguous 1 KB load instructions;
//  * each weight dword decodes through the same LDS tables as K2 (decode_dword: four table
//    reads, six dwords of natural-order bf16 trit pairs), and v_dot2c_f32_bf16 multiplies a
//    trit pair with an activation pair and adds both products to the lane's float sum;
//  * the 64 lane sums of a row meet in DPP adds within each 16-lane row and three
//    v_readlane reads across them (fixed order), and lane 0 stores the row.
// Limbs past L meet zero activations; rows past N load nothing and are not stored.
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                 CTRL, 0xF, 0xF, false));
}

template <int D>
__global__ __launch_bounds__(256) void gemv_valu_kernel(const uint16_t *__restrict__ x,
                                                        const uint8_t *__restrict__ w,
                                                        float *__restrict__ y, int N, int K,
                                                        int L) {
    __shared__ __attribute__((aligned(16))) uint8_t lut[t81hip::kLutBytes];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    t81hip::lut_init(lut, tid, 256);
    const int gw = blockIdx.x * 4 + (tid >> 6);
    const int G = gridDim.x * 4;
    uint32_t xv[2][24];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int limb = lane + 64 * j;
#pragma unroll
        for (int c = 0; c < 6; ++c) {
            const int k0 = 48 * limb + 8 * c;
            u32x4v v = {0u, 0u, 0u, 0u};
            if (limb < L && k0 + 8 <= K) {
                v = *reinterpret_cast<const u32x4v *>(x + k0);
            } else if (limb < L) {
                uint32_t h[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = k0 + e < K ? x[k0 + e] : 0u;
                v = u32x4v{h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16};
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[j][4 * c + e] = v[e];
        }
    }
    const bool two = L > 64;
    for (int r0 = gw; r0 < N; r0 += G * D) {
        u32x4v wl[D][2];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int r = r0 + d * G;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int limb = lane + 64 * j;
                wl[d][j] = u32x4v{0u, 0u, 0u, 0u};
                if (r < N && limb < L && (j == 0 || two))
                    wl[d][j] = *reinterpret_cast<const u32x4v *>(
                        w + (static_cast<int64_t>(r) * L + limb) * t81hip::kTrytes);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int r = r0 + d * G;
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (j == 1 && !two) break;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    uint32_t pairs[6];
                    t81hip::decode_dword(lut, wl[d][j][q], pairs);
#pragma unroll
                    for (int p = 0; p < 6; ++p)
                        acc = __builtin_amdgcn_fdot2_f32_bf16(
                            __builtin_bit_cast(bf16x2v, pairs[p]),
                            __builtin_bit_cast(bf16x2v, xv[j][6 * q + p]), acc, false);
                }
            }
            // the row's 64 lane sums: DPP adds within each row of 16 lanes (xor 1, xor 2,
            // half mirror, mirror: every lane then holds its row's sum), then lane 0 adds the
            // other three rows' sums read with v_readlane
            acc += dpp_f32<0xB1>(acc);    // quad_perm [1, 0, 3, 2]
            acc += dpp_f32<0x4E>(acc);    // quad_perm [2, 3, 0, 1]
            acc += dpp_f32<0x141>(acc);   // row_half_mirror
            acc += dpp_f32<0x140>(acc);   // row_mirror
            const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 16));
            const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 32));
            const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 48));
            if (lane == 0 && r < N) y[r] = ((acc + r1) + r2) + r3;
        }
    }
}

}  // namespace

// One bf16 token x (K values, 16-byte aligned, K % 8 == 0 not required), packed weights w
// (N x L x 16, L = ceil(K / 48) <= 128), y (N float32) = x T^T.  `blocks` workgroups of
// four waves, `depth` rows in flight per wave (1, 2 or 4).  0, or -1 for bad arguments.
extern "C" int t81_floor_gemv_valu(const void *x, const void *w, float *y, int n, int k,
                                   int blocks, int depth, void *stream) {
    const int L = (k + 47) / 48;
    if (x == nullptr || w == nullptr || y == nullptr || n <= 0 || k <= 0 || L > 128 ||
        blocks <= 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(w) % 16 != 0 || (depth != 1 && depth != 2 && depth != 4))
        return -1;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const auto *xp = static_cast<const uint16_t *>(x);
    const auto *wp = static_cast<const uint8_t *>(w);
    if (depth == 4)
        gemv_valu_kernel<4><<<dim3(blocks), dim3(256), 0, s>>>(xp, wp, y, n, k, L);
    else if (depth == 2)
        gemv_valu_kernel<2><<<dim3(blocks), dim3(256), 0, s>>>(xp, wp, y, n, k, L);
    else
        gemv_valu_kernel<1><<<dim3(blocks), dim3(256), 0, s>>>(xp, wp, y, n, k, L);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

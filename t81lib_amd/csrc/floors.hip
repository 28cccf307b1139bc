// t81lib_amd/csrc/floors.hip -- measurement kernels for bench.py (libt81_floors.so), not
// part of the t81lib path: a plain streaming read of a buffer, the floor that any kernel
// reading the same bytes in one launch can be compared with.
//
// t81_floor_read: the buffer is cut into `blocks` contiguous spans of whole 16-byte words;
// each workgroup of 256 threads streams its span in rounds of U loads per thread, all U
// issued before any is used (consecutive threads, consecutive words: every load
// instruction reads 4 KB contiguously), XOR-folds them and writes one word per workgroup
// to out[blockIdx.x], so the loads cannot be optimised away.  U = unroll (1, 4 or 8):
// the bytes in flight per thread.  bytes must be a multiple of 16 and src 16-byte aligned.
#include <hip/hip_runtime.h>
#include <stdint.h>

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

// t81lib_amd/csrc/floors.hip -- measurement kernels for bench.py (libt81_floors.so), not
// part of the t81lib path: a plain streaming read of a buffer, the floor that any kernel
// reading the same bytes in one launch can be compared with.
//
// t81_floor_read: every thread reads 16-byte words of [src, src + bytes) in a grid-stride
// loop (consecutive threads, consecutive words: fully coalesced), XOR-folds them and
// writes one word per workgroup to out[blockIdx.x], so the loads cannot be optimised away.
// bytes must be a multiple of 16 and src 16-byte aligned.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__global__ __launch_bounds__(256) void read_floor_kernel(const uint4 *__restrict__ src,
                                                         int64_t words,
                                                         uint32_t *__restrict__ out) {
    uint4 acc = {0u, 0u, 0u, 0u};
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < words;
         i += stride) {
        const uint4 a = src[i];
        acc.x ^= a.x;
        acc.y ^= a.y;
        acc.z ^= a.z;
        acc.w ^= a.w;
    }
    uint32_t v = acc.x ^ acc.y ^ acc.z ^ acc.w;
    for (int o = 32; o > 0; o >>= 1) v ^= __shfl_xor(v, o);
    __shared__ uint32_t red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

}  // namespace

extern "C" int t81_floor_read(const void *src, int64_t bytes, uint32_t *out, int blocks,
                              void *stream) {
    if (src == nullptr || out == nullptr || bytes <= 0 || bytes % 16 != 0 || blocks <= 0 ||
        reinterpret_cast<uintptr_t>(src) % 16 != 0)
        return -1;
    read_floor_kernel<<<dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint4 *>(src), bytes / 16, out);
    return hipGetLastError() == hipSuccess ? 0 : -6;
}

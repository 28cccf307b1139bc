// t81lib_amd/csrc/transpose.hip -- the packed trit matrix transposed, in the same layout.
//
// in:  rows x L x 16 bytes, L = ceil(cols / 48): row r holds trits T[r, 0 .. cols)
// out: cols x Lt x 16 bytes, Lt = ceil(rows / 48): row k holds T[0 .. rows, k],
//      tryte j of limb l = 13 + t0 + 3 t1 + 9 t2 with t_i = T[48 l + 3 j + i, k]
//      (include/t81/core/detail/lut.hpp:13-49), trits past `rows` zero (tryte 13).
//
// The backward of y = x T^T needs dx = dy T, which is the forward product with T^T as
// the weight matrix: the transposed limbs let it run on the prefill GEMM kernel (K3)
// instead of materialising T as floats (t81/torch/__init__.py:291-304 unpacks it to
// float32 and multiplies on the host).
//
// A workgroup takes 192 input rows (four output limb columns) x 192 input columns (four
// input limbs): each input limb is read once (rows of 64 contiguous bytes) and decoded to
// int8 trits in LDS; after one barrier each output limb is assembled from a column of the
// tile, four consecutive threads writing the four consecutive limbs (64 contiguous bytes)
// of one output row.  Every byte in and out is touched once: HBM-bound.
#include "t81_device.hpp"
#include "t81_kernels.hpp"

namespace t81hip {

namespace {

constexpr int kTileLimbs = 4;                   // input limbs per tile row
constexpr int kOutLimbs = 4;                    // output limbs per tile column
constexpr int kTileCols = kTileLimbs * kTrits;  // 192 input columns = output rows
constexpr int kTileRows = kOutLimbs * kTrits;   // 192 input rows
constexpr int kPitch = kTileCols + 4;           // LDS row pitch (bytes), spreads banks

__global__ __launch_bounds__(256) void transpose_packed_kernel(const uint8_t *__restrict__ in,
                                                               uint8_t *__restrict__ out,
                                                               int64_t rows, int64_t cols,
                                                               int64_t L, int64_t Lt) {
    __shared__ __attribute__((aligned(16))) int8_t tile[kTileRows * kPitch];
    const int tid = threadIdx.x;
    const int64_t lt0 = static_cast<int64_t>(blockIdx.x) * kOutLimbs;  // first output limb
    const int64_t c0 = static_cast<int64_t>(blockIdx.y) * kTileLimbs;  // first input limb

    for (int i = tid; i < kTileRows * kTileLimbs; i += 256) {
        const int r = i / kTileLimbs;
        const int l = i % kTileLimbs;
        const int64_t row = lt0 * kTrits + r;
        const int64_t limb = c0 + l;
        uint32_t w[4] = {0x0D0D0D0Du, 0x0D0D0D0Du, 0x0D0D0D0Du, 0x0D0D0D0Du};  // zero trits
        if (row < rows && limb < L) {
            const uint4 v = *reinterpret_cast<const uint4 *>(in + (row * L + limb) * kTrytes);
            w[0] = v.x, w[1] = v.y, w[2] = v.z, w[3] = v.w;
        }
        int8_t *dst = tile + r * kPitch + l * kTrits;
#pragma unroll
        for (int b = 0; b < kTrytes; ++b) {
            const int u = static_cast<int>((w[b >> 2] >> (8 * (b & 3))) & 0xFFu);
            dst[3 * b] = static_cast<int8_t>(trit_of(u, 0));
            dst[3 * b + 1] = static_cast<int8_t>(trit_of(u, 1));
            dst[3 * b + 2] = static_cast<int8_t>(trit_of(u, 2));
        }
    }
    __syncthreads();

    for (int i = tid; i < kTileCols * kOutLimbs; i += 256) {
        const int kk = i / kOutLimbs;     // output row within the tile
        const int ol = i % kOutLimbs;     // output limb within the tile
        const int64_t k = c0 * kTrits + kk;
        const int64_t lt = lt0 + ol;
        if (k >= cols || lt >= Lt) continue;
        const int8_t *src = tile + ol * kTrits * kPitch + kk;
        uint32_t o[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            uint32_t word = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int j = 4 * d + b;  // output tryte
                const int t0 = src[(3 * j) * kPitch];
                const int t1 = src[(3 * j + 1) * kPitch];
                const int t2 = src[(3 * j + 2) * kPitch];
                word |= static_cast<uint32_t>(13 + t0 + 3 * t1 + 9 * t2) << (8 * b);
            }
            o[d] = word;
        }
        *reinterpret_cast<uint4 *>(out + (k * Lt + lt) * kTrytes) = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

}  // namespace

hipError_t launch_transpose_packed(const uint8_t *in, uint8_t *out, int64_t rows, int64_t cols,
                                   hipStream_t s) {
    if (rows == 0 || cols == 0) return hipSuccess;
    const int64_t L = (cols + kTrits - 1) / kTrits;
    const int64_t Lt = (rows + kTrits - 1) / kTrits;
    const dim3 grid(static_cast<unsigned>((Lt + kOutLimbs - 1) / kOutLimbs),
                    static_cast<unsigned>((L + kTileLimbs - 1) / kTileLimbs));
    transpose_packed_kernel<<<grid, 256, 0, s>>>(in, out, rows, cols, L, Lt);
    return hipGetLastError();
}

}  // namespace t81hip

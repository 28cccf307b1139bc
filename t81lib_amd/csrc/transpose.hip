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
// input limbs).  Phase 1: each input limb is read once (rows of 64 contiguous bytes) and
// its 48 trits go to LDS as biased digits t + 1 (one byte each, row-major), through a
// 32-entry LDS table (tryte -> its three digit bytes) and v_perm_b32: 4 table reads, 3
// permutes and 3 dword stores per 4 trytes.  Phase 2 (after one barrier): a thread takes
// four consecutive input columns x one output limb, reading the 48 rows of those four
// columns as 48 dwords; since digits are 0..2, d0 + 3 d1 + 9 d2 <= 26 per byte, so the
// trytes of the four columns come out of ordinary 32-bit multiply-adds with no carry
// between bytes, and a 4 x 4 byte transpose (v_perm_b32) turns the sixteen tryte dwords
// into the four output limbs.  Four consecutive threads write the four limbs of one output
// row (64 contiguous bytes).  Every byte in and out is touched once: HBM-bound.  (Bytes
// above 26 are not trytes; their output is unspecified.)
//
// Tile order: a tile's 64-byte input runs share 128-byte lines with the tile of the next
// input limb group, and its 64-byte output runs with the tile of the next output limb
// group.  Workgroups are dealt to the eight XCDs (each with its own L2) in turn, so the
// grid is one-dimensional and workgroup b takes tile number (b / 8) within XCD b % 8's
// contiguous share of the tiles, input limb group fastest: tiles sharing lines then run
// on one XCD at about the same time (14336 x 4096: 16.4 -> 11.4 us).
#include "t81_device.hpp"
#include "t81_kernels.hpp"

namespace t81hip {

namespace {

constexpr int kTileLimbs = 4;                   // input limbs per tile row
constexpr int kOutLimbs = 4;                    // output limbs per tile column
constexpr int kTileCols = kTileLimbs * kTrits;  // 192 input columns = output rows
constexpr int kTileRows = kOutLimbs * kTrits;   // 192 input rows
// LDS row pitch (bytes): 49 dwords, so the phase-2 dword reads of a wave -- 16 column
// groups x 4 output limbs 48 rows apart (48 * 49 = 2352 dwords = 48 mod 64 banks) -- fall
// on 64 distinct banks
constexpr int kPitch = kTileCols + 4;

// Digits of tryte u (u = 13 + t0 + 3 t1 + 9 t2): bytes t0 + 1, t1 + 1, t2 + 1; zero trits
// for the 5 byte values past 26.
__device__ __forceinline__ uint32_t digit_word(int u) {
    if (u >= 27) return 0x010101u;
    return static_cast<uint32_t>(trit_of(u, 0) + 1) |
           static_cast<uint32_t>(trit_of(u, 1) + 1) << 8 |
           static_cast<uint32_t>(trit_of(u, 2) + 1) << 16;
}

// 4 x 4 byte transpose: out[c] = byte c of a, b, cc, d.
__device__ __forceinline__ void byte_transpose4(uint32_t a, uint32_t b, uint32_t cc, uint32_t d,
                                                uint32_t (&out)[4]) {
    const uint32_t ab_lo = __builtin_amdgcn_perm(b, a, 0x05010400u);    // a0 b0 a1 b1
    const uint32_t ab_hi = __builtin_amdgcn_perm(b, a, 0x07030602u);    // a2 b2 a3 b3
    const uint32_t cd_lo = __builtin_amdgcn_perm(d, cc, 0x05010400u);
    const uint32_t cd_hi = __builtin_amdgcn_perm(d, cc, 0x07030602u);
    out[0] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u);       // a0 b0 c0 d0
    out[1] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u);       // a1 b1 c1 d1
    out[2] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u);
    out[3] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u);
}

__global__ __launch_bounds__(256) void transpose_packed_kernel(const uint8_t *__restrict__ in,
                                                               uint8_t *__restrict__ out,
                                                               int64_t rows, int64_t cols,
                                                               int64_t L, int64_t Lt, int ny) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[kTileRows * kPitch];
    __shared__ uint32_t lut[32];
    const int tid = threadIdx.x;
    // tile number tn (input limb group tn % ny, output limb group tn / ny) of workgroup wg
    const int ntiles = static_cast<int>(gridDim.x);
    const int wg = static_cast<int>(blockIdx.x);
    const int xcd = wg & 7;
    const int per = ntiles >> 3, extra = ntiles & 7;
    const int tn = xcd * per + (xcd < extra ? xcd : extra) + (wg >> 3);
    const int64_t lt0 = static_cast<int64_t>(tn / ny) * kOutLimbs;  // first output limb
    const int64_t c0 = static_cast<int64_t>(tn % ny) * kTileLimbs;  // first input limb
    if (tid < 32) lut[tid] = digit_word(tid);
    __syncthreads();

    // ---- phase 1: input limbs -> digit bytes, row-major ----
    constexpr int kIt = kTileRows * kTileLimbs / 256;
    uint4 v[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
        const int i = tid + 256 * it;
        const int64_t row = lt0 * kTrits + i / kTileLimbs;
        const int64_t limb = c0 + i % kTileLimbs;
        v[it] = make_uint4(0x0D0D0D0Du, 0x0D0D0D0Du, 0x0D0D0D0Du, 0x0D0D0D0Du);
        if (row < rows && limb < L)
            v[it] = *reinterpret_cast<const uint4 *>(in + (row * L + limb) * kTrytes);
    }
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
        const int i = tid + 256 * it;
        const int r = i / kTileLimbs;
        const int l = i % kTileLimbs;
        const uint32_t w[4] = {v[it].x, v[it].y, v[it].z, v[it].w};
        uint32_t *dst = reinterpret_cast<uint32_t *>(tile + r * kPitch + l * kTrits);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            uint32_t t[4];
#pragma unroll
            for (int b = 0; b < 4; ++b) t[b] = lut[(w[d] >> (8 * b)) & 0x1Fu];
            dst[3 * d] = __builtin_amdgcn_perm(t[1], t[0], 0x04020100u);
            dst[3 * d + 1] = __builtin_amdgcn_perm(t[2], t[1], 0x05040201u);
            dst[3 * d + 2] = __builtin_amdgcn_perm(t[3], t[2], 0x06050402u);
        }
    }
    __syncthreads();

    // ---- phase 2: four columns x one output limb per thread (192 threads) ----
    if (tid < (kTileCols / 4) * kOutLimbs) {
        const int ol = tid & 3;          // output limb within the tile
        const int kk = 4 * (tid >> 2);   // first of the four columns (output rows)
        const uint8_t *src = tile + ol * kTrits * kPitch + kk;
        uint32_t tw[16];                 // tryte j of the four columns, one per byte
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t d0 = *reinterpret_cast<const uint32_t *>(src + (3 * j) * kPitch);
            const uint32_t d1 = *reinterpret_cast<const uint32_t *>(src + (3 * j + 1) * kPitch);
            const uint32_t d2 = *reinterpret_cast<const uint32_t *>(src + (3 * j + 2) * kPitch);
            tw[j] = d0 + 3u * d1 + 9u * d2;
        }
        uint32_t o[4][4];   // o[column][dword]
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t t4[4];
            byte_transpose4(tw[4 * q], tw[4 * q + 1], tw[4 * q + 2], tw[4 * q + 3], t4);
#pragma unroll
            for (int c = 0; c < 4; ++c) o[c][q] = t4[c];
        }
        const int64_t lt = lt0 + ol;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int64_t k = c0 * kTrits + kk + c;
            if (k < cols && lt < Lt)
                *reinterpret_cast<uint4 *>(out + (k * Lt + lt) * kTrytes) =
                    make_uint4(o[c][0], o[c][1], o[c][2], o[c][3]);
        }
    }
}

}  // namespace

hipError_t launch_transpose_packed(const uint8_t *in, uint8_t *out, int64_t rows, int64_t cols,
                                   hipStream_t s) {
    if (rows == 0 || cols == 0) return hipSuccess;
    const int64_t L = (cols + kTrits - 1) / kTrits;
    const int64_t Lt = (rows + kTrits - 1) / kTrits;
    const int64_t nx = (Lt + kOutLimbs - 1) / kOutLimbs;
    const int64_t ny = (L + kTileLimbs - 1) / kTileLimbs;
    if (nx * ny > 0x7FFFFFFF) return hipErrorInvalidValue;   // tile numbers are ints
    transpose_packed_kernel<<<dim3(static_cast<unsigned>(nx * ny)), 256, 0, s>>>(
        in, out, rows, cols, L, Lt, static_cast<int>(ny));
    return hipGetLastError();
}

}  // namespace t81hip

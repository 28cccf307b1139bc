// t81lib_amd/csrc/pack.hip -- K1 threshold-quantize + pack, and the small codec kernels.
//
// K1 is HBM-bound: it reads 4 bytes per float and writes one byte per three
// trits.  One thread produces one output dword (4 trytes = 12 trits = 12
// consecutive input floats): consecutive threads read consecutive 48-byte runs
// and write consecutive dwords, so both streams are fully coalesced.
#include "pack_common.hpp"
#include "t81_device.hpp"
#include "t81_kernels.hpp"

namespace t81hip {

// K1: w (rows x cols) -> out (rows x L x 16 bytes).  Thread d owns dword q = d % 4 of
// limb l of row r, i.e. columns 48l + 12q .. 48l + 12q + 11.
template <typename T, bool kVec>
__global__ __launch_bounds__(256) void quantize_pack_rows_kernel(const T *__restrict__ w,
                                                                 uint32_t *__restrict__ out,
                                                                 int64_t rows, int64_t cols,
                                                                 int64_t limbs, float thr,
                                                                 int torch_form) {
    const int64_t d = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t per_row = limbs * 4;
    if (d >= rows * per_row) return;
    const int64_t r = d / per_row;
    const int64_t rem = d - r * per_row;
    const int64_t c0 = (rem >> 2) * kTrits + (rem & 3) * 12;
    out[d] = pack12<T, kVec>(w + r * cols, c0, cols, thr, torch_form);
}

// Column-wise activation pack: x (tokens x k) -> out (L x tokens x 16 bytes).
template <typename T, bool kVec>
__global__ __launch_bounds__(256) void quantize_pack_cols_kernel(const T *__restrict__ x,
                                                                 uint32_t *__restrict__ out,
                                                                 int64_t tokens, int64_t k,
                                                                 int64_t limbs, float thr,
                                                                 int torch_form) {
    const int64_t d = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t per_limb = tokens * 4;
    if (d >= limbs * per_limb) return;
    const int64_t l = d / per_limb;
    const int64_t rem = d - l * per_limb;
    const int64_t n = rem >> 2;
    const int64_t c0 = l * kTrits + (rem & 3) * 12;
    out[d] = pack12<T, kVec>(x + n * k, c0, k, thr, torch_form);
}

template <typename T>
__global__ __launch_bounds__(256) void quantize_kernel(const T *__restrict__ src,
                                                       int8_t *__restrict__ out, int64_t count,
                                                       float thr, int torch_form) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count) return;
    out[i] = static_cast<int8_t>(quantize_one(load_as_float<T>(src + i), thr, torch_form));
}

// out[r, c] = trit c of row r; one thread per output trit.
__global__ __launch_bounds__(256) void unpack_kernel(const uint8_t *__restrict__ packed,
                                                     int8_t *__restrict__ out, int64_t rows,
                                                     int64_t limbs, int64_t cols) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= rows * cols) return;
    const int64_t r = i / cols;
    const int64_t c = i - r * cols;
    const uint32_t u = packed[(r * limbs + c / kTrits) * kTrytes + (c % kTrits) / 3];
    const int p = static_cast<int>(c % 3);
    const uint32_t digit = p == 0 ? u % 3u : (p == 1 ? (u / 3u) % 3u : u / 9u);
    out[i] = static_cast<int8_t>(static_cast<int>(digit) - 1);
}

__global__ void fill_i32_kernel(int32_t *p, int32_t v) { *p = v; }

__global__ __launch_bounds__(256) void validate_kernel(const uint8_t *__restrict__ packed,
                                                       int64_t count, int32_t *bad) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    int32_t n = 0;
    if (i < count) n = packed[i] > 26 ? 1 : 0;
    // wavefront vote, then one atomic per wave
    const uint64_t mask = __ballot(n);
    if ((threadIdx.x & 63) == 0 && mask) atomicAdd(bad, static_cast<int32_t>(__popcll(mask)));
}

// ------------------------------------------------------------------ launchers --
static inline int64_t blocks_for(int64_t n) { return (n + 255) / 256; }

template <typename T>
static hipError_t launch_pack_rows_t(const void *w, uint8_t *out, int64_t rows, int64_t cols,
                                     float thr, int torch_form, hipStream_t s) {
    const int64_t limbs = (cols + kTrits - 1) / kTrits;
    const int64_t total = rows * limbs * 4;
    const bool vec = (cols % 4 == 0) && (reinterpret_cast<uintptr_t>(w) % 16 == 0);
    if (vec)
        quantize_pack_rows_kernel<T, true><<<dim3(blocks_for(total)), dim3(256), 0, s>>>(
            static_cast<const T *>(w), reinterpret_cast<uint32_t *>(out), rows, cols, limbs,
            thr, torch_form);
    else
        quantize_pack_rows_kernel<T, false><<<dim3(blocks_for(total)), dim3(256), 0, s>>>(
            static_cast<const T *>(w), reinterpret_cast<uint32_t *>(out), rows, cols, limbs,
            thr, torch_form);
    return hipGetLastError();
}

hipError_t launch_quantize_pack_rows(const void *w, int dtype, uint8_t *out, int64_t rows,
                                     int64_t cols, float thr, int torch_form, hipStream_t s) {
    if (rows == 0 || cols == 0) return hipSuccess;
    switch (dtype) {
        case kDtypeF32: return launch_pack_rows_t<float>(w, out, rows, cols, thr, torch_form, s);
        case kDtypeBF16: return launch_pack_rows_t<uint16_t>(w, out, rows, cols, thr, torch_form, s);
        default: return launch_pack_rows_t<_Float16>(w, out, rows, cols, thr, torch_form, s);
    }
}

template <typename T>
static hipError_t launch_pack_cols_t(const void *x, uint8_t *out, int64_t tokens, int64_t k,
                                     float thr, int torch_form, hipStream_t s) {
    const int64_t limbs = (k + kTrits - 1) / kTrits;
    const int64_t total = limbs * tokens * 4;
    const bool vec = (k % 4 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
    if (vec)
        quantize_pack_cols_kernel<T, true><<<dim3(blocks_for(total)), dim3(256), 0, s>>>(
            static_cast<const T *>(x), reinterpret_cast<uint32_t *>(out), tokens, k, limbs, thr,
            torch_form);
    else
        quantize_pack_cols_kernel<T, false><<<dim3(blocks_for(total)), dim3(256), 0, s>>>(
            static_cast<const T *>(x), reinterpret_cast<uint32_t *>(out), tokens, k, limbs, thr,
            torch_form);
    return hipGetLastError();
}

hipError_t launch_quantize_pack_cols(const void *x, int dtype, uint8_t *out, int64_t tokens,
                                     int64_t k, float thr, int torch_form, hipStream_t s) {
    if (tokens == 0 || k == 0) return hipSuccess;
    switch (dtype) {
        case kDtypeF32: return launch_pack_cols_t<float>(x, out, tokens, k, thr, torch_form, s);
        case kDtypeBF16: return launch_pack_cols_t<uint16_t>(x, out, tokens, k, thr, torch_form, s);
        default: return launch_pack_cols_t<_Float16>(x, out, tokens, k, thr, torch_form, s);
    }
}

hipError_t launch_quantize(const void *src, int dtype, int8_t *out, int64_t count, float thr,
                           int torch_form, hipStream_t s) {
    if (count == 0) return hipSuccess;
    const dim3 grid(blocks_for(count));
    switch (dtype) {
        case kDtypeF32:
            quantize_kernel<float><<<grid, dim3(256), 0, s>>>(static_cast<const float *>(src), out,
                                                             count, thr, torch_form);
            break;
        case kDtypeBF16:
            quantize_kernel<uint16_t><<<grid, dim3(256), 0, s>>>(
                static_cast<const uint16_t *>(src), out, count, thr, torch_form);
            break;
        default:
            quantize_kernel<_Float16><<<grid, dim3(256), 0, s>>>(
                static_cast<const _Float16 *>(src), out, count, thr, torch_form);
            break;
    }
    return hipGetLastError();
}

hipError_t launch_unpack(const uint8_t *packed, int8_t *out, int64_t rows, int64_t limbs,
                         int64_t cols, hipStream_t s) {
    const int64_t total = rows * cols;
    if (total == 0) return hipSuccess;
    unpack_kernel<<<dim3(blocks_for(total)), dim3(256), 0, s>>>(packed, out, rows, limbs, cols);
    return hipGetLastError();
}

hipError_t launch_validate(const uint8_t *packed, int64_t count, int32_t *bad, hipStream_t s) {
    fill_i32_kernel<<<dim3(1), dim3(1), 0, s>>>(bad, 0);
    if (count > 0)
        validate_kernel<<<dim3(blocks_for(count)), dim3(256), 0, s>>>(packed, count, bad);
    return hipGetLastError();
}

}  // namespace t81hip

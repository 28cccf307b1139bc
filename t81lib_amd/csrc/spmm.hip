// t81lib_amd/csrc/spmm.hip -- sparse ternary x dense: C = alpha * A B + beta * C with A a
// COO list of (row, col, value) entries, as t81::sparse::spmm_simple computes it
// (include/t81/sparse/simple.hpp:37-94):
//
//   C[r, k] = beta == 0 ? 0 : float(double(C[r, k]) * double(beta))
//   for every entry e in list order with row r:
//       w = double(value_e) * double(alpha)
//       C[r, k] = float(double(C[r, k]) + w * double(B[col_e, k]))
//
// Each output element is a chain of float roundings in list order, so the result depends
// on the order of a row's entries; entries of different rows never interact.  The device
// form therefore keeps, per row, the entries in their original order:
//
//  plan  (once per sparse matrix): a stable LSD radix sort of the entry positions by row
//        (8-bit digits, 1024-entry tiles; per tile a digit histogram, one exclusive scan
//        over all [digit][tile] counts, then a scatter whose in-tile ranks come from
//        wavefront ballots, so equal rows keep list order), then the entries' columns and
//        values gathered in that order and row_ptr[r] = first sorted position of row r.
//  apply (the hot kernel): G lanes per (row, feature chunk), each lane V adjacent features;
//        the lane walks the row's entries in order and replays the chain above in double,
//        with contraction off so every multiply and add is rounded as the reference's.
//        Reads per entry: its column (4 B), its value (8 B) and one G*V-float slice of B
//        (reused across rows through L2); C is read (beta != 0) and written once.
#include "t81_device.hpp"
#include "t81_kernels.hpp"

#pragma clang fp contract(off)

namespace t81hip {

namespace {

constexpr int kSortThreads = 256;
constexpr int kSortItems = 4;
constexpr int kSortTile = kSortThreads * kSortItems;  // entries per tile
constexpr int kScanThreads = 1024;
constexpr int kScanItems = 4;

__global__ __launch_bounds__(256) void spmm_first_bad_kernel(const int32_t *__restrict__ row_idx,
                                                             const int32_t *__restrict__ col_idx,
                                                             int64_t nnz, int rows, int cols,
                                                             unsigned long long *first_bad) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < nnz;
         e += stride) {
        const int r = row_idx[e];
        const int c = col_idx[e];
        if (r < 0 || r >= rows || c < 0 || c >= cols)
            atomicMin(first_bad, static_cast<unsigned long long>(e));
    }
}

__global__ void spmm_set_u64_kernel(unsigned long long *p, unsigned long long v) { *p = v; }

// Digit counts per tile: hist[d * ntiles + tile].
__global__ __launch_bounds__(kSortThreads) void radix_hist_kernel(const uint32_t *__restrict__ keys,
                                                                  int64_t n, int shift,
                                                                  int64_t ntiles,
                                                                  uint32_t *__restrict__ hist) {
    __shared__ uint32_t cnt[256];
    const int tid = threadIdx.x;
    cnt[tid] = 0;
    __syncthreads();
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int64_t i = base + j * kSortThreads + tid;
        if (i < n) atomicAdd(&cnt[(keys[i] >> shift) & 0xFFu], 1u);
    }
    __syncthreads();
    hist[static_cast<int64_t>(tid) * ntiles + blockIdx.x] = cnt[tid];
}

// In-place exclusive scan of m uint32 values (sum < 2^32) by one workgroup.
__global__ __launch_bounds__(kScanThreads) void exclusive_scan_kernel(uint32_t *__restrict__ data,
                                                                      int64_t m) {
    __shared__ uint32_t wsum[kScanThreads / 64];
    __shared__ uint32_t total;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    uint32_t carry = 0;
    for (int64_t base = 0; base < m; base += kScanThreads * kScanItems) {
        uint32_t v[kScanItems];
        uint32_t local = 0;
#pragma unroll
        for (int q = 0; q < kScanItems; ++q) {
            const int64_t idx = base + static_cast<int64_t>(tid) * kScanItems + q;
            v[q] = idx < m ? data[idx] : 0u;
            local += v[q];
        }
        uint32_t x = local;  // inclusive scan over the wavefront
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t y = __shfl_up(x, off, 64);
            if (lane >= off) x += y;
        }
        if (lane == 63) wsum[wave] = x;
        __syncthreads();
        if (wave == 0) {
            uint32_t s = lane < kScanThreads / 64 ? wsum[lane] : 0u;
#pragma unroll
            for (int off = 1; off < kScanThreads / 64; off <<= 1) {
                const uint32_t y = __shfl_up(s, off, 64);
                if (lane >= off) s += y;
            }
            if (lane < kScanThreads / 64) wsum[lane] = s;  // inclusive over waves
            if (lane == kScanThreads / 64 - 1) total = s;
        }
        __syncthreads();
        uint32_t run = carry + (wave ? wsum[wave - 1] : 0u) + x - local;
#pragma unroll
        for (int q = 0; q < kScanItems; ++q) {
            const int64_t idx = base + static_cast<int64_t>(tid) * kScanItems + q;
            if (idx < m) data[idx] = run;
            run += v[q];
        }
        carry += total;
        __syncthreads();  // wsum / total are rewritten by the next chunk
    }
}

// Stable scatter of one 8-bit digit.  vals_in == nullptr reads the identity (position i).
__global__ __launch_bounds__(kSortThreads) void radix_scatter_kernel(
    const uint32_t *__restrict__ keys_in, const uint32_t *__restrict__ vals_in,
    uint32_t *__restrict__ keys_out, uint32_t *__restrict__ vals_out, int64_t n, int shift,
    int64_t ntiles, const uint32_t *__restrict__ offs) {
    __shared__ uint32_t base[256];
    __shared__ uint32_t wcnt[kSortThreads / 64][256];
    const int tid = threadIdx.x;
    const int w = tid >> 6;
    base[tid] = offs[static_cast<int64_t>(tid) * ntiles + blockIdx.x];
    const int64_t tile0 = static_cast<int64_t>(blockIdx.x) * kSortTile;
    for (int j = 0; j < kSortItems; ++j) {
#pragma unroll
        for (int q = 0; q < kSortThreads / 64; ++q) wcnt[q][tid] = 0;  // column tid only
        __syncthreads();
        const int64_t i = tile0 + j * kSortThreads + tid;
        const bool valid = i < n;
        const uint32_t key = valid ? keys_in[i] : 0u;
        const uint32_t val = valid ? (vals_in ? vals_in[i] : static_cast<uint32_t>(i)) : 0u;
        const uint32_t d = (key >> shift) & 0xFFu;
        uint64_t peers = __builtin_amdgcn_ballot_w64(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const bool bit = (d >> b) & 1u;
            const uint64_t bal = __builtin_amdgcn_ballot_w64(bit);
            peers &= bit ? bal : ~bal;
        }
        // lanes below this one holding the same digit
        const uint32_t rank = __builtin_amdgcn_mbcnt_hi(
            static_cast<uint32_t>(peers >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(peers), 0u));
        if (valid && rank == 0) wcnt[w][d] = static_cast<uint32_t>(__builtin_popcountll(peers));
        __syncthreads();
        if (valid) {
            uint32_t pos = base[d] + rank;
            for (int q = 0; q < w; ++q) pos += wcnt[q][d];
            keys_out[pos] = key;
            vals_out[pos] = val;
        }
        __syncthreads();
        uint32_t add = 0;
#pragma unroll
        for (int q = 0; q < kSortThreads / 64; ++q) add += wcnt[q][tid];
        base[tid] += add;
    }
}

__global__ __launch_bounds__(256) void spmm_gather_kernel(const uint32_t *__restrict__ perm,
                                                          const int32_t *__restrict__ col_idx,
                                                          const int64_t *__restrict__ values,
                                                          int32_t *__restrict__ cols_out,
                                                          double *__restrict__ vals_out, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint32_t e = perm[i];
        cols_out[i] = col_idx[e];
        // exact integer -> double, rounded once to nearest even: the value of
        // limb_to_double (simple.hpp:25-33) for a limb built from this integer
        vals_out[i] = static_cast<double>(values[e]);
    }
}

// row_ptr[r] = first sorted position whose row is >= r, r = 0 .. rows.
__global__ __launch_bounds__(256) void spmm_row_ptr_kernel(const uint32_t *__restrict__ keys, int64_t n,
                                                           int rows, int32_t *__restrict__ row_ptr) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r > rows) return;
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (static_cast<int64_t>(keys[mid]) < r)
            lo = mid + 1;
        else
            hi = mid;
    }
    row_ptr[r] = static_cast<int32_t>(lo);
}

template <int V>
struct FloatVec;
template <>
struct FloatVec<1> {
    using type = float;
};
template <>
struct FloatVec<2> {
    using type = float2;
};
template <>
struct FloatVec<4> {
    using type = float4;
};

template <int V>
__device__ __forceinline__ void vload(const float *p, float (&out)[V]) {
    const auto v = *reinterpret_cast<const typename FloatVec<V>::type *>(p);
    if constexpr (V == 1) {
        out[0] = v;
    } else if constexpr (V == 2) {
        out[0] = v.x, out[1] = v.y;
    } else {
        out[0] = v.x, out[1] = v.y, out[2] = v.z, out[3] = v.w;
    }
}

template <int V>
__device__ __forceinline__ void vstore(float *p, const float (&in)[V]) {
    using T = typename FloatVec<V>::type;
    if constexpr (V == 1) {
        *p = in[0];
    } else if constexpr (V == 2) {
        *reinterpret_cast<T *>(p) = make_float2(in[0], in[1]);
    } else {
        *reinterpret_cast<T *>(p) = make_float4(in[0], in[1], in[2], in[3]);
    }
}

constexpr int kApplyUnroll = 4;

// One group of G = 2^gshift lanes per (row, chunk of G*V features); N % V == 0.
template <int V>
__global__ __launch_bounds__(256) void spmm_apply_kernel(const int32_t *__restrict__ row_ptr,
                                                         const int32_t *__restrict__ cols,
                                                         const double *__restrict__ vals,
                                                         const float *__restrict__ B,
                                                         float *__restrict__ C, int64_t rows,
                                                         int64_t N, int gshift, int64_t nchunks,
                                                         double alpha, double beta, int beta_zero) {
    const int lig = threadIdx.x & ((1 << gshift) - 1);
    const int64_t total = rows * nchunks;
    const int64_t step = static_cast<int64_t>(gridDim.x) * (blockDim.x >> gshift);
    for (int64_t g = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> gshift;
         g < total; g += step) {
        const int64_t row = g / nchunks;
        const int64_t k0 = (((g - row * nchunks) << gshift) + lig) * V;
        const bool active = k0 < N;
        float acc[V];
        float *c = C + row * N + k0;
        if (beta_zero || !active) {
#pragma unroll
            for (int v = 0; v < V; ++v) acc[v] = 0.0f;
        } else {
            vload<V>(c, acc);
#pragma unroll
            for (int v = 0; v < V; ++v) acc[v] = static_cast<float>(static_cast<double>(acc[v]) * beta);
        }
        const int32_t e_end = row_ptr[row + 1];
        int32_t e = row_ptr[row];
        if (active) {
            const float *bk = B + k0;
            for (; e + kApplyUnroll <= e_end; e += kApplyUnroll) {
                float b[kApplyUnroll][V];
                double w[kApplyUnroll];
#pragma unroll
                for (int u = 0; u < kApplyUnroll; ++u) {
                    vload<V>(bk + static_cast<int64_t>(cols[e + u]) * N, b[u]);
                    w[u] = vals[e + u];
                }
#pragma unroll
                for (int u = 0; u < kApplyUnroll; ++u) {
                    const double wu = w[u] * alpha;
#pragma unroll
                    for (int v = 0; v < V; ++v)
                        acc[v] = static_cast<float>(static_cast<double>(acc[v]) +
                                                    wu * static_cast<double>(b[u][v]));
                }
            }
            for (; e < e_end; ++e) {
                float b[V];
                vload<V>(bk + static_cast<int64_t>(cols[e]) * N, b);
                const double wu = vals[e] * alpha;
#pragma unroll
                for (int v = 0; v < V; ++v)
                    acc[v] = static_cast<float>(static_cast<double>(acc[v]) + wu * static_cast<double>(b[v]));
            }
            vstore<V>(c, acc);
        }
    }
}

inline unsigned grid_for(int64_t work, int64_t per_block, int64_t cap) {
    const int64_t blocks = (work + per_block - 1) / per_block;
    return static_cast<unsigned>(blocks < 1 ? 1 : (blocks > cap ? cap : blocks));
}

}  // namespace

hipError_t launch_spmm_first_bad(const int32_t *row_idx, const int32_t *col_idx, int64_t nnz,
                                 int rows, int cols, unsigned long long *first_bad, hipStream_t s) {
    spmm_set_u64_kernel<<<1, 1, 0, s>>>(first_bad, static_cast<unsigned long long>(nnz));
    if (nnz > 0)
        spmm_first_bad_kernel<<<grid_for(nnz, 256, 8192), 256, 0, s>>>(row_idx, col_idx, nnz, rows,
                                                                        cols, first_bad);
    return hipGetLastError();
}

size_t spmm_sort_scratch_bytes(int64_t n) {
    const int64_t ntiles = (n + kSortTile - 1) / kSortTile;
    return static_cast<size_t>(4 * n + 256 * ntiles) * sizeof(uint32_t);
}

hipError_t launch_spmm_build(const int64_t *values, const int32_t *row_idx, const int32_t *col_idx,
                             int64_t n, int rows, void *scratch, int32_t *row_ptr,
                             int32_t *cols_out, double *vals_out, hipStream_t s) {
    if (n > 0) {
        const int64_t ntiles = (n + kSortTile - 1) / kSortTile;
        uint32_t *keys[2] = {static_cast<uint32_t *>(scratch), static_cast<uint32_t *>(scratch) + n};
        uint32_t *perm[2] = {keys[1] + n, keys[1] + 2 * n};
        uint32_t *hist = keys[1] + 3 * n;
        int bits = 0;
        while (bits < 31 && (int64_t{1} << bits) < rows) ++bits;  // row < 2^bits
        const int passes = bits <= 8 ? 1 : (bits + 7) / 8;
        for (int p = 0; p < passes; ++p) {
            const uint32_t *kin = p == 0 ? reinterpret_cast<const uint32_t *>(row_idx) : keys[(p - 1) & 1];
            const uint32_t *vin = p == 0 ? nullptr : perm[(p - 1) & 1];
            radix_hist_kernel<<<static_cast<unsigned>(ntiles), kSortThreads, 0, s>>>(kin, n, 8 * p,
                                                                                    ntiles, hist);
            exclusive_scan_kernel<<<1, kScanThreads, 0, s>>>(hist, 256 * ntiles);
            radix_scatter_kernel<<<static_cast<unsigned>(ntiles), kSortThreads, 0, s>>>(
                kin, vin, keys[p & 1], perm[p & 1], n, 8 * p, ntiles, hist);
        }
        const int last = (passes - 1) & 1;
        spmm_gather_kernel<<<grid_for(n, 256, 8192), 256, 0, s>>>(perm[last], col_idx, values,
                                                                    cols_out, vals_out, n);
        spmm_row_ptr_kernel<<<grid_for(int64_t{rows} + 1, 256, INT32_MAX), 256, 0, s>>>(
            keys[last], n, rows, row_ptr);
    } else {
        spmm_row_ptr_kernel<<<grid_for(int64_t{rows} + 1, 256, INT32_MAX), 256, 0, s>>>(
            nullptr, 0, rows, row_ptr);
    }
    return hipGetLastError();
}

hipError_t launch_spmm_apply(const int32_t *row_ptr, const int32_t *cols, const double *vals,
                             const float *B, float *C, int rows, int64_t N, float alpha, float beta,
                             hipStream_t s) {
    if (rows == 0 || N == 0) return hipSuccess;
    const uintptr_t align = reinterpret_cast<uintptr_t>(B) | reinterpret_cast<uintptr_t>(C);
    int V = 1;
    if (N % 4 == 0 && N >= 256 && align % 16 == 0)
        V = 4;
    else if (N % 2 == 0 && N >= 128 && align % 8 == 0)
        V = 2;
    const int64_t lanes = (N + V - 1) / V;
    int gshift = 0;
    while (gshift < 6 && (int64_t{1} << gshift) < lanes) ++gshift;
    const int64_t nchunks = (lanes + (int64_t{1} << gshift) - 1) >> gshift;
    const int64_t threads = static_cast<int64_t>(rows) * nchunks << gshift;
    const unsigned grid = grid_for(threads, 256, int64_t{1} << 20);
    const double ad = static_cast<double>(alpha), bd = static_cast<double>(beta);
    const int bz = beta == 0.0f ? 1 : 0;
    if (V == 4)
        spmm_apply_kernel<4><<<grid, 256, 0, s>>>(row_ptr, cols, vals, B, C, rows, N, gshift, nchunks,
                                                  ad, bd, bz);
    else if (V == 2)
        spmm_apply_kernel<2><<<grid, 256, 0, s>>>(row_ptr, cols, vals, B, C, rows, N, gshift, nchunks,
                                                  ad, bd, bz);
    else
        spmm_apply_kernel<1><<<grid, 256, 0, s>>>(row_ptr, cols, vals, B, C, rows, N, gshift, nchunks,
                                                  ad, bd, bz);
    return hipGetLastError();
}

}  // namespace t81hip

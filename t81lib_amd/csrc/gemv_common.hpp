// t81lib_amd/csrc/gemv_common.hpp -- pieces shared by the decode-GEMV kernels
// (gemv.hip, gemv_strip.hip): activation loads, limb loads, the MFMA step.
// Everything here has internal linkage: each translation unit gets its own copy.
#pragma once

#include "t81_device.hpp"
#include "t81_kernels.hpp"

namespace t81hip {

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Cache-policy operand of a buffer load: the non-temporal (streaming) hint, bit 1 of
// the gfx950 cache-policy field.
constexpr int kCpolNt = 2;

// ---- activation fragments: 8 consecutive X[m, k0 .. k0+8) as bf16 (hi, lo) ----
// Out-of-range lanes read from kZeroBlock / kPadLimb instead of selecting a value
// after the load: the loads stay unconditional and nothing has to wait for them
// until the data is used, so the compiler can count outstanding loads exactly
// (s_waitcnt vmcnt(n) rather than vmcnt(0)) and the weight ring stays in flight.
// Both are ordinary (read-only in practice) global arrays: a `const` qualifier would
// place them in the constant address space and turn the selected loads into flat loads.
__device__ uint32_t kZeroBlock[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
__device__ uint32_t kPadLimb[4] = {0x0D0D0D0Du, 0x0D0D0D0Du, 0x0D0D0D0Du, 0x0D0D0D0Du};

// Raw bits of 8 activations: bf16 -> a (16 bytes); fp32 -> a, b (32 bytes); int8 -> a.xy.
struct XRaw {
    u32x4 a, b;
};

// kAligned: K % 8 == 0 and x 16-byte aligned (8-byte for int8), so a chunk of 8 is
// either entirely inside K or entirely past it.
template <int XT, bool kAligned>
__device__ __forceinline__ XRaw load_x8_raw(const void *x, int64_t row_off, int64_t k0,
                                            int64_t K, bool valid) {
    constexpr int kElem = XT == kDtypeF32 ? 4 : (XT == kDtypeBF16 ? 2 : 1);
    XRaw raw;
    if constexpr (kAligned) {
        const bool ok = valid && k0 < K;
        const uint8_t *p = ok ? static_cast<const uint8_t *>(x) + (row_off + k0) * kElem
                              : reinterpret_cast<const uint8_t *>(kZeroBlock);
        if constexpr (XT == kDtypeBF16) {
            raw.a = *reinterpret_cast<const u32x4 *>(p);
        } else if constexpr (XT == kDtypeF32) {
            raw.a = reinterpret_cast<const u32x4 *>(p)[0];
            raw.b = reinterpret_cast<const u32x4 *>(p)[1];
        } else {
            const uint2 v = *reinterpret_cast<const uint2 *>(p);
            raw.a = u32x4{v.x, v.y, 0u, 0u};
        }
    } else {
        uint32_t e[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const bool ok = valid && (k0 + i < K);
            const uint8_t *p = ok ? static_cast<const uint8_t *>(x) + (row_off + k0 + i) * kElem
                                  : reinterpret_cast<const uint8_t *>(kZeroBlock);
            if constexpr (XT == kDtypeBF16) e[i] = *reinterpret_cast<const uint16_t *>(p);
            else if constexpr (XT == kDtypeF32) e[i] = *reinterpret_cast<const uint32_t *>(p);
            else e[i] = *p;
        }
        if constexpr (XT == kDtypeBF16) {
            raw.a = u32x4{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16),
                          e[6] | (e[7] << 16)};
        } else if constexpr (XT == kDtypeF32) {
            raw.a = u32x4{e[0], e[1], e[2], e[3]};
            raw.b = u32x4{e[4], e[5], e[6], e[7]};
        } else {
            raw.a = u32x4{e[0] | (e[1] << 8) | (e[2] << 16) | (e[3] << 24),
                          e[4] | (e[5] << 8) | (e[6] << 16) | (e[7] << 24), 0u, 0u};
        }
    }
    return raw;
}

// bf16 operands of 8 raw activations: bf16 as is; fp32 as x = hi + lo with
// hi = bf16(x), lo = bf16(x - hi), |x - hi - lo| <= 2^-18 |x|; int8 exactly.
template <int XT>
__device__ __forceinline__ void cvt_x8(const XRaw &raw, bf16x8 &hi, bf16x8 &lo) {
    const u32x4 zero = {0u, 0u, 0u, 0u};
    if constexpr (XT == kDtypeBF16) {
        hi = __builtin_bit_cast(bf16x8, raw.a);
        lo = __builtin_bit_cast(bf16x8, zero);
    } else if constexpr (XT == kDtypeF32) {
        const uint32_t v[8] = {raw.a[0], raw.a[1], raw.a[2], raw.a[3],
                               raw.b[0], raw.b[1], raw.b[2], raw.b[3]};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float f = __uint_as_float(v[i]);
            const __bf16 h = static_cast<__bf16>(f);
            hi[i] = h;
            lo[i] = static_cast<__bf16>(f - static_cast<float>(h));
        }
    } else {
        const uint32_t w[2] = {raw.a[0], raw.a[1]};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int8_t b = static_cast<int8_t>((w[i / 4] >> (8 * (i % 4))) & 0xFFu);
            hi[i] = static_cast<__bf16>(static_cast<float>(b));
        }
        lo = __builtin_bit_cast(bf16x8, zero);
    }
}

template <int XT, bool kAligned>
__device__ __forceinline__ void load_x8(const void *x, int64_t row_off, int64_t k0, int64_t K,
                                        bool valid, bf16x8 &hi, bf16x8 &lo) {
    cvt_x8<XT>(load_x8_raw<XT, kAligned>(x, row_off, k0, K, valid), hi, lo);
}

// Limb `limb` of weight row `row`, or the padding limb (all-zero trits) past the
// matrix or past the caller's limb range [.., limb_end).
__device__ __forceinline__ u32x4 load_limb(const uint8_t *w, int64_t row, int64_t limb,
                                           int64_t N, int64_t L, int64_t limb_end) {
    const bool ok = row < N && limb < limb_end && limb < L;
    const uint8_t *p = ok ? w + (row * L + limb) * kTrytes
                          : reinterpret_cast<const uint8_t *>(kPadLimb);
    return *reinterpret_cast<const u32x4 *>(p);
}

// acc += A x B over the six 8-trit slots of one limb per lane-quarter; pairs[] holds
// the limb decoded to 24 bf16 pairs (A), bh / bl the activations (lo plane for fp32).
template <int XT>
__device__ __forceinline__ floatx4 mfma_pairs(const uint32_t *pairs, const bf16x8 *bh,
                                              const bf16x8 *bl, floatx4 acc) {
#pragma unroll
    for (int j = 0; j < 6; ++j) {
        const u32x4 araw = {pairs[4 * j], pairs[4 * j + 1], pairs[4 * j + 2], pairs[4 * j + 3]};
        const bf16x8 a = __builtin_bit_cast(bf16x8, araw);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bh[j], acc, 0, 0, 0);
        if constexpr (XT == kDtypeF32)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl[j], acc, 0, 0, 0);
    }
    return acc;
}

// mfma_pairs with the six MFMAs alternating between two accumulators.
template <int XT>
__device__ __forceinline__ void mfma_pairs2(const uint32_t *pairs, const bf16x8 *bh,
                                            const bf16x8 *bl, floatx4 &acc0, floatx4 &acc1) {
#pragma unroll
    for (int j = 0; j < 6; ++j) {
        const u32x4 araw = {pairs[4 * j], pairs[4 * j + 1], pairs[4 * j + 2], pairs[4 * j + 3]};
        const bf16x8 a = __builtin_bit_cast(bf16x8, araw);
        floatx4 &acc = (j & 1) ? acc1 : acc0;
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bh[j], acc, 0, 0, 0);
        if constexpr (XT == kDtypeF32)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl[j], acc, 0, 0, 0);
    }
}

// acc += T(16 rows, one limb per lane-quarter) x B  over the six 8-trit slots of the limb.
template <int XT>
__device__ __forceinline__ floatx4 mfma_limb(const uint8_t *lut, u32x4 wl, const bf16x8 *bh,
                                             const bf16x8 *bl, floatx4 acc) {
    uint32_t pairs[24];
#pragma unroll
    for (int d = 0; d < 4; ++d) decode_dword(lut, wl[d], pairs + 6 * d);
    return mfma_pairs<XT>(pairs, bh, bl, acc);
}


}  // namespace

}  // namespace t81hip

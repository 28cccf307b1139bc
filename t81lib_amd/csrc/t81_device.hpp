// t81lib_amd/csrc/t81_device.hpp -- device-side helpers shared by the gfx950 kernels.
//
// Tryte code (include/t81/core/detail/lut.hpp:13-49): byte u = 13 + t0 + 3*t1 + 9*t2,
// i.e. the base-3 digits of u are t_i + 1.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace t81hip {

constexpr int kTrits = 48;
constexpr int kTrytes = 16;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

__host__ __device__ constexpr int trit_of(int u, int p) {
    return p == 0 ? (u % 3) - 1 : (p == 1 ? ((u / 3) % 3) - 1 : (u / 9) - 1);
}

__host__ __device__ constexpr uint32_t bf16_bits_of_trit(int t) {
    return t > 0 ? 0x3F80u : (t < 0 ? 0xBF80u : 0u);
}

// ---------------------------------------------------------------------------
// Decode tables in LDS.  For a byte u (one tryte = trits t0,t1,t2):
//   E[u] = { bf16(t0) | bf16(t1) << 16,  bf16(t2) }
//   F[u] = { bf16(t0) << 16,             bf16(t1) | bf16(t2) << 16 }
// Two consecutive bytes (a, b) hold trits 0..5 of a 6-trit run; the three
// natural-order bf16 pairs are E[a].x, E[a].y | F[b].x and F[b].y.  Entries are
// 8 bytes, so a byte value u addresses offset 8u; u < 32 for every valid byte,
// which lets (word << 3) place each byte's 8u in its own 8-bit field.  The
// field is masked to 8 bits, so even an invalid byte (> 26) addresses at most
// 255 + 8 bytes past a table start: the region below is zero-filled to cover it.
constexpr int kLutE = 0;                    // byte offset of E
constexpr int kLutF = 256;                  // byte offset of F
constexpr int kLutBytes = 256 + 256 + 16;   // F start + max field + one entry

// Writes the E/F tables (and the zero fill around them) with one pass: thread i
// owns word i, so no barrier is needed between fill and entries.  The caller
// issues the __syncthreads() that publishes the table.
__device__ __forceinline__ void lut_fill(uint8_t *lds, int tid, int nthreads) {
    uint32_t *words = reinterpret_cast<uint32_t *>(lds);
    for (int i = tid; i < kLutBytes / 4; i += nthreads) {
        const int off = 4 * i;
        uint32_t v = 0u;
        const bool in_e = off < kLutF;
        const int rel = in_e ? off - kLutE : off - kLutF;
        const int u = rel / 8;
        const int part = (rel % 8) / 4;
        if (rel >= 0 && u < 27 && off < kLutF + 8 * 27) {
            const uint32_t b0 = bf16_bits_of_trit(trit_of(u, 0));
            const uint32_t b1 = bf16_bits_of_trit(trit_of(u, 1));
            const uint32_t b2 = bf16_bits_of_trit(trit_of(u, 2));
            if (in_e) v = part == 0 ? (b0 | (b1 << 16)) : b2;
            else v = part == 0 ? (b0 << 16) : (b1 | (b2 << 16));
        }
        words[i] = v;
    }
}

__device__ __forceinline__ void lut_init(uint8_t *lds, int tid, int nthreads) {
    lut_fill(lds, tid, nthreads);
    __syncthreads();
}

// Decodes one packed dword (4 bytes = 12 trits, natural order) into 6 dwords of
// bf16 pairs: out[i] = { bf16(t[2i]), bf16(t[2i+1]) }.
__device__ __forceinline__ void decode_dword(const uint8_t *lds, uint32_t w, uint32_t *out) {
    const uint32_t w8 = w << 3;
    const uint32_t a0 = w8 & 0xFFu;
    const uint32_t a1 = (w8 >> 8) & 0xFFu;
    const uint32_t a2 = (w8 >> 16) & 0xFFu;
    const uint32_t a3 = w8 >> 24;
    const uint2 e0 = *reinterpret_cast<const uint2 *>(lds + kLutE + a0);
    const uint2 f1 = *reinterpret_cast<const uint2 *>(lds + kLutF + a1);
    const uint2 e2 = *reinterpret_cast<const uint2 *>(lds + kLutE + a2);
    const uint2 f3 = *reinterpret_cast<const uint2 *>(lds + kLutF + a3);
    out[0] = e0.x;
    out[1] = e0.y | f1.x;
    out[2] = f1.y;
    out[3] = e2.x;
    out[4] = e2.y | f3.x;
    out[5] = f3.y;
}

// Immediate of an s_waitcnt that waits until at most N vector-memory loads of the wave are
// outstanding and leaves the other counters alone (gfx9 encoding: vmcnt in bits 3:0 and
// 15:14, expcnt in 6:4 at its maximum 7, lgkmcnt in 11:8 at its maximum 15).  Loads
// complete in issue order, so this waits exactly for every load issued before the newest N.
template <int N>
constexpr int waitcnt_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt holds 0..63");
    return (N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8);
}
static_assert(waitcnt_vm<4>() == 0x0F74 && waitcnt_vm<9>() == 0x0F79, "gfx9 s_waitcnt layout");

// Global -> LDS loads (buffer loads with the LDS bit) gave wrong results when their target
// reached past 128 KiB of the 160 KiB LDS; kernels that issue them keep every static LDS
// object below this bound (their total static LDS <= kLdsDmaLimit, checked where declared).
constexpr int kLdsDmaLimit = 128 * 1024;

__device__ __forceinline__ uint16_t bf16_bits_rne(float f) {
    // round-to-nearest-even float -> bf16 (NaN kept quiet)
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float bf16_bits_to_float(uint32_t b) { return __uint_as_float(b << 16); }

}  // namespace t81hip

// t81lib_amd/csrc/gemm_i8.hip -- K3 for int8 activations on the integer matrix cores.
//
//   C[m, n] = sum_k X[m, k] * T[n, k] (+ C[m, n] when beta == 1), int32, exact
//
// The bf16 big-tile kernel (gemm.hip) with the integer MFMA v_mfma_i32_32x32x32_i8 in
// place of v_mfma_f32_32x32x16_bf16: trits decode to int8 (-1, 0, +1), the activations
// go to the matrix cores as they are, and the sums are int32 -- exact for any K the
// int32 result can hold (|sum| <= 128 K), at twice the bf16 rate (5 POP/s dense).
//
// Tiling (as the bf16 kernel): a workgroup of four waves, one per SIMD, computes a
// 256 x 256 tile of C^T (or a tall 512 x 128 one, the waves along the rows); wave (wn, wm)
// owns 128 weight rows x 128 tokens, 4 x 4 blocks of 32 x 32 int32 accumulators (all 256
// AGPRs).  A k-step is two limbs (96 trits):
//  * lane (r, h) loads the 16 bytes of limb 2s + h of row 32 rb + r and decodes it into
//    three 16-trit operands (J = 0, 1, 2: trits 16J .. 16J + 15 of the limb, one int8
//    each); B lane (c, h) reads X[c, 96 s + 48 h + 16 J .. + 16], 16 bytes of the
//    activation tile.  A lane's element e and the B lane's element e are the same k, so
//    every MFMA pairs each trit with its own activation;
//  * decode: a 64 KB LDS pair table maps two trytes (the weight dword's bytes 0-1 or 2-3,
//    addressed as (w & 0x1F1F) << 3 -- two VALU ops) to their six int8 trits; a weight
//    dword's two entries become the three natural-order dwords of its twelve trits with
//    one v_perm_b32 and one v_alignbit_b32 (2 table reads and 6 VALU ops per dword, where
//    a one-tryte table took 4 reads and 8: M = 2048 gate_up 274 -> 263 us, M = 8192
//    1000 -> 954 us);
//  * the activation tile of step s + 1 (256 tokens x 96 int8, rows of 7 16-byte slots,
//    one a pad slot so that the 16-byte B reads of 16 lanes fall on distinct banks) goes
//    straight from global memory into the other LDS buffer with buffer loads carrying
//    the LDS bit, issued during step s; one barrier per step.  Chunks past K or past M,
//    and the pad slots, load zeros (out-of-range buffer offsets), so K must be a multiple
//    of 16 (a chunk never straddles the end of a row).
// Work items, rounds, the rows after whole rounds (one round of half-width tiles, or
// split-K items) and the LDS-staged epilogue follow the bf16 kernel; split partials are
// int32 and sum exactly.
#include "t81_device.hpp"
#include "t81_kernels.hpp"

namespace t81hip {

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kI8Threads = 256;
constexpr int kI8Rows = 256;                      // weight rows per workgroup
constexpr int kI8Tokens = 256;                    // tokens per workgroup
constexpr int kI8StepK = 2 * kTrits;              // trits per k-step
constexpr int kI8RowSlots = kI8StepK / 16 + 1;    // 16-byte slots per tile row (+1 pad)
constexpr int kI8RowBytes = 16 * kI8RowSlots;     // 112
constexpr int kI8TileBytes = kI8Tokens * kI8RowBytes;
constexpr uint32_t kI8Oob = 0x80000000u;
constexpr int kI8StageStride = 68;                // int32 per staged output row (64 + 4 pad)
constexpr int kI8StageWave = 32 * kI8StageStride * 4;   // bytes of one wave's staging region
// pair table: entry b0 + 256 b1 (8 bytes) for every pair of 5-bit byte values
constexpr int kI8LutBytes = 32 * 256 * 8;

static_assert(kI8Tokens * kI8RowSlots % (64 * 4) == 0, "tile loads must split evenly");

__device__ __forceinline__ __amdgpu_buffer_rsrc_t i8_rsrc(const void *base, int64_t bytes) {
    const uint64_t p = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32));
    const int n = __builtin_amdgcn_readfirstlane(bytes < 0x7FFFFFFF ? static_cast<int>(bytes)
                                                                    : 0x7FFFFFFF);
    return __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void *>((static_cast<uint64_t>(hi) << 32) | lo), 0, n, 0x00020000);
}

// Three int8 trits of tryte u (u = 13 + t0 + 3 t1 + 9 t2) in bytes 0-2, zero past 26.
__device__ __forceinline__ uint32_t i8_trits(int u) {
    if (u >= 27) return 0u;
    return static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(trit_of(u, 0)))) |
           static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(trit_of(u, 1)))) << 8 |
           static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(trit_of(u, 2)))) << 16;
}
// Entry b0 + 256 b1 = the six trits of trytes b0, b1 in bytes 0-5 (bytes 6, 7 zero), for
// b0, b1 < 32: a weight dword's bytes 0-1 (or 2-3) address theirs as (w & 0x1F1F) << 3.
// Only those 1024 of the 8192 slots are ever read.
__device__ __forceinline__ void i8_lut_fill(uint8_t *lds, int tid, int nthreads) {
    uint32_t *words = reinterpret_cast<uint32_t *>(lds);
    for (int i = tid; i < 1024; i += nthreads) {
        const int b0 = i & 31, b1 = i >> 5;
        const uint32_t lo = i8_trits(b0), hi = i8_trits(b1);
        words[2 * (b0 + 256 * b1)] = lo | (hi << 24);
        words[2 * (b0 + 256 * b1) + 1] = hi >> 8;
    }
}

// Work items.  Rows [0, n1) run as whole 256 x 256 tiles.  Rows [n1, N) run either as
// split-K items (nsplit > 0), storing raw int32 partials to part in (split, tile, wave,
// block, a4, lane) order, summed by gemm_split_reduce_i8_kernel, or (half != 0) as
// half-width tiles of 256 rows x 128 tokens over all k-steps, straight to C, when those
// fill about one round of the CUs.  Half of the remainder's items come first in the item
// order and half last (see the bf16 kernel).
// kHalf: the instance with the half-width path (compiled apart, so that the whole-tile
// instance keeps its register allocation: the combined one spills 27 scalar registers and
// ran M = 8192 gate_up 1.2 % slower).
// WR = 4: tall 512 x 128 tiles (the four waves side by side along the rows, each still
// 128 rows x 128 tokens; half the activation-tile loads per step), half-width 512 x 64,
// no split-K items (their sum assumes 2 x 2 waves).
template <bool kHalf, bool kAcc, int WR = 2>
__global__ __launch_bounds__(kI8Threads) void gemm_w4_i8_kernel(
    const int8_t *__restrict__ x, const uint8_t *__restrict__ w, int32_t *__restrict__ c, int M,
    int N, int ldc, int K, int L, int accumulate, int n1, int sps, i32x4 *__restrict__ part,
    int nsplit) {
    constexpr bool half = kHalf;
    // the table first: its larger alignment puts it at LDS address 0, so a table address is
    // just the byte field.  A half-width item uses the first half of each tile buffer.
    __shared__ __attribute__((aligned(1024))) uint8_t lut[kI8LutBytes];
    __shared__ __attribute__((aligned(16))) uint8_t xs0[kI8TileBytes];
    __shared__ __attribute__((aligned(16))) uint8_t xs1[kI8TileBytes];
    // Epilogue staging, one region per wave, in the tile buffers (waves 0-2 in the first,
    // wave 3 in the second): past an item's last barrier the tiles are dead, and each item
    // starts with a barrier, so no wave's next tile loads overwrite a region another wave
    // is still using.  The static LDS is then the table and the two tiles only, below the
    // bound for global -> LDS load targets wherever the compiler places them.
    static_assert(3 * kI8StageWave <= kI8TileBytes && kI8StageWave <= kI8TileBytes,
                  "the epilogue staging must fit the tile buffers");
    // (+ 1024: the most alignment padding any placement of the three objects can add)
    static_assert(kI8LutBytes + 2 * kI8TileBytes + 1024 <= kLdsDmaLimit,
                  "LDS-load targets past 128 KiB");
    auto tile = [&](auto bufc) -> uint8_t * {
        if constexpr (decltype(bufc)::value == 0) return xs0;
        else return xs1;
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    static_assert(WR == 2 || WR == 4, "waves 2 x 2, or 4 along the rows");
    if constexpr (WR == 4) nsplit = 0;
    constexpr int WT = 4 / WR;           // waves along the tokens
    constexpr int kRowsT = 128 * WR;     // weight rows per tile
    constexpr int kTokT = 128 * WT;      // tokens per whole tile
    const int wn = WR == 4 ? wave : wave & 1;
    const int wm = WR == 4 ? 0 : wave >> 1;

    const int tiles_m = (M + kTokT - 1) / kTokT;
    const int tiles_mh = (M + kTokT / 2 - 1) / (kTokT / 2);   // half-width tiles
    const int tn1 = (n1 + kRowsT - 1) / kRowsT;
    const int tn2 = (N - n1 + kRowsT - 1) / kRowsT;
    const int full_items = tn1 * tiles_m;
    const int tiles2 = tn2 * tiles_m;
    const int rem_items = half ? tn2 * tiles_mh : (nsplit > 0 ? tiles2 * nsplit : 0);
    const int head = rem_items / 2;
    const int total = full_items + rem_items;
    const int all_steps = (L + 1) / 2;
    i8_lut_fill(lut, tid, kI8Threads);  // published by the first item's barrier

    // One item: 128 WR weight rows (nwg..) x 32 CB WT tokens (m0..) over k-steps
    // [s_begin, s_end); wave (wn, wm) owns 128 rows x 32 CB tokens.  CB = 4: whole or
    // split-K tiles; CB = 2: half-width tiles.
    auto run_item = [&](auto cbc, int nwg, int m0, int s_begin, int s_end, bool split, int sp,
                        int tt) {
        constexpr int CB = decltype(cbc)::value;          // 32-token blocks per wave
        // tile loads per workgroup (28, 14, 7) and per wave (7; 4, the last wave 2; 2, the
        // last wave 1)
        constexpr int kTL = 32 * CB * WT * kI8RowSlots / 64;
        constexpr int LPW = (kTL + 3) / 4;
        constexpr int NCH = 3 * CB;                        // chunks of four MFMAs per step
        constexpr int NFC = CB == 4 ? 8 : 4;               // chunks that issue table reads
        constexpr int kWLoads = 4;                         // loads of fetch_w: one per row block
        // all but the newest fetch_w: the tile loads issued before it have landed
        constexpr int kWaitW = waitcnt_vm<kWLoads>();
        // every wave is past the previous item's epilogue (staged in the tile buffers)
        // before this item's tile loads
        __syncthreads();
        constexpr int FR = 8 / NFC;                        // ... for FR x 2 row blocks each
        // The lane index passes through an empty asm once per item (its derived offsets are
        // recomputed per item, not kept live across the epilogue).
        int lane = tid & 63;
        asm volatile("" : "+v"(lane));
        const int r = lane & 31;
        const int h = lane >> 5;

        // weights: rows past N read zeros; a limb past L (odd L, last step) reads the next
        // row's first limb or zeros -- finite trits that meet zero activations
        const __amdgpu_buffer_rsrc_t wsrc = i8_rsrc(w + static_cast<int64_t>(nwg) * L * kTrytes,
                                                    static_cast<int64_t>(N - nwg) * L * kTrytes);
        uint32_t woff[4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
            woff[rb] = (static_cast<uint32_t>(128 * wn + 32 * rb + r) * static_cast<uint32_t>(L) +
                        static_cast<uint32_t>(h)) * kTrytes;
        auto fetch_w = [&](int step, u32x4 (&dst)[4]) {
            const uint32_t koff = static_cast<uint32_t>(step) * (2 * kTrytes);
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
                dst[rb] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(wsrc, woff[rb] + koff, 0, 0));
        };

        // activation tile: load i of wave w fills slots q = 64 (LPW w + i) + lane, tile row
        // q / 7, slot q % 7; tokens past M read zeros (buffer based at token m0)
        const __amdgpu_buffer_rsrc_t xsrc = i8_rsrc(x + static_cast<int64_t>(m0) * K,
                                                    static_cast<int64_t>(M - m0) * K);
        uint32_t tbase[LPW];
        uint32_t tslot[(LPW + 3) / 4];
#pragma unroll
        for (int i = 0; i < (LPW + 3) / 4; ++i) tslot[i] = 0u;
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const uint32_t qq = static_cast<uint32_t>(64 * (LPW * wave + i) + lane);
            const uint32_t row = qq / kI8RowSlots;
            const uint32_t slot = qq - row * kI8RowSlots;
            tbase[i] = slot < kI8RowSlots - 1 ? row * static_cast<uint32_t>(K) + 16 * slot : kI8Oob;
            tslot[i / 4] |= (16 * slot) << (8 * (i % 4));
        }
        // The last wave's spare loads of a half-width or tall tile (LDS bytes 14336..16383 or
        // 7168..8191, inside the buffer and never read) load zeros through an out-of-range
        // offset, not a branch.
        auto load_tile_part = [&](int step, auto bufc, int i) {
            const bool spare = LPW * 4 != kTL && i >= kTL - 3 * LPW && LPW * wave + i >= kTL;
            const int k0 = step * kI8StepK;
            const uint32_t lim = k0 < K && !spare ? static_cast<uint32_t>(K - k0) : 0u;
            const uint32_t slot16 = (tslot[i / 4] >> (8 * (i % 4))) & 0xFFu;
            const uint32_t off = slot16 < lim ? tbase[i] + static_cast<uint32_t>(k0) : kI8Oob;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xsrc,
                (__attribute__((address_space(3))) void *)(
                    &tile(bufc)[16 * 64 * (LPW * wave + i)]),
                16, off, 0, 0, 0);
        };
        auto load_tile = [&](int step, auto bufc) {
#pragma unroll
            for (int i = 0; i < LPW; ++i) load_tile_part(step, bufc, i);
        };

        // decode: the pair-table entries of weight dword `wd` (trytes 0-1, then 2-3)
        auto table_fetch = [&](uint32_t wd, uint32_t (&t)[4]) {
            const uint2 e0 = *reinterpret_cast<const uint2 *>(lut + ((wd << 3) & 0xF8F8u));
            const uint2 e1 = *reinterpret_cast<const uint2 *>(lut + ((wd >> 13) & 0xF8F8u));
            t[0] = e0.x;
            t[1] = e0.y;
            t[2] = e1.x;
            t[3] = e1.y;
        };
        // the twelve trits of those entries (six bytes each) as three dwords, natural order
        auto table_merge = [&](const uint32_t (&t)[4], uint32_t *out) {
            out[0] = t[0];
            out[1] = __builtin_amdgcn_perm(t[2], t[1], 0x05040100u);
            out[2] = __builtin_amdgcn_alignbit(t[3], t[2], 16);
        };

        i32x16 acc[4][CB];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < CB; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

        // B fragment g of a step: J = g / CB, token block cb = g % CB.  B lane (c, h): token
        // 32 CB wm + 32 cb + c of the tile, bytes 48 h + 16 J of the step.
        const int brow = (32 * CB * wm + r) * kI8RowBytes + 48 * h;
        auto read_b = [&](auto bufc, int g) -> i32x4 {
            const int j = g / CB;
            const int cb = g % CB;
            return *reinterpret_cast<const i32x4 *>(
                &tile(bufc)[brow + 32 * cb * kI8RowBytes + 16 * j]);
        };

        // Weights run three steps ahead: wcur holds step s, wnxt step s + 1, wn2 step s + 2
        // (loaded during step s - 1), and step s + 3 is loaded into wn3 during step s.
        u32x4 wcur[4], wnxt[4], wn2[4], wn3[4];
        i32x4 a[2][4][3];   // operands of the step with parity P / of the other one
        // merge the table words of weight dword dw of row block rb into operand dwords
        // 3 dw .. 3 dw + 2 (operand d / 4, component d % 4)
        auto merge_into = [&](const uint32_t (&t)[4], i32x4 (&ops)[4][3], int rb, int dw) {
            uint32_t o[3];
            table_merge(t, o);
#pragma unroll
            for (int e = 0; e < 3; ++e) {
                const int d = 3 * dw + e;
                ops[rb][d / 4][d % 4] = static_cast<int>(o[e]);
            }
        };
        // chunk gf < NFC reads the table words of weight dword fdw(gf) of row blocks
        // frb(gf, e), e < FR: the first half of those chunks dwords 2 and 3 of this step
        // (the rest of its J = 1 and J = 2 operands), the second half dwords 0 and 1 of the
        // next step (its J = 0 operands and the start of its J = 1)
        auto fdw = [&](int gf) {
            if constexpr (CB == 4) return gf < 4 ? 2 + gf / 2 : (gf - 4) / 2;
            else return gf < 2 ? 2 + gf : gf - 2;
        };
        auto frb = [&](int gf, int e) {
            if constexpr (CB == 4) return 2 * (gf % 2) + e;
            else return e;
        };

        if (s_begin < s_end) {
            fetch_w(s_begin, wcur);
            fetch_w(s_begin + 1, wnxt);
            load_tile(s_begin, B0());
        }
        fetch_w(s_begin + 2, wn2);            // stays in flight across the barrier
        __builtin_amdgcn_s_waitcnt(kWaitW);   // the tile has landed before the barrier
        __syncthreads();
        if (s_begin < s_end) {
            // the first step's J = 0 operands and dwords 4, 5 of its J = 1 operands
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int dw = 0; dw < 2; ++dw) {
                    uint32_t t[4];
                    table_fetch(wcur[rb][dw], t);
                    merge_into(t, a[0], rb, dw);
                }
        }

        // One k-step as NCH chunks of four MFMAs (chunk g: J = g / CB, token block cb =
        // g % CB, row blocks 0..3), one B fragment each, read two chunks ahead; chunks
        // g < NFC issue table reads (above), merged in the next chunk.  The first LPW chunks
        // issue the next step's tile loads, chunk LPW the weights of step + 3: issued after
        // the tile loads, they stay in flight across the step's wait (vmcnt(4)), so they
        // have two steps to land (M = 8192 gate_up 929 -> 916 us, M = 2048 down 136.2 ->
        // 134.5 us).  Past the last step the loads read zeros or unused weight bytes.
        auto step_body = [&](int step, auto bufc, auto otherc) {
            constexpr int P = decltype(bufc)::value;
            i32x4 bq[3];
            bq[0] = read_b(bufc, 0);
            bq[1] = read_b(bufc, 1);
            uint32_t t[2][2 * FR][4];
#pragma unroll
            for (int g = 0; g < NCH; ++g) {
                if (g + 2 < NCH) bq[(g + 2) % 3] = read_b(bufc, g + 2);
                if (g < LPW) load_tile_part(step + 1, otherc, g);
                if (g == LPW) fetch_w(step + 3, wn3);
                if (g >= 1 && g <= NFC) {   // merge the reads of chunk g - 1
                    const int gp = g - 1;
#pragma unroll
                    for (int e = 0; e < 2 * FR; ++e) {
                        if (gp < NFC / 2) merge_into(t[gp & 1][e], a[P], frb(gp, e), fdw(gp));
                        else merge_into(t[gp & 1][e], a[P ^ 1], frb(gp, e), fdw(gp));
                    }
                }
                if (g < NFC) {
#pragma unroll
                    for (int e = 0; e < 2 * FR; ++e)
                        table_fetch((g < NFC / 2 ? wcur : wnxt)[frb(g, e)][fdw(g)], t[g & 1][e]);
                }
#pragma unroll
                for (int rb = 0; rb < 4; ++rb)
                    acc[rb][g % CB] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                        a[P][rb][g / CB], bq[g % 3], acc[rb][g % CB], 0, 0, 0);
                // each MFMA followed by a few of the chunk's other instructions (three LDS
                // reads, four VALU / SALU, one buffer load), as in the bf16 kernel: issue is
                // in order with one wave per SIMD (M = 2048 gate_up 278 -> 270 us with the
                // one-tryte table; with the pair table two reads and three VALU measured the
                // same or up to 2 % slower)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);   // LDS read
                    __builtin_amdgcn_sched_group_barrier(0x006, 4, 0);   // VALU, SALU
                    __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);   // buffer load
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                wcur[rb] = wnxt[rb];
                wnxt[rb] = wn2[rb];
                wn2[rb] = wn3[rb];
            }
            // this step's tile loads (and everything older) have landed; the weights of
            // step + 3, issued after them, stay in flight
            __builtin_amdgcn_s_waitcnt(kWaitW);
            __syncthreads();
        };
        int step = s_begin;
        for (; step + 1 < s_end; step += 2) {
            step_body(step, B0(), B1());
            step_body(step + 1, B1(), B0());
        }
        if (step < s_end)  // odd step count: the last step, peeled
            step_body(step, B0(), B1());

        if constexpr (CB == 4) {
            if (split) {
                i32x4 *dst =
                    part + (((static_cast<int64_t>(sp) * tiles2 + tt) * 4 + wave) * 64) * 64 + lane;
#pragma unroll
                for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                        for (int a4 = 0; a4 < 4; ++a4)
                            dst[((rb * 4 + cb) * 4 + a4) * 64] =
                                i32x4{acc[rb][cb][4 * a4], acc[rb][cb][4 * a4 + 1],
                                      acc[rb][cb][4 * a4 + 2], acc[rb][cb][4 * a4 + 3]};
                return;
            }
        }

        // epilogue through the wave's LDS region, as in the bf16 kernel
        const int col0 = nwg;
        const bool vec4 = ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(c) & 15u) == 0;
        int32_t *st = reinterpret_cast<int32_t *>(wave < 3 ? xs0 + wave * kI8StageWave : xs1);
        const int tq = lane >> 4;
        const int tc = 4 * (lane & 15);
        // Accumulating (the kAcc instance): each pass's C values are loaded one pass ahead,
        // as in the bf16 kernel, so only the first pass waits for them.
        constexpr int kPasses = CB * 2;
        auto c_pass = [&](int p, i32x4 (&cv)[8]) {
            const int cb = p / 2;
            const int rp = p % 2;
            const int nb = col0 + 128 * wn + 64 * rp + tc;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int m = m0 + 32 * CB * wm + 32 * cb + 4 * i + tq;
                const bool ok = vec4 && m < M && nb + 3 < N;
                // non-temporal, as the bf16 kernel's C reads (gate_up M = 2048 with C
                // accumulated: 283.0 -> 270.9 us)
                i32x4 t = {0, 0, 0, 0};
                if (ok)
                    t = __builtin_nontemporal_load(
                        reinterpret_cast<const i32x4 *>(c + static_cast<int64_t>(m) * ldc + nb));
                cv[i] = t;
            }
        };
        i32x4 cva[8], cvb[8];
        if constexpr (kAcc) c_pass(0, cva);
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
            for (int rp = 0; rp < 2; ++rp) {
                const int pass = 2 * cb + rp;
                i32x4 (&cvc)[8] = pass % 2 == 0 ? cva : cvb;
                i32x4 (&cvn)[8] = pass % 2 == 0 ? cvb : cva;
                if constexpr (kAcc)
                    if (pass + 1 < kPasses) c_pass(pass + 1, cvn);
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int a4 = 0; a4 < 4; ++a4)
                        *reinterpret_cast<i32x4 *>(&st[r * kI8StageStride + 32 * j + 8 * a4 + 4 * h]) =
                            i32x4{acc[2 * rp + j][cb][4 * a4], acc[2 * rp + j][cb][4 * a4 + 1],
                                  acc[2 * rp + j][cb][4 * a4 + 2], acc[2 * rp + j][cb][4 * a4 + 3]};
                const int nb = col0 + 128 * wn + 64 * rp + tc;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int tok = 4 * i + tq;
                    const i32x4 v = *reinterpret_cast<const i32x4 *>(&st[tok * kI8StageStride + tc]);
                    const int m = m0 + 32 * CB * wm + 32 * cb + tok;
                    if (m >= M) continue;
                    int32_t *cr = c + static_cast<int64_t>(m) * ldc;
                    int32_t y[4] = {v[0], v[1], v[2], v[3]};
                    if (vec4 && nb + 3 < N) {
                        if constexpr (kAcc) {
                            const i32x4 cv = cvc[i];
                            y[0] += cv[0];
                            y[1] += cv[1];
                            y[2] += cv[2];
                            y[3] += cv[3];
                        }
                        // non-temporal, as the bf16 kernel's C (M = 2048 gate_up 296 -> 275 us)
                        __builtin_nontemporal_store(i32x4{y[0], y[1], y[2], y[3]},
                                                    reinterpret_cast<i32x4 *>(cr + nb));
                    } else {
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            const int n = nb + b;
                            if (n < N) cr[n] = kAcc ? y[b] + cr[n] : y[b];
                        }
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    for (int q = static_cast<int>(blockIdx.x); q < total; q += static_cast<int>(gridDim.x)) {
        const bool rem = q < head || q >= head + full_items;
        const int item =
            __builtin_amdgcn_readfirstlane(q < head ? q : (rem ? q - full_items : q - head));
        if constexpr (kHalf) {
            if (rem) {
                const int tn = __builtin_amdgcn_readfirstlane(item % tn2);
                const int tm = __builtin_amdgcn_readfirstlane(item / tn2);
                run_item(std::integral_constant<int, 2>(), n1 + tn * kRowsT,
                         tm * (kTokT / 2), 0, all_steps, false, 0, 0);
                continue;
            }
        }
        {
            const bool split = rem;
            const int sp = split ? item / tiles2 : 0;
            const int tt = split ? item - sp * tiles2 : item;
            const int tiles_n = split ? tn2 : tn1;
            const int tn = __builtin_amdgcn_readfirstlane(tt % tiles_n);
            const int tm = __builtin_amdgcn_readfirstlane(tt / tiles_n);
            const int s_begin = split ? sp * sps : 0;
            const int s_end = split && s_begin + sps < all_steps ? s_begin + sps : all_steps;
            run_item(std::integral_constant<int, 4>(), (split ? n1 : 0) + tn * kRowsT,
                     tm * kTokT, s_begin, s_end, split, sp, tt);
        }
    }  // work items
}

constexpr int kI8ReducePitch = 132;

// C from the int32 split partials: workgroup (tile, wave, token block cb) sums that block's
// 1024 slots over the splits in split order, stages 32 tokens x 128 rows in LDS and writes
// them as runs of C rows (adding C when accumulating).
__global__ __launch_bounds__(256) void gemm_split_reduce_i8_kernel(
    const i32x4 *__restrict__ part, int32_t *__restrict__ c, int64_t M, int64_t N, int64_t ldc,
    int tiles, int nsplit, int accumulate) {
    __shared__ __attribute__((aligned(16))) int32_t st[32 * kI8ReducePitch];
    const int tt = static_cast<int>(blockIdx.x >> 4);
    const int wave = static_cast<int>((blockIdx.x >> 2) & 3);
    const int cb = static_cast<int>(blockIdx.x & 3);
    const int wn = wave & 1, wm = wave >> 1;
    const int tiles_n = static_cast<int>((N + kI8Rows - 1) / kI8Rows);
    const int64_t m0 = static_cast<int64_t>(tt / tiles_n) * kI8Tokens + 128 * wm + 32 * cb;
    if (m0 >= M) return;
    const int64_t per_split = static_cast<int64_t>(tiles) * 4 * 64 * 64;
    const i32x4 *src = part + (static_cast<int64_t>(tt) * 4 + wave) * 4096;
    for (int i = threadIdx.x; i < 1024; i += 256) {
        const int lane = i & 63, a4 = (i >> 6) & 3, rb = i >> 8;
        const int slot = ((rb * 4 + cb) * 4 + a4) * 64 + lane;
        i32x4 v = src[slot];
        for (int s = 1; s < nsplit; ++s) v += src[s * per_split + slot];
        const int r = lane & 31, h = lane >> 5;
        *reinterpret_cast<i32x4 *>(&st[r * kI8ReducePitch + 32 * rb + 8 * a4 + 4 * h]) = v;
    }
    __syncthreads();
    const int64_t n0 = static_cast<int64_t>(tt % tiles_n) * kI8Rows + 128 * wn;
    // whole 16-byte quads as one vector store (and load, when accumulating)
    const bool vec4 = ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(c) & 15u) == 0;
    for (int i = threadIdx.x; i < 32 * 32; i += 256) {
        const int tok = i >> 5, c4 = i & 31;
        const int64_t m = m0 + tok;
        if (m >= M) continue;
        i32x4 v = *reinterpret_cast<const i32x4 *>(&st[tok * kI8ReducePitch + 4 * c4]);
        int32_t *cr = c + m * ldc;
        const int64_t nb = n0 + 4 * c4;
        if (vec4 && nb + 3 < N) {
            if (accumulate) v += *reinterpret_cast<const i32x4 *>(cr + nb);
            *reinterpret_cast<i32x4 *>(cr + nb) = v;
        } else {
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int64_t n = nb + b;
                if (n < N) cr[n] = accumulate ? v[b] + cr[n] : v[b];
            }
        }
    }
}

// Weight rows run as whole rounds of 256 x 256 tiles (the bf16 kernel's rule).
int64_t i8_rows_whole_rounds(int64_t m, int64_t n) {
    const int64_t tiles_m = (m + kI8Tokens - 1) / kI8Tokens;
    const int64_t tiles_big = ((n + kI8Rows - 1) / kI8Rows) * tiles_m;
    if (tiles_big < 160) return 0;
    const int64_t cus = cu_count();
    const int64_t rem = tiles_big % cus;
    const int64_t n1 = (tiles_big - rem) / tiles_m * kI8Rows;
    if (tiles_big > cus && rem != 0 && 2 * rem <= cus && n1 > 0 && n1 < n) return n1;
    return n;
}

struct I8Plan {
    int64_t n1;                       // rows [0, n1) as whole tiles
    int64_t nsplit, sps, tiles;       // rows [n1, n): split-K items (nsplit > 1)
    bool half;                        // ... or one round of half-width tiles
};

// Rows past whole rounds run as half-width tiles when those fill one round of the CUs
// (three quarters of them or more; the bf16 kernel's rule): no workspace, no second launch.
bool i8_use_half(int64_t m, int64_t n, int64_t n1) {
    const int64_t t =
        ((n - n1 + kI8Rows - 1) / kI8Rows) * ((m + kI8Tokens / 2 - 1) / (kI8Tokens / 2));
    const int64_t cus = cu_count();
    return n1 > 0 && n1 < n && t <= cus && 4 * t >= 3 * cus;
}

// About one workgroup per CU for the rows that do not fill whole rounds, at least four
// k-steps per split.
I8Plan i8_plan(int64_t m, int64_t n, int64_t k) {
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t nsteps = (L + 1) / 2;
    I8Plan p{i8_rows_whole_rounds(m, n), 1, nsteps, 0, false};
    if (p.n1 == n) return p;
    if (i8_use_half(m, n, p.n1)) {
        p.half = true;
        return p;
    }
    p.tiles = ((n - p.n1 + kI8Rows - 1) / kI8Rows) * ((m + kI8Tokens - 1) / kI8Tokens);
    int64_t ns = (cu_count() + p.tiles / 2) / p.tiles;
    if (ns > nsteps / 4) ns = nsteps / 4;
    if (ns < 2) {
        ns = 1;
    } else {
        p.sps = (nsteps + ns - 1) / ns;
        ns = (nsteps + p.sps - 1) / p.sps;
    }
    p.nsplit = ns;
    return p;
}

}  // namespace

// Whether the integer big-tile kernel takes this shape: more than 64 tokens, K a multiple
// of 16 (whole 16-byte activation chunks), 16-byte aligned activations, 32-bit buffer
// offsets and int indices.
bool gemm_i8_fits(const void *x, int64_t m, int64_t n, int64_t k) {
    const int64_t L = (k + kTrits - 1) / kTrits;
    return m > 64 && k > 0 && k % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
           int64_t(kI8Rows) * L * kTrytes < 0x7FFFFFFF && int64_t(kI8Tokens) * k < 0x7FFFFFFF &&
           m < (int64_t(1) << 30) && n < (int64_t(1) << 30) &&
           ((m + kI8Tokens - 1) / kI8Tokens) * ((n + kI8Rows - 1) / kI8Rows) < (int64_t(1) << 26);
}

int64_t gemm_i8_workspace_bytes(int64_t m, int64_t n, int64_t k) {
    const I8Plan p = i8_plan(m, n, k);
    return p.nsplit > 1 ? p.nsplit * p.tiles * kI8Rows * kI8Tokens * 4 : 0;
}

// Rows [0, n1) as whole tiles and the rest as one round of half-width tiles, or as split-K
// items over ws when it is large enough (else rows [n1, n) run as whole tiles too), in the
// same launch.
hipError_t launch_gemm_i8(const void *x, const uint8_t *w, int32_t *c, int64_t m, int64_t n,
                          int64_t k, bool accumulate, hipStream_t s, void *ws, int64_t ws_bytes) {
    const int64_t L = (k + kTrits - 1) / kTrits;
    const int64_t cus = cu_count();
    // Tall tiles (gemm_tall_plan) up to K = 8192: gate_up M = 2048 249.7 -> 242.7 us, M =
    // 8192 946.7 -> 923.6 us, qkv M = 8192 208.2 -> 204.8 us; down (K = 14336) at M = 8192
    // measured 453.2 -> 457.4 us and keeps the 256 x 256 tiles.
    int64_t tn1 = 0;
    bool thalf = false;
    if (k <= 8192 && gemm_tall_plan(m, n, k, &tn1, &thalf)) {
        const int64_t items = ((tn1 + 511) / 512) * ((m + 127) / 128) +
                              (thalf ? ((n - tn1 + 511) / 512) * ((m + 63) / 64) : 0);
        const dim3 grid(static_cast<unsigned>(items < cus ? items : cus));
        auto kernel = thalf ? (accumulate ? gemm_w4_i8_kernel<true, true, 4>
                                          : gemm_w4_i8_kernel<true, false, 4>)
                            : (accumulate ? gemm_w4_i8_kernel<false, true, 4>
                                          : gemm_w4_i8_kernel<false, false, 4>);
        kernel<<<grid, dim3(kI8Threads), 0, s>>>(
            static_cast<const int8_t *>(x), w, c, static_cast<int>(m), static_cast<int>(n),
            static_cast<int>(n), static_cast<int>(k), static_cast<int>(L), accumulate ? 1 : 0,
            static_cast<int>(tn1), 0, nullptr, 0);
        return hipGetLastError();
    }
    I8Plan p = i8_plan(m, n, k);
    const bool split = !p.half && p.nsplit > 1 && ws != nullptr &&
                       ws_bytes >= p.nsplit * p.tiles * kI8Rows * kI8Tokens * 4;
    if (!split && !p.half) p.n1 = n;
    const int64_t tiles_m = (m + kI8Tokens - 1) / kI8Tokens;
    const int64_t half_items =
        p.half ? ((n - p.n1 + kI8Rows - 1) / kI8Rows) * ((m + kI8Tokens / 2 - 1) / (kI8Tokens / 2))
               : 0;
    const int64_t items = ((p.n1 + kI8Rows - 1) / kI8Rows) * tiles_m +
                          (split ? p.nsplit * p.tiles : 0) + half_items;
    if (items <= 0) return hipSuccess;
    const dim3 grid(static_cast<unsigned>(items < cus ? items : cus));
    // (split items store raw partials; the split sum adds C)
    if (p.half) {
        auto kernel = accumulate ? gemm_w4_i8_kernel<true, true> : gemm_w4_i8_kernel<true, false>;
        kernel<<<grid, dim3(kI8Threads), 0, s>>>(
            static_cast<const int8_t *>(x), w, c, static_cast<int>(m), static_cast<int>(n),
            static_cast<int>(n), static_cast<int>(k), static_cast<int>(L), accumulate ? 1 : 0,
            static_cast<int>(p.n1), 0, nullptr, 0);
    } else {
        auto kernel = accumulate ? gemm_w4_i8_kernel<false, true> : gemm_w4_i8_kernel<false, false>;
        kernel<<<grid, dim3(kI8Threads), 0, s>>>(
            static_cast<const int8_t *>(x), w, c, static_cast<int>(m), static_cast<int>(n),
            static_cast<int>(n), static_cast<int>(k), static_cast<int>(L), accumulate ? 1 : 0,
            static_cast<int>(p.n1), split ? static_cast<int>(p.sps) : 0, static_cast<i32x4 *>(ws),
            split ? static_cast<int>(p.nsplit) : 0);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !split) return e;
    gemm_split_reduce_i8_kernel<<<dim3(static_cast<unsigned>(p.tiles * 16)), dim3(256), 0, s>>>(
        static_cast<const i32x4 *>(ws), c + p.n1, m, n - p.n1, n, static_cast<int>(p.tiles),
        static_cast<int>(p.nsplit), accumulate ? 1 : 0);
    return hipGetLastError();
}

}  // namespace t81hip

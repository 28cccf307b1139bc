/*
 * oracle/t81_gguf_oracle.c -- CPU restatement of t81lib's GGUF ternary block codecs
 * (TQ1_0, TQ2_0) and of a matmul over TQ2_0 weights.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT.  Linked into liboracle.so next to
 * t81_oracle.c; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg load it.
 *
 * The formats are llama.cpp's ggml block_tq1_0 / block_tq2_0 (256 weights per
 * block; ggml types 34 and 35), which the reference writes and reads with numpy
 * in t81/gguf.py.  Each function restates those numpy lines with the same float32
 * arithmetic (numpy evaluates `blocks * inv_d` etc. in float32; a Python float
 * operand adopts the array's float32 type).  How each is pinned (closed forms,
 * brute force over all digit patterns, numpy's own float16 conversion, the
 * reference tests' round-trip cases) is listed in tests/test_gguf_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define QK 256 /* GGUF_QUANT_BLOCK_ROWS, t81/gguf.py:53 */

/* float32 -> IEEE binary16 bits, round to nearest even, overflow to inf, NaN kept
 * (numpy's float32.astype(np.float16), used for the block scale at
 * t81/gguf.py:544 and :615). */
uint16_t orc_f32_to_f16_bits(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu)); /* NaN */
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520: inf */
    if (ax < 0x38800000u) {
        /* subnormal half (or zero): value = m * 2^-24, m = round(|f| * 2^24) */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to 0 */
        const uint32_t e = ax >> 23;
        const uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e; /* 14 .. 24 */
        uint32_t m = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (m & 1u))) ++m;
        return (uint16_t)(sign | m);
    }
    /* normal: rebias the exponent, round the 13 dropped mantissa bits to even */
    uint32_t h = ((ax >> 13) - (112u << 10));
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

float orc_f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m * 2^-24 */
            float v = (float)m * 5.9604644775390625e-8f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7F800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* _quantize_trits (t81/gguf.py:518-522): with a threshold, |v| >= thr -> sign(v)
 * else 0 (NaN -> 0); without one (thr <= 0), round half away from zero
 * (where(v >= 0, floor(v + 0.5), ceil(v - 0.5)), float32) clipped to [-1, 1].
 * numpy turns a NaN there into an undefined int8; here it is 0. */
static int8_t tq_trit(float v, int use_thr, float thr) {
    if (use_thr) {
        if (!(fabsf(v) >= thr)) return 0;
        return v > 0.0f ? 1 : (v < 0.0f ? -1 : 0);
    }
    if (isnan(v)) return 0;
    float r = v >= 0.0f ? floorf(v + 0.5f) : ceilf(v - 0.5f);
    if (r > 1.0f) r = 1.0f;
    if (r < -1.0f) r = -1.0f;
    return (int8_t)r;
}

/* Block scale and digits q = trit + 1 of one block (t81/gguf.py:526-530, 602-606):
 * d = max|v| (NaN if any value is NaN, as np.max), inv_d = 0 if d == 0 else 1/d,
 * trits of v * inv_d.  Returns d. */
static float tq_block_digits(const float *v, int use_thr, float thr, uint8_t *q) {
    float d = 0.0f;
    int nan = 0;
    for (int j = 0; j < QK; ++j) {
        const float a = fabsf(v[j]);
        if (isnan(a)) nan = 1;
        else if (a > d) d = a;
    }
    if (nan) d = NAN;
    const float inv_d = d == 0.0f ? 0.0f : 1.0f / d;
    for (int j = 0; j < QK; ++j) q[j] = (uint8_t)(tq_trit(v[j] * inv_d, use_thr, thr) + 1);
    return d;
}

/* TQ2_0 block (66 bytes), t81/gguf.py:601-615: qs[a*32 + c] holds the digits of
 * elements a*128 + s*32 + c at bits 2s (a < 2, s < 4, c < 32); then the scale as
 * little-endian float16. */
static void tq2_pack(const uint8_t *q, float d, uint8_t *out) {
    for (int a = 0; a < 2; ++a)
        for (int c = 0; c < 32; ++c) {
            uint8_t b = 0;
            for (int s = 0; s < 4; ++s) b |= (uint8_t)(q[a * 128 + s * 32 + c] << (2 * s));
            out[a * 32 + c] = b;
        }
    const uint16_t h = orc_f32_to_f16_bits(d);
    out[64] = (uint8_t)(h & 0xFF);
    out[65] = (uint8_t)(h >> 8);
}

/* TQ1_0 block (54 bytes), t81/gguf.py:525-545: base-3 numbers of 5 digits (first
 * digit weighted 81) over elements i*32 + c (bytes 0..31) and 160 + i*16 + c
 * (bytes 32..47), of 4 digits weighted 81, 27, 9, 3 over 240 + i*4 + c (bytes
 * 48..51); each number v < 243 is stored as (v * 256 + 242) / 243, then the
 * float16 scale. */
static void tq1_pack(const uint8_t *q, float d, uint8_t *out) {
    static const unsigned w5[5] = {81, 27, 9, 3, 1};
    static const unsigned w4[4] = {81, 27, 9, 3};
    unsigned v[52];
    for (int c = 0; c < 32; ++c) {
        v[c] = 0;
        for (int i = 0; i < 5; ++i) v[c] += q[i * 32 + c] * w5[i];
    }
    for (int c = 0; c < 16; ++c) {
        v[32 + c] = 0;
        for (int i = 0; i < 5; ++i) v[32 + c] += q[160 + i * 16 + c] * w5[i];
    }
    for (int c = 0; c < 4; ++c) {
        v[48 + c] = 0;
        for (int i = 0; i < 4; ++i) v[48 + c] += q[240 + i * 4 + c] * w4[i];
    }
    for (int k = 0; k < 52; ++k) out[k] = (uint8_t)((v[k] * 256u + 242u) / 243u);
    const uint16_t h = orc_f32_to_f16_bits(d);
    out[52] = (uint8_t)(h & 0xFF);
    out[53] = (uint8_t)(h >> 8);
}

int orc_tq_block_bytes(int quant) { return quant == 34 ? 54 : (quant == 35 ? 66 : -1); }

/* _quantize_tensor (t81/gguf.py:665-690): rows of `cols` float32 values, each
 * zero-padded to whole blocks; threshold clipped to [0, 1], a threshold of 0
 * selecting the rounding form.  quant: 34 = TQ1_0, 35 = TQ2_0.  Returns 0, or -1
 * for an unknown quant. */
int orc_tq_quantize(const float *src, int64_t rows, int64_t cols, float threshold, int quant,
                    uint8_t *dst) {
    const int bb = orc_tq_block_bytes(quant);
    if (bb < 0) return -1;
    float thr = threshold < 0.0f ? 0.0f : (threshold > 1.0f ? 1.0f : threshold);
    if (isnan(threshold)) thr = threshold; /* np.clip keeps NaN; NaN > 0 is false */
    const int use_thr = thr > 0.0f;
    const int64_t nb = (cols + QK - 1) / QK;
    float blk[QK];
    uint8_t q[QK];
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            for (int j = 0; j < QK; ++j) {
                const int64_t col = b * QK + j;
                blk[j] = col < cols ? src[r * cols + col] : 0.0f;
            }
            const float d = tq_block_digits(blk, use_thr, thr, q);
            uint8_t *out = dst + (r * nb + b) * bb;
            if (quant == 35) tq2_pack(q, d, out);
            else tq1_pack(q, d, out);
        }
    return 0;
}

/* One block back to 256 float32 values d * (digit - 1) (t81/gguf.py:618-663):
 * TQ2_0 digit of element a*128 + s*32 + c = (qs[a*32 + c] >> 2s) & 3; TQ1_0 digit n
 * of a stored byte = ((uint8)(byte * 3^n) * 3) >> 8 (uint8 product wraps), element
 * n*32 + c / 160 + n*16 + c / 240 + n*4 + c. */
static void tq_block_values(const uint8_t *blk, int quant, float *out) {
    if (quant == 35) {
        const float d = orc_f16_bits_to_f32((uint16_t)(blk[64] | (blk[65] << 8)));
        for (int a = 0; a < 2; ++a)
            for (int s = 0; s < 4; ++s)
                for (int c = 0; c < 32; ++c) {
                    const int q = (blk[a * 32 + c] >> (2 * s)) & 3;
                    out[a * 128 + s * 32 + c] = d * (float)(int8_t)(q - 1);
                }
        return;
    }
    static const uint8_t pow3[5] = {1, 3, 9, 27, 81};
    const float d = orc_f16_bits_to_f32((uint16_t)(blk[52] | (blk[53] << 8)));
    for (int n = 0; n < 5; ++n) {
        for (int c = 0; c < 32; ++c) {
            const uint8_t q = (uint8_t)(blk[c] * pow3[n]);
            out[n * 32 + c] = d * (float)((int8_t)(((uint16_t)q * 3) >> 8) - 1);
        }
        for (int c = 0; c < 16; ++c) {
            const uint8_t q = (uint8_t)(blk[32 + c] * pow3[n]);
            out[160 + n * 16 + c] = d * (float)((int8_t)(((uint16_t)q * 3) >> 8) - 1);
        }
    }
    for (int n = 0; n < 4; ++n)
        for (int c = 0; c < 4; ++c) {
            const uint8_t q = (uint8_t)(blk[48 + c] * pow3[n]);
            out[240 + n * 4 + c] = d * (float)((int8_t)(((uint16_t)q * 3) >> 8) - 1);
        }
}

/* _decode_quant_tensor (t81/gguf.py:1020-1069): rows x cols float32, each row the
 * first `cols` values of its decoded blocks. */
int orc_tq_dequantize(const uint8_t *src, int64_t rows, int64_t cols, int quant, float *dst) {
    const int bb = orc_tq_block_bytes(quant);
    if (bb < 0) return -1;
    const int64_t nb = (cols + QK - 1) / QK;
    float vals[QK];
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            tq_block_values(src + (r * nb + b) * bb, quant, vals);
            for (int j = 0; j < QK; ++j) {
                const int64_t col = b * QK + j;
                if (col < cols) dst[r * cols + col] = vals[j];
            }
        }
    return 0;
}

/* y[m, n] = sum_k x[m, k] * W[n, k] over the dequantized TQ2_0 weights, in fp64;
 * abs_out (if not NULL) gets sum_k |x[m, k] * W[n, k]|, the scale of the
 * floating-point tolerance. */
void orc_tq2_matmul_f64(const double *x, int64_t M, int64_t K, const uint8_t *w, int64_t N,
                        double *out, double *abs_out) {
    const int64_t nb = (K + QK - 1) / QK;
    float vals[QK];
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t m = 0; m < M; ++m) {
            out[m * N + n] = 0.0;
            if (abs_out) abs_out[m * N + n] = 0.0;
        }
        for (int64_t b = 0; b < nb; ++b) {
            tq_block_values(w + (n * nb + b) * 66, 35, vals);
            for (int j = 0; j < QK; ++j) {
                const int64_t k = b * QK + j;
                if (k >= K) break;
                for (int64_t m = 0; m < M; ++m) {
                    const double p = x[m * K + k] * (double)vals[j];
                    out[m * N + n] += p;
                    if (abs_out) abs_out[m * N + n] += fabs(p);
                }
            }
        }
    }
}

/* ---- t81::core::gguf row codec (src/t81/core/gguf_quants.h): 8 trits per 13-bit
 * block stored as uint16, one float scale per row, and the tensor framing of the
 * dequant_tq1_0 / dequant_tq2_0 bindings (python/bindings.cpp:561-638).  Pinned
 * against the compiled header (oracle/_ref) in tests/test_gguf_oracle.py. ---- */

/* compute_scale (gguf_quants.h:55-64): the largest |v| that compares greater than the
 * running maximum, starting from 0; NaN never does. */
float orc_tq1r_scale(const float *v, int64_t n) {
    float m = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        const float a = fabsf(v[i]);
        if (a > m) m = a;
    }
    return m;
}

/* quantize_trit (:23-32) after clamp_threshold (:19-21, std::clamp keeps NaN): fmin /
 * fmax take the non-NaN operand, so a NaN value clamps to +1. */
static int tq1r_trit(float v, float thr) {
    const float c = isnan(v) ? 1.0f : (v > 1.0f ? 1.0f : (v < -1.0f ? -1.0f : v));
    if (c >= thr) return 1;
    if (c <= -thr) return -1;
    return 0;
}

static float tq1r_clamp_threshold(float t) {
    return t < 0.0f ? 0.0f : (0.9999f < t ? 0.9999f : t);
}

/* quantize_row_tq1_0 (:116-144): scale = supplied if > 0 else compute_scale; each block of
 * 8 values becomes digits d_i = {+1: 0, 0: 1, -1: 2} of trit(v * (1 / scale)) (trit 0
 * past the row or when scale <= 0), stored as sum_i d_i 3^i (digit 0 least
 * significant).  Returns the scale used. */
float orc_tq1r_quantize_row(const float *v, int64_t n, float threshold, float supplied,
                            uint16_t *dst) {
    if (n <= 0 || dst == NULL) return 0.0f;
    const float scale = supplied > 0.0f ? supplied : orc_tq1r_scale(v, n);
    const float thr = tq1r_clamp_threshold(threshold);
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    const int64_t blocks = (n + 7) / 8;
    for (int64_t b = 0; b < blocks; ++b) {
        unsigned word = 0;
        for (int i = 7; i >= 0; --i) {
            const int64_t k = b * 8 + i;
            int t = 0;
            if (k < n && scale > 0.0f) t = tq1r_trit(v[k] * inv, thr);
            word = word * 3u + (unsigned)(t > 0 ? 0 : (t < 0 ? 2 : 1));
        }
        dst[b] = (uint16_t)(word & 0x1FFFu);
    }
    return scale;
}

/* dequantize_row_tq1_0 (:146-168): scale == 0 gives zeros; else value = trit * scale with
 * the low 8 base-3 digits of each word (digit 0 -> +1, 2 -> -1, else 0). */
void orc_tq1r_dequantize_row(const uint16_t *src, int64_t n, float scale, float *dst) {
    if (n <= 0 || dst == NULL || src == NULL) return;
    if (scale == 0.0f) {
        for (int64_t i = 0; i < n; ++i) dst[i] = 0.0f;
        return;
    }
    for (int64_t i = 0; i < n; ++i) {
        unsigned w = src[i / 8];
        for (int64_t d = 0; d < i % 8; ++d) w /= 3u;
        const unsigned digit = w % 3u;
        const float t = digit == 0 ? 1.0f : (digit == 2 ? -1.0f : 0.0f);
        dst[i] = t * scale;
    }
}

/* dequant_tensor_tq1_impl (python/bindings.cpp:561-638): groups of max(1, block_rows)
 * rows, each a little-endian float16 scale, 8 skipped bytes when `refinements`, then
 * each row's ceil(cols / 8) uint16 words.  Returns 0, or the first check that fails as
 * the binding meets it: 1 "buffer truncated while reading scale", 2 "... while skipping
 * refinement bytes", 3 "... while reading quantized rows"; -1 negative rows / cols.
 * Rows decoded before the failure are left in dst. */
int orc_tq1r_dequant_tensor(const uint8_t *buf, int64_t nbytes, int64_t rows, int64_t cols,
                            int64_t block_rows, int refinements, float *dst) {
    if (rows < 0 || cols < 0) return -1;
    const int64_t words = (cols + 7) / 8;
    const int64_t row_bytes = words * 2;
    const int64_t group = block_rows > 1 ? block_rows : 1;
    int64_t off = 0;
    int64_t r = 0;
    uint16_t row[4096];
    while (r < rows) {
        if (off + 2 > nbytes) return 1;
        const uint16_t h = (uint16_t)(buf[off] | (buf[off + 1] << 8));
        off += 2;
        if (refinements) {
            if (off + 8 > nbytes) return 2;
            off += 8;
        }
        const float scale = orc_f16_bits_to_f32(h);
        const int64_t in_group = group < rows - r ? group : rows - r;
        for (int64_t g = 0; g < in_group; ++g) {
            if (off + row_bytes > nbytes) return 3;
            for (int64_t w0 = 0; w0 < words; w0 += 4096) {
                const int64_t cnt = words - w0 < 4096 ? words - w0 : 4096;
                for (int64_t i = 0; i < cnt; ++i)
                    row[i] = (uint16_t)(buf[off + 2 * (w0 + i)] | (buf[off + 2 * (w0 + i) + 1] << 8));
                const int64_t c0 = w0 * 8;
                const int64_t nc = cols - c0 < cnt * 8 ? cols - c0 : cnt * 8;
                orc_tq1r_dequantize_row(row, nc, scale, dst + r * cols + c0);
            }
            off += row_bytes;
            ++r;
        }
    }
    return 0;
}

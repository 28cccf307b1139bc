/*
 * include/t81_hip.h -- C ABI of libt81_hip.so, the MI355X (gfx950) backend of
 * t81lib's packed-ternary GEMM path.
 *
 * Plain C: pointers, sizes and an opaque stream handle (a hipStream_t, or NULL
 * for the null stream).  No function throws.  Every entry point validates its
 * arguments on the host, enqueues its kernels on `stream` and returns without
 * synchronising; results are ordered with later work on the same stream.
 * Device pointers must come from the same device that is current on the
 * calling thread.  Returns T81_HIP_OK or a negative T81_HIP_E* code; the text
 * of the last error on the calling thread is t81_hip_last_error().
 *
 * Packed-limb layout (the reference's, include/t81/core/limb.hpp:145-181 and
 * docs/t81lib-spec-v0.1.0.md:179-234): a limb is 16 bytes holding 48 trits,
 * byte j = 13 + t[3j] + 3*t[3j+1] + 9*t[3j+2] (values 0..26).  A packed
 * matrix of `rows` x `cols` trits is rows x L x 16 bytes, L = ceil(cols/48),
 * row-major; trits past `cols` are 0 (byte 13 for a fully padded triple).
 */
#ifndef T81_HIP_H
#define T81_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* return codes */
#define T81_HIP_OK 0
#define T81_HIP_EINVAL_SHAPE (-1)     /* negative or inconsistent dimensions      */
#define T81_HIP_EINVAL_K48 (-2)       /* K not a multiple of 48 (limb GEMM)       */
#define T81_HIP_EINVAL_THRESHOLD (-3) /* threshold outside (0, 1] (C++ form)      */
#define T81_HIP_EINVAL_DTYPE (-4)     /* unsupported dtype / alpha-beta combo     */
#define T81_HIP_EINVAL_POINTER (-5)   /* NULL where data is required              */
#define T81_HIP_EHIP (-6)             /* HIP runtime error (text in last_error)   */
#define T81_HIP_ENODEV (-7)           /* no gfx950 device                         */
#define T81_HIP_EINVAL_INDEX (-8)     /* sparse entry index out of range          */

/* element types of activations / float inputs */
#define T81_DTYPE_F32 0
#define T81_DTYPE_BF16 1
#define T81_DTYPE_I8 2
#define T81_DTYPE_F16 3

/* threshold forms of the quantizer */
#define T81_THR_CPP 0   /* python/bindings.cpp:405-414: >=thr -> +1 else <=-thr -> -1; */
                        /* thr must lie in (0, 1] (bindings.cpp:419-421, 463-465)      */
#define T81_THR_TORCH 1 /* t81/torch/__init__.py:44-50: thr clamped to [0, 0.9999] by */
                        /* the caller (in double, then float32); -1 wins on ties       */

/* 1 if a gfx950 device is present and usable, else 0.  Never fails.
 * Replaces: t81::linalg::detail::rocm_available(), include/t81/linalg/gemm_gpu.hpp:70-72. */
int t81_hip_available(void);

/* Text of the last error returned on the calling thread ("" if none). */
const char *t81_hip_last_error(void);

/* K1 -- threshold-quantize a rows x cols float matrix (row-major, dtype
 * T81_DTYPE_F32/BF16/F16) and pack it row-wise into out (rows x L x 16 bytes).
 * Bit-exact with the reference packer.
 * Replaces: pack_dense_matrix, python/bindings.cpp:460-517 (thr_mode T81_THR_CPP);
 *           TernaryTensor.from_float / _quantize_tensor + _pack_rowwise,
 *           t81/torch/__init__.py:214-231, 44-50, 68-80 (thr_mode T81_THR_TORCH). */
int t81_hip_quantize_pack(const void *w, int w_dtype, uint8_t *out, int64_t rows, int64_t cols,
                          float threshold, int thr_mode, void *stream);

/* Elementwise quantize of `count` floats to int8 trits.
 * Replaces: quantize_to_trits, python/bindings.cpp:416-445. */
int t81_hip_quantize(const void *src, int dtype, int8_t *out, int64_t count, float threshold,
                     int thr_mode, void *stream);

/* Column-wise pack of activations: x is tokens x K (row-major), out is
 * L x tokens x 16 bytes holding limb l of column n of x^T at (l*tokens+n)*16.
 * Replaces: TernaryTensor._pack_rhs_for_gemm / _pack_columnwise,
 *           t81/torch/__init__.py:257-262, 83-97. */
int t81_hip_pack_cols(const void *x, int x_dtype, uint8_t *out, int64_t tokens, int64_t k,
                      float threshold, int thr_mode, void *stream);

/* Unpack rows x limbs_per_row x 16 bytes into a rows x cols int8 trit matrix
 * (cols <= 48 * limbs_per_row).  Bytes > 26 decode to unspecified trits; call
 * t81_hip_validate_packed first where the input is untrusted.
 * Replaces: unpack_packed_limbs, python/bindings.cpp:640-686, and
 *           _limbs_to_trits, t81/torch/__init__.py:100-112. */
int t81_hip_unpack(const uint8_t *packed, int8_t *out, int64_t rows, int64_t limbs_per_row,
                   int64_t cols, void *stream);

/* Counts bytes > 26 in `count` packed bytes; *bad_count (device int32) is
 * overwritten.  Mirrors the check of limb::from_bytes, limb.hpp:160-168. */
int t81_hip_validate_packed(const uint8_t *packed, int64_t count, int32_t *bad_count,
                            void *stream);

/* K2/K3 -- ternary matmul, dot-product semantics over the packed weights:
 *     C[m, n] = alpha * sum_{k<K} X[m, k] * T[n, k] + beta * C[m, n] + bias[n]
 * X is M x K row-major (x_dtype F32 or BF16; C is float32 M x N) or I8 (C is
 * int32 M x N, exact; requires alpha == 1, beta in {0, 1}, bias == NULL,
 * K <= 131071).  W is N x L x 16 packed bytes.  beta == 0 does not read C.
 * bias may be NULL.  M <= 16 runs the decode GEMV kernel (K2), larger M the
 * prefill GEMM kernel (K3).
 * Replaces: the hot path of TernaryTensor.matmul_input / t8.nn.Linear
 *           (t81/torch/__init__.py:241-246, t81/nn/linear.py:53-70) with the
 *           trit-dot reading of gemm_ternary (t81/torch/__init__.py:291-304). */
int t81_hip_ternary_matmul(const void *x, int x_dtype, const uint8_t *w, void *c, int64_t m,
                           int64_t n, int64_t k, float alpha, float beta, const float *bias,
                           void *stream);

/* Same, forcing the kernel: which = 2 (K2 GEMV, M <= 16) or 3 (K3 GEMM). */
int t81_hip_ternary_matmul_kernel(int which, const void *x, int x_dtype, const uint8_t *w,
                                  void *c, int64_t m, int64_t n, int64_t k, float alpha,
                                  float beta, const float *bias, void *stream);

/* Same, with a caller-owned device workspace: which = 0 (by M, as
 * t81_hip_ternary_matmul), 2 or 3.  When K3 has few output tiles for its shape, or K2
 * runs 9..16 tokens over a long K with float32 activations, int8 ones with K not a
 * multiple of 16, or bf16 ones with K not a multiple of 8, and workspace_bytes is at least
 * t81_hip_ternary_matmul_workspace_size(...), K is split over several workgroups
 * per tile: each writes its partial tile to the workspace and a second kernel sums
 * the partials in split order (deterministic).  With float32 activations past 64 tokens
 * (K % 8 == 0) the workspace may instead hold the activations' bf16 hi and lo planes,
 * chunk by chunk, and each chunk runs as two bf16 launches (the second adding the lo
 * plane's product to C).  NULL / 0 bytes: no split, no planes.  The workspace must be
 * 16-byte aligned and not used by another call at the same time.
 * Replaces: the same reference interfaces as t81_hip_ternary_matmul; the
 *           reference's CPU path needs no workspace, so it has no such argument. */
int t81_hip_ternary_matmul_ws(int which, const void *x, int x_dtype, const uint8_t *w, void *c,
                              int64_t m, int64_t n, int64_t k, float alpha, float beta,
                              const float *bias, void *workspace, int64_t workspace_bytes,
                              void *stream);

/* Bytes of workspace t81_hip_ternary_matmul_ws uses for this shape on the current
 * device (0: the shape does not split).  Never fails.  It does not look at x's
 * alignment: int8 activations at 5+ tokens with K % 16 == 0 report 0, and such a call
 * runs in one launch with no split whether or not x is 16-byte aligned (bf16 likewise at
 * the column-block kernel's 17..48 tokens, where an unaligned x runs K3 unsplit).  For
 * M <= 16 it is K2's workspace: K3 forced there (which = 3) runs unsplit. */
int64_t t81_hip_ternary_matmul_workspace_size(int64_t m, int64_t n, int64_t k, int x_dtype);

/* Same as t81_hip_ternary_matmul_ws(which, ...) given a workspace of exactly
 * t81_hip_ternary_matmul_workspace_size(m, n, k, x_dtype) bytes -- identical kernels,
 * split plan and results, bit for bit -- but allocating nothing: the workspace is a
 * static 64 MiB device array in the library, one copy per device, reserved when the
 * library's code object is loaded on that device and held until the process ends.
 * Shapes whose workspace needs more than 64 MiB are rejected (T81_HIP_EINVAL_SHAPE, nothing
 * launched).  Every call on a device shares that array: calls that may overlap on one
 * device (other streams or threads) race and must be serialised by the caller.
 * No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops that forbid hipMalloc). */
int t81_hip_ternary_matmul_noalloc(int which, const void *x, int x_dtype, const uint8_t *w,
                                   void *c, int64_t m, int64_t n, int64_t k, float alpha,
                                   float beta, const float *bias, void *stream);

/* K4 -- the reference's literal gemm_ternary: A (M x K/48 limbs), B (K/48 x N
 * limbs), C (M x N float32, read and written):
 *     C[i,j] = float( C[i,j]*beta + sum_l alpha * V(A[i,l]) * V(B[l,j]) )
 * with V the limb's balanced-ternary integer value, each product formed
 * exactly and converted as low + high * 3^48 through the reference's tryte
 * tables, accumulated in double with l ascending (no FMA contraction).
 * Bit-exact with src/linalg/gemm_cpu.cpp:8-71 (including +-inf outputs).
 * Replaces: t81::linalg::detail::rocm_gemm_ternary, gemm_gpu.hpp:131-140 and
 *           src/linalg/gemm_rocm.cpp:335-396 (device pointers instead of spans). */
int t81_hip_gemm_ternary_limb(const uint8_t *a, const uint8_t *b, float *c, int m, int n, int k,
                              float alpha, float beta, void *stream);

/* Elementwise float32 ops of the backend contract, over n contiguous elements,
 * bit-exact with the reference's CPU loops (each multiply and add rounded
 * separately; a NaN condition counts as nonzero; a NaN clamp input passes
 * through).  In-place use (out equal to an input) is allowed.
 *   where:   out[i] = cond[i] != 0 ? x[i] : y[i]
 *   clamp:   out[i] = in[i] < lo ? lo : (in[i] > hi ? hi : in[i])
 *   lerp:    out[i] = start[i] + weight[i] * (end[i] - start[i])
 *   addcmul: out[i] = in[i] + value * t1[i] * t2[i]
 * Replace: t81::linalg::detail::rocm_where / rocm_clamp / rocm_lerp /
 *          rocm_addcmul, include/t81/linalg/gemm_gpu.hpp:80-85, 233-249, with the
 *          semantics of cpu_where / cpu_clamp / cpu_lerp / cpu_addcmul,
 *          src/linalg/gemm_dispatch.cpp:145-211. */
int t81_hip_where(const float *cond, const float *x, const float *y, float *out, int64_t n,
                  void *stream);
int t81_hip_clamp(const float *in, float *out, int64_t n, float lo, float hi, void *stream);
int t81_hip_lerp(const float *start, const float *end, const float *weight, float *out,
                 int64_t n, void *stream);
int t81_hip_addcmul(const float *in, const float *t1, const float *t2, float value, float *out,
                    int64_t n, void *stream);

/* The reference's literal matmul_input in one kernel: the activations x (tokens x k,
 * T81_DTYPE_F32 / BF16 / F16, row-major) are quantized with the torch form of the
 * threshold (already clamped to [0, 0.9999], T81_THR_TORCH rules) and packed
 * column-wise inside the limb GEMM, then
 *   c[i, j] = float(double(c[i, j]) * beta + sum_l product(w[i, l], xpacked[l, j]) * alpha)
 * for c (rows x tokens) -- bit-identical to t81_hip_pack_cols + t81_hip_gemm_ternary_limb.
 * w: rows x ceil(k / 48) x 16, 16-byte aligned.
 * Replaces: TernaryTensor.matmul_input -> _pack_rhs_for_gemm -> _compute_gemm,
 *           t81/torch/__init__.py:241-276 (quantize 0.5, _pack_columnwise :83-97,
 *           then gemm_ternary, src/linalg/gemm_cpu.cpp:8-71). */
int t81_hip_matmul_input_reference(const uint8_t *w, const void *x, int x_dtype, float *c,
                                   int64_t rows, int64_t tokens, int64_t k, float threshold,
                                   float alpha, float beta, void *stream);

/* The transposed trit matrix in the same layout: in is rows x ceil(cols / 48) x 16
 * (row r = T[r, 0 .. cols)), out is cols x ceil(rows / 48) x 16 (row k = T[0 .. rows, k],
 * trits past rows zero).  Both 16-byte aligned.  With it the backward of
 * y = x T^T, dx = dy T, is t81_hip_ternary_matmul(dy, out) with K = rows.
 * Replaces: the float unpack + matmul of _TernaryGemmFunction.backward,
 *           t81/torch/__init__.py:291-304 (_limbs_to_trits, :100-112). */
int t81_hip_transpose_packed(const uint8_t *packed, uint8_t *out, int64_t rows, int64_t cols,
                             void *stream);

/* ---- GGUF ternary block formats (llama.cpp ggml block_tq1_0 / block_tq2_0) ----
 * 256 weights per block; a row of `cols` weights is ceil(cols / 256) blocks.
 *   T81_TQ1_0 (ggml type 34, 54 bytes): base-3 digits packed 5 (and 4) per byte as
 *             (v * 256 + 242) / 243, then an IEEE half scale.
 *   T81_TQ2_0 (ggml type 35, 66 bytes): 2-bit digits, byte a*32 + c holding elements
 *             a*128 + s*32 + c at bits 2s, then an IEEE half scale.
 * Weight = scale * (digit - 1). */
#define T81_TQ1_0 34
#define T81_TQ2_0 35

/* Bytes per 256-weight block of `quant` (54, 66), or T81_HIP_EINVAL_DTYPE. */
int t81_hip_tq_block_bytes(int quant);

/* Quantize rows x cols float32 (row-major) into rows x ceil(cols / 256) blocks.
 * threshold is clipped to [0, 1]; > 0 selects |v / d| >= threshold -> sign(v),
 * 0 rounds v / d half away from zero (d = max |v| of the block, stored as half).
 * Replaces: _quantize_tensor + _quantize_blocks_tq1 / _quantize_blocks_tq2,
 *           t81/gguf.py:665-690, 525-545, 601-615 (trits: _quantize_trits, :518-522). */
int t81_hip_tq_quantize(const float *src, uint8_t *dst, int64_t rows, int64_t cols,
                        float threshold, int quant, void *stream);

/* Decode rows x ceil(cols / 256) blocks into rows x cols float32.
 * Replaces: _decode_quant_tensor + _dequantize_blocks_tq1 / _dequantize_blocks_tq2,
 *           t81/gguf.py:1020-1069, 618-635, 654-662. */
int t81_hip_tq_dequantize(const uint8_t *src, float *dst, int64_t rows, int64_t cols, int quant,
                          void *stream);

/* c[m, n] = alpha * sum_k x[m, k] * W[n, k] + beta * c[m, n] + bias[n] with W given as
 * n rows of TQ2_0 blocks (K = k weights per row), read directly (no dequantized copy).
 * x: T81_DTYPE_BF16 / F32 / I8 (int8 values exact; the result is float32 since the
 * block scales are).  w must be 4-byte aligned.
 * Replaces: the dequantize-then-multiply a consumer of t81.gguf.read_gguf performs
 *           (t81/gguf.py:1072-1121 reads, F.linear multiplies); no reference kernel. */
int t81_hip_tq2_matmul(const void *x, int x_dtype, const uint8_t *w, float *c, int64_t m,
                       int64_t n, int64_t k, float alpha, float beta, const float *bias,
                       void *stream);

/* ---- the reference's own TQ1_0 row codec (src/t81/core/gguf_quants.h:14-168) ----
 * A row of n values is ceil(n / 8) uint16 words; word w holds trits 8w .. 8w + 7 as
 * base-3 digits d = {+1: 0, 0: 1, -1: 2}, trit 8w + i weighted 3^i (pad trits 0), and
 * the row has one float scale.  This is not the llama.cpp block format above. */
#define T81_TQ1_TRITS_PER_BLOCK 8 /* gguf_quants.h:14 */
#define T81_TQ1_BLOCK_ROWS 32     /* gguf_quants.h:15: rows per scale in a tensor payload */

/* rows x cols float32 (row-major) -> rows x ceil(cols / 8) words (row-major).  Row r uses
 * scale s = scales_in[r] when scales_in is given and scales_in[r] > 0, else max |v| over
 * the row (NaN values skipped); trit of v * (1 / s) with the value clamped to [-1, 1] (NaN
 * to +1) against threshold clamped to [0, 0.9999]; all trits 0 when s <= 0.  The scale
 * used goes to scales_out[r] when scales_out is given.  values 4-byte, dst 2-byte aligned.
 * Replaces: quantize_row_tq1_0 + compute_scale, gguf_quants.h:55-64, 116-144, one call
 *           per row, as the quantize_row_tq1_0 binding makes it (python/bindings.cpp:519-540). */
int t81_hip_tq1_quantize_rows(const float *values, int64_t rows, int64_t cols, float threshold,
                              const float *scales_in, float *scales_out, uint16_t *dst,
                              void *stream);

/* rows x ceil(cols / 8) words -> rows x cols float32: trit * scales[r] (zeros when
 * scales[r] == 0); only the low 8 base-3 digits of a word are read.
 * Replaces: dequantize_row_tq1_0, gguf_quants.h:146-168 (binding dequant_row_tq1_0,
 *           python/bindings.cpp:542-559). */
int t81_hip_tq1_dequantize_rows(const uint16_t *src, int64_t rows, int64_t cols,
                                const float *scales, float *dst, void *stream);

/* Tensor payload: groups of max(1, block_rows) rows, each a little-endian IEEE half scale,
 * 8 reserved bytes when refinements != 0 (the TQ2_0 variant), then the group's rows of
 * words (2 * ceil(cols / 8) bytes each).  Any alignment.  Size of a whole payload: */
int64_t t81_hip_tq1_payload_bytes(int64_t rows, int64_t cols, int64_t block_rows,
                                  int refinements);

/* Writes such a payload (t81_hip_tq1_payload_bytes bytes): per group h = half(max |v|)
 * (round to nearest even), zero reserved bytes, each row quantized as
 * t81_hip_tq1_quantize_rows with scales_in = float(h).
 * No reference counterpart: the reference reads these payloads but has no writer. */
int t81_hip_tq1_quantize_payload(const float *values, int64_t rows, int64_t cols,
                                 int64_t block_rows, int refinements, float threshold,
                                 uint8_t *payload, void *stream);

/* payload (payload_bytes bytes) -> rows x cols float32.  A payload shorter than the layout
 * returns T81_HIP_EINVAL_SHAPE with the binding's message for the first check its
 * sequential walk fails: "buffer truncated while reading scale", "... while skipping
 * refinement bytes" or "... while reading quantized rows".
 * Replaces: dequant_tensor_tq1_impl behind dequant_tq1_0 (refinements 0) and dequant_tq2_0
 *           (refinements 1), python/bindings.cpp:561-638, 975-995. */
int t81_hip_tq1_dequantize_payload(const uint8_t *payload, int64_t payload_bytes, int64_t rows,
                                   int64_t cols, int64_t block_rows, int refinements, float *dst,
                                   void *stream);

/* Sparse ternary x dense (COO entries, list order significant):
 *     C[r, :] = beta == 0 ? 0 : float(double(C[r, :]) * beta), then for each entry e in
 *     list order: C[row_e, k] = float(double(C[row_e, k]) + double(value_e) * alpha *
 *     double(B[col_e, k])), each multiply and add rounded in double, for k < N.
 * B is cols x N, C rows x N, float32 row-major; values are the entries' integers (the
 * reference's limbs built from long long).  Bit-exact with the reference.
 * Replaces: t81::sparse::spmm_simple, include/t81/sparse/simple.hpp:37-94, as the
 *           spmm_simple binding calls it, python/bindings.cpp:888-940. */
typedef struct t81_hip_spmm_plan t81_hip_spmm_plan;

/* Builds the device form of the matrix (entries stably sorted by row, values as double).
 * Allocates device memory and synchronises `stream` (it reads the index check back).
 * values / row_idx / col_idx: nnz device elements, nnz <= 2^31 - 1.  On an index
 * outside [0, rows) x [0, cols) returns T81_HIP_EINVAL_INDEX ("Row index out of bounds"
 * or "Column index out of bounds", the reference's messages, simple.hpp:79-84) with
 * *first_bad = the first such entry and *plan still built from the entries before it:
 * applying that plan leaves C as the reference leaves it when it throws.  Otherwise
 * *first_bad = -1.  Every plan returned must be destroyed. */
int t81_hip_spmm_plan_create(const int64_t *values, const int32_t *row_idx,
                             const int32_t *col_idx, int64_t nnz, int rows, int cols,
                             t81_hip_spmm_plan **plan, int64_t *first_bad, void *stream);

/* C = the product above with the plan's entries; B (cols x N) and C (rows x N) device,
 * 4-byte aligned.  Enqueues one kernel, no allocation, no synchronisation. */
int t81_hip_spmm_plan_apply(const t81_hip_spmm_plan *plan, const float *B, float *C, int N,
                            float alpha, float beta, void *stream);

/* rows / cols / stored entries of a plan (any pointer may be NULL). */
int t81_hip_spmm_plan_info(const t81_hip_spmm_plan *plan, int *rows, int *cols, int64_t *nnz);

/* Frees the plan's device memory (after the work that uses it has completed). */
void t81_hip_spmm_plan_destroy(t81_hip_spmm_plan *plan);

/* create + apply + destroy in one call, synchronising `stream`: the binding's
 * spmm_simple on device buffers, including the partial update of C on a bad index. */
int t81_hip_spmm_simple(const int64_t *values, const int32_t *row_idx, const int32_t *col_idx,
                        int64_t nnz, int rows, int cols, const float *B, float *C, int N,
                        float alpha, float beta, void *stream);

/* Host-only test hook, no device needed: writes the 16 x 27 tryte-contribution
 * table K4 uses (constant-evaluated like build_tryte_contributions,
 * include/t81/linalg/gemm.hpp:28-41), so it can be compared bit for bit. */
void t81_hip_limb_tryte_table(double *out);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* T81_HIP_H */

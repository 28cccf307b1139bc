// t81lib_amd/csrc/t81_kernels.hpp -- host-side launchers of the gfx950 kernels.
// Shapes and pointers are validated by the C ABI (abi.hip) before any launcher runs;
// launchers only enqueue work on the given stream.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace t81hip {

constexpr int kDtypeF32 = 0;
constexpr int kDtypeBF16 = 1;
constexpr int kDtypeI8 = 2;
constexpr int kDtypeF16 = 3;

// abi.hip: records msg as the calling thread's last error and returns code
int report_error(int code, const char *msg);
// The argument checks of t81_hip_ternary_matmul_ws (0 or the code it would return, with
// its error text recorded).
int check_matmul_args(int which, const void *x, int x_dtype, const uint8_t *w, void *c,
                      int64_t m, int64_t n, int64_t k, float alpha, float beta,
                      const float *bias);

// pack.hip
hipError_t launch_quantize_pack_rows(const void *w, int dtype, uint8_t *out, int64_t rows,
                                     int64_t cols, float thr, int torch_form, hipStream_t s);
hipError_t launch_quantize_pack_cols(const void *x, int dtype, uint8_t *out, int64_t tokens,
                                     int64_t k, float thr, int torch_form, hipStream_t s);
hipError_t launch_quantize(const void *src, int dtype, int8_t *out, int64_t count, float thr,
                           int torch_form, hipStream_t s);
hipError_t launch_unpack(const uint8_t *packed, int8_t *out, int64_t rows, int64_t limbs,
                         int64_t cols, hipStream_t s);
hipError_t launch_validate(const uint8_t *packed, int64_t count, int32_t *bad, hipStream_t s);

// gemv.hip (K2): M <= 16.  ws (ws_bytes of device memory, may be null) lets 9..16 tokens
// over a long K split it over workgroups (float32 activations, int8 with K % 16 != 0,
// bf16 with K % 8 != 0); gemv_workspace_bytes says how much a shape uses.
// 17..gemv_column_blocks_max_tokens(K, dtype) tokens (64 up to K = 8192, else 48; bf16 32
// from K = 12288), bf16 (K % 8 == 0) or int8 (K % 16 == 0) activations at a 16-byte aligned
// x: the column-block stream kernel of gemv.hip (two or three 16-token blocks; 49..64 tokens
// as two launches); the K3 launcher tries it first.
int64_t gemv_column_blocks_max_tokens(int64_t k, int x_dtype);
bool gemv_column_blocks_fits(const void *x, int x_dtype, int64_t m, int64_t n, int64_t k);
hipError_t launch_gemv_column_blocks(bool *handled, const void *x, int x_dtype,
                                     const uint8_t *w, void *c, int m, int64_t n, int64_t k,
                                     float alpha, float beta, const float *bias, hipStream_t s);
hipError_t launch_gemv(const void *x, int x_dtype, const uint8_t *w, void *c, int m, int64_t n,
                       int64_t k, float alpha, float beta, const float *bias, hipStream_t s,
                       void *ws = nullptr, int64_t ws_bytes = 0);
int64_t gemv_workspace_bytes(int64_t m, int64_t n, int64_t k, int x_dtype);

// gemv_strip.hip (K2, M <= 4; bf16 and int8 at 5..8 tokens over >= 12288 rows and K <=
// 4096): sets *handled = false (and launches nothing) when the shape is outside what it
// covers
hipError_t launch_gemv_strip(bool *handled, const void *x, int x_dtype, const uint8_t *w,
                             void *c, int m, int64_t n, int64_t k, float alpha, float beta,
                             const float *bias, hipStream_t s);

// transpose.hip: the packed trit matrix transposed (same limb layout)
hipError_t launch_transpose_packed(const uint8_t *in, uint8_t *out, int64_t rows, int64_t cols,
                                   hipStream_t s);

// spmm.hip: sparse ternary (COO) x dense; plan = entries stably sorted by row
hipError_t launch_spmm_first_bad(const int32_t *row_idx, const int32_t *col_idx, int64_t nnz,
                                 int rows, int cols, unsigned long long *first_bad, hipStream_t s);
size_t spmm_sort_scratch_bytes(int64_t n);
hipError_t launch_spmm_build(const int64_t *values, const int32_t *row_idx, const int32_t *col_idx,
                             int64_t n, int rows, void *scratch, int32_t *row_ptr,
                             int32_t *cols_out, double *vals_out, hipStream_t s);
hipError_t launch_spmm_apply(const int32_t *row_ptr, const int32_t *cols, const double *vals,
                             const float *B, float *C, int rows, int64_t N, float alpha, float beta,
                             hipStream_t s);

// tq.hip: GGUF TQ1_0 (quant 34) / TQ2_0 (quant 35) block codecs
hipError_t launch_tq_quantize(const float *src, uint8_t *dst, int64_t rows, int64_t cols,
                              float thr, int use_thr, int quant, hipStream_t s);
hipError_t launch_tq_dequantize(const uint8_t *src, float *dst, int64_t rows, int64_t cols,
                                int quant, hipStream_t s);

// tq_row.hip: the TQ1_0 row codec (8 trits per uint16 word, a float scale per row) and the
// grouped tensor payload; payload_check returns the binding's first failing check (0 none,
// 1 scale, 2 reserved bytes, 3 rows)
int64_t tq1r_payload_bytes(int64_t rows, int64_t n, int64_t block_rows, bool refinements);
int tq1r_payload_check(int64_t nbytes, int64_t rows, int64_t n, int64_t block_rows,
                       bool refinements);
hipError_t launch_tq1r_quantize_rows(const float *values, int64_t rows, int64_t n, float thr,
                                     const float *scales_in, float *scales_out, uint16_t *dst,
                                     hipStream_t s);
hipError_t launch_tq1r_dequantize_rows(const uint16_t *src, int64_t rows, int64_t n,
                                       const float *scales, float *dst, hipStream_t s);
hipError_t launch_tq1r_dequantize_payload(const uint8_t *payload, int64_t rows, int64_t n,
                                          int64_t block_rows, bool refinements, float *dst,
                                          hipStream_t s);
hipError_t launch_tq1r_quantize_payload(const float *values, int64_t rows, int64_t n,
                                        int64_t block_rows, bool refinements, float thr,
                                        uint8_t *payload, hipStream_t s);

// gemv_tq2.hip: matmul straight from TQ2_0 weights (tokens in groups of four)
bool tq2_matmul_fits(int64_t n, int64_t k);
hipError_t launch_tq2_matmul(const void *x, int x_dtype, const uint8_t *w, float *c, int64_t m,
                             int64_t n, int64_t k, float alpha, float beta, const float *bias,
                             hipStream_t s);

// gemm.hip (K3): any M.  ws (ws_bytes of device memory, may be null) lets shapes with
// few tiles split K; gemm_workspace_bytes says how much such a shape uses (0: none).
hipError_t launch_gemm(const void *x, int x_dtype, const uint8_t *w, void *c, int64_t m,
                       int64_t n, int64_t k, float alpha, float beta, const float *bias,
                       hipStream_t s, void *ws = nullptr, int64_t ws_bytes = 0);
int64_t gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int x_dtype);

// gemm_i8.hip (K3, int8 activations, integer matrix cores): whether a shape takes it, the
// workspace its split-K plan uses, and the launch (C int32; accumulate: C += product)
bool gemm_i8_fits(const void *x, int64_t m, int64_t n, int64_t k);
int64_t gemm_i8_workspace_bytes(int64_t m, int64_t n, int64_t k);
hipError_t launch_gemm_i8(const void *x, const uint8_t *w, int32_t *c, int64_t m, int64_t n,
                          int64_t k, bool accumulate, hipStream_t s, void *ws, int64_t ws_bytes);

// Compute units of the current device (256 on MI355X), cached per device.
int cu_count();

// Whether the big-tile kernels run a shape as tall 512 x 128 tiles (gemm.hip): rows
// [0, *n1) as whole tiles, and with *half the rest as one round of 512 x 64 tiles.
bool gemm_tall_plan(int64_t m, int64_t n, int64_t k, int64_t *n1, bool *half);

// limb.hip (K4)
hipError_t launch_gemm_limb(const uint8_t *a, const uint8_t *b, float *c, int m, int n,
                            int k_limbs, float alpha, float beta, hipStream_t s);
// K4 with the activations quantized (torch form) and column-packed inside the kernel
hipError_t launch_gemm_limb_fused(const uint8_t *a, const void *x, int x_dtype, float *c, int m,
                                  int n, int64_t k, float thr, float alpha, float beta,
                                  hipStream_t s);

// elementwise.hip: the backend contract's where / clamp / lerp / addcmul (float32)
hipError_t launch_where(const float *cond, const float *x, const float *y, float *out, int64_t n,
                        hipStream_t s);
hipError_t launch_clamp(const float *in, float *out, int64_t n, float lo, float hi,
                        hipStream_t s);
hipError_t launch_lerp(const float *start, const float *end, const float *weight, float *out,
                       int64_t n, hipStream_t s);
hipError_t launch_addcmul(const float *in, const float *t1, const float *t2, float value,
                          float *out, int64_t n, hipStream_t s);

}  // namespace t81hip

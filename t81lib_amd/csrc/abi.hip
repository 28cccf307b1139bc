// t81lib_amd/csrc/abi.hip -- the extern "C" boundary of libt81_hip.so (include/t81_hip.h).
//
// Every entry point: validates on the host (the reference's checks and messages,
// cited per function), checks that the current device is a gfx950, enqueues on
// the caller's stream and returns.  No exceptions cross the boundary.  Nothing is
// allocated or synchronised, except by the sparse plan's create / destroy (and the
// one-shot t81_hip_spmm_simple built on them), which own device memory.
#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <new>
#include <string>

#include "../../include/t81_hip.h"
#include "t81_kernels.hpp"

namespace t81hip {
void host_tryte_table(double *out);
}

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char *where) {
    return fail(T81_HIP_EHIP, std::string(where) + ": " + hipGetErrorString(e));
}

constexpr int kMaxDevices = 64;
std::atomic<int> g_arch_state[kMaxDevices];  // 0 unknown, 1 gfx950, -1 other

// Checks the current device once per device id: the kernels are built for gfx950 only.
int require_device(const char *where) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, where);
    if (dev < 0 || dev >= kMaxDevices) return fail(T81_HIP_ENODEV, "device index out of range");
    int state = g_arch_state[dev].load(std::memory_order_relaxed);
    if (state == 0) {
        hipDeviceProp_t prop;
        e = hipGetDeviceProperties(&prop, dev);
        if (e != hipSuccess) return hip_fail(e, where);
        state = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : -1;
        g_arch_state[dev].store(state, std::memory_order_relaxed);
    }
    if (state != 1) return fail(T81_HIP_ENODEV, std::string(where) + ": device is not gfx950");
    return T81_HIP_OK;
}

int finish(hipError_t e, const char *where) {
    if (e != hipSuccess) return hip_fail(e, where);
    g_last_error.clear();
    return T81_HIP_OK;
}

bool float_dtype(int d) { return d == T81_DTYPE_F32 || d == T81_DTYPE_BF16 || d == T81_DTYPE_F16; }

// a * b elements (a, b >= 0) beyond any device buffer (2^40, far above 288 GB of
// elements of any type): rejected before a launch forms the product, which could overflow.
bool too_many(int64_t a, int64_t b) {
    constexpr int64_t kLimit = int64_t{1} << 40;
    return a > kLimit || b > kLimit || (a > 0 && b > kLimit / a);
}

// python/bindings.cpp:419-421 / 463-465 (C++ form); t81/torch/__init__.py:45 (torch form,
// clamped by the caller -- here only range-checked).
int check_threshold(float thr, int mode) {
    if (mode == T81_THR_CPP) {
        if (thr <= 0.0f || thr > 1.0f)
            return fail(T81_HIP_EINVAL_THRESHOLD, "threshold must be between 0 (exclusive) and 1");
        return T81_HIP_OK;
    }
    if (mode == T81_THR_TORCH) {
        if (!(thr >= 0.0f && thr <= 1.0f))
            return fail(T81_HIP_EINVAL_THRESHOLD,
                        "torch-form threshold must already be clamped to [0, 0.9999]");
        return T81_HIP_OK;
    }
    return fail(T81_HIP_EINVAL_THRESHOLD, "unknown threshold mode");
}

int check_matmul(const void *x, int x_dtype, const uint8_t *w, void *c, int64_t m, int64_t n,
                 int64_t k, float alpha, float beta, const float *bias) {
    if (m < 0 || n < 0 || k < 0)
        return fail(T81_HIP_EINVAL_SHAPE, "gemm_ternary dimensions must be non-negative");
    if (m > INT_MAX / 2 || n > (int64_t(1) << 40) || k > (int64_t(1) << 31))
        return fail(T81_HIP_EINVAL_SHAPE, "ternary_matmul dimensions too large");
    if (x_dtype != T81_DTYPE_F32 && x_dtype != T81_DTYPE_BF16 && x_dtype != T81_DTYPE_I8)
        return fail(T81_HIP_EINVAL_DTYPE, "activations must be float32, bfloat16 or int8");
    if (x_dtype == T81_DTYPE_I8) {
        if (alpha != 1.0f || !(beta == 0.0f || beta == 1.0f) || bias != nullptr)
            return fail(T81_HIP_EINVAL_DTYPE,
                        "int8 activations produce exact int32: alpha must be 1, beta 0 or 1, "
                        "no bias");
        if (k > 131071)
            return fail(T81_HIP_EINVAL_SHAPE, "int8 activations require K <= 131071 (exact sums)");
    }
    if ((m > 0 && k > 0 && x == nullptr) || (n > 0 && k > 0 && w == nullptr) ||
        (m > 0 && n > 0 && c == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (reinterpret_cast<uintptr_t>(w) % 16 != 0)
        return fail(T81_HIP_EINVAL_POINTER, "packed weights must be 16-byte aligned");
    const uintptr_t elem = x_dtype == T81_DTYPE_F32 ? 4 : (x_dtype == T81_DTYPE_BF16 ? 2 : 1);
    if (reinterpret_cast<uintptr_t>(x) % elem != 0 || reinterpret_cast<uintptr_t>(c) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(bias) % 4 != 0)
        return fail(T81_HIP_EINVAL_POINTER, "misaligned activation, output or bias pointer");
    return T81_HIP_OK;
}

}  // namespace

int t81hip::report_error(int code, const char *msg) { return fail(code, msg); }

int t81hip::check_matmul_args(int which, const void *x, int x_dtype, const uint8_t *w, void *c,
                              int64_t m, int64_t n, int64_t k, float alpha, float beta,
                              const float *bias) {
    if (int rc = check_matmul(x, x_dtype, w, c, m, n, k, alpha, beta, bias)) return rc;
    if (which == 2 && m > 16) return fail(T81_HIP_EINVAL_SHAPE, "the GEMV kernel takes M <= 16");
    if (which != 0 && which != 2 && which != 3)
        return fail(T81_HIP_EINVAL_SHAPE, "kernel must be 0, 2 or 3");
    return T81_HIP_OK;
}

extern "C" {

int t81_hip_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return 0;
    return require_device("t81_hip_available") == T81_HIP_OK ? 1 : 0;
}

const char *t81_hip_last_error(void) { return g_last_error.c_str(); }

int t81_hip_quantize_pack(const void *w, int w_dtype, uint8_t *out, int64_t rows, int64_t cols,
                          float threshold, int thr_mode, void *stream) {
    if (int rc = check_threshold(threshold, thr_mode)) return rc;
    if (rows < 0 || cols < 0) return fail(T81_HIP_EINVAL_SHAPE, "rows and cols must be non-negative");
    if (too_many(rows, cols)) return fail(T81_HIP_EINVAL_SHAPE, "rows x cols too large");
    if (!float_dtype(w_dtype)) return fail(T81_HIP_EINVAL_DTYPE, "weights must be a float dtype");
    if (rows > 0 && cols > 0 && (w == nullptr || out == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (reinterpret_cast<uintptr_t>(out) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(w) % (w_dtype == T81_DTYPE_F32 ? 4 : 2) != 0)
        return fail(T81_HIP_EINVAL_POINTER, "misaligned input or output pointer");
    if (int rc = require_device("t81_hip_quantize_pack")) return rc;
    return finish(t81hip::launch_quantize_pack_rows(w, w_dtype, out, rows, cols, threshold,
                                                    thr_mode == T81_THR_TORCH,
                                                    static_cast<hipStream_t>(stream)),
                  "t81_hip_quantize_pack");
}

int t81_hip_quantize(const void *src, int dtype, int8_t *out, int64_t count, float threshold,
                     int thr_mode, void *stream) {
    if (int rc = check_threshold(threshold, thr_mode)) return rc;
    if (count < 0) return fail(T81_HIP_EINVAL_SHAPE, "count must be non-negative");
    if (too_many(count, 1)) return fail(T81_HIP_EINVAL_SHAPE, "count too large");
    if (!float_dtype(dtype)) return fail(T81_HIP_EINVAL_DTYPE, "input must be a float dtype");
    if (count > 0 && (src == nullptr || out == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (int rc = require_device("t81_hip_quantize")) return rc;
    return finish(t81hip::launch_quantize(src, dtype, out, count, threshold,
                                          thr_mode == T81_THR_TORCH,
                                          static_cast<hipStream_t>(stream)),
                  "t81_hip_quantize");
}

int t81_hip_pack_cols(const void *x, int x_dtype, uint8_t *out, int64_t tokens, int64_t k,
                      float threshold, int thr_mode, void *stream) {
    if (int rc = check_threshold(threshold, thr_mode)) return rc;
    if (tokens < 0 || k < 0) return fail(T81_HIP_EINVAL_SHAPE, "dimensions must be non-negative");
    if (too_many(tokens, k)) return fail(T81_HIP_EINVAL_SHAPE, "tokens x k too large");
    if (!float_dtype(x_dtype)) return fail(T81_HIP_EINVAL_DTYPE, "input must be a float dtype");
    if (tokens > 0 && k > 0 && (x == nullptr || out == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (reinterpret_cast<uintptr_t>(out) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(x) % (x_dtype == T81_DTYPE_F32 ? 4 : 2) != 0)
        return fail(T81_HIP_EINVAL_POINTER, "misaligned input or output pointer");
    if (int rc = require_device("t81_hip_pack_cols")) return rc;
    return finish(t81hip::launch_quantize_pack_cols(x, x_dtype, out, tokens, k, threshold,
                                                    thr_mode == T81_THR_TORCH,
                                                    static_cast<hipStream_t>(stream)),
                  "t81_hip_pack_cols");
}

// python/bindings.cpp:643-661: non-negative sizes, cols within the packed capacity.
int t81_hip_unpack(const uint8_t *packed, int8_t *out, int64_t rows, int64_t limbs_per_row,
                   int64_t cols, void *stream) {
    if (rows < 0 || cols < 0 || limbs_per_row < 0)
        return fail(T81_HIP_EINVAL_SHAPE, "rows and cols must be non-negative");
    // limbs needed for cols trits, compared without forming limbs_per_row * 48 (overflow)
    if (cols / 48 + (cols % 48 != 0 ? 1 : 0) > limbs_per_row)
        return fail(T81_HIP_EINVAL_SHAPE, "cols exceeds packed trit capacity");
    if (too_many(rows, cols) || too_many(rows, limbs_per_row))
        return fail(T81_HIP_EINVAL_SHAPE, "unpack dimensions too large");
    if (rows > 0 && cols > 0 && (packed == nullptr || out == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (int rc = require_device("t81_hip_unpack")) return rc;
    return finish(t81hip::launch_unpack(packed, out, rows, limbs_per_row, cols,
                                        static_cast<hipStream_t>(stream)),
                  "t81_hip_unpack");
}

int t81_hip_validate_packed(const uint8_t *packed, int64_t count, int32_t *bad_count,
                            void *stream) {
    if (count < 0) return fail(T81_HIP_EINVAL_SHAPE, "count must be non-negative");
    if (too_many(count, 1)) return fail(T81_HIP_EINVAL_SHAPE, "count too large");
    if (bad_count == nullptr || (count > 0 && packed == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (int rc = require_device("t81_hip_validate_packed")) return rc;
    return finish(t81hip::launch_validate(packed, count, bad_count,
                                          static_cast<hipStream_t>(stream)),
                  "t81_hip_validate_packed");
}

int t81_hip_ternary_matmul_ws(int which, const void *x, int x_dtype, const uint8_t *w, void *c,
                              int64_t m, int64_t n, int64_t k, float alpha, float beta,
                              const float *bias, void *workspace, int64_t workspace_bytes,
                              void *stream) {
    if (int rc = check_matmul(x, x_dtype, w, c, m, n, k, alpha, beta, bias)) return rc;
    if (which == 0) which = m <= 16 ? 2 : 3;
    if (which == 2 && m > 16) return fail(T81_HIP_EINVAL_SHAPE, "the GEMV kernel takes M <= 16");
    if (which != 2 && which != 3) return fail(T81_HIP_EINVAL_SHAPE, "kernel must be 0, 2 or 3");
    if (workspace_bytes < 0 || (workspace_bytes > 0 && workspace == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "workspace pointer and size do not match");
    if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
        return fail(T81_HIP_EINVAL_POINTER, "workspace must be 16-byte aligned");
    if (int rc = require_device("t81_hip_ternary_matmul")) return rc;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e;
    if (which == 2)
        e = t81hip::launch_gemv(x, x_dtype, w, c, static_cast<int>(m), n, k, alpha, beta, bias, s,
                                workspace, workspace_bytes);
    else
        e = t81hip::launch_gemm(x, x_dtype, w, c, m, n, k, alpha, beta, bias, s, workspace,
                                workspace_bytes);
    return finish(e, "t81_hip_ternary_matmul");
}

int t81_hip_ternary_matmul_kernel(int which, const void *x, int x_dtype, const uint8_t *w,
                                  void *c, int64_t m, int64_t n, int64_t k, float alpha,
                                  float beta, const float *bias, void *stream) {
    if (which != 2 && which != 3) return fail(T81_HIP_EINVAL_SHAPE, "kernel must be 2 or 3");
    return t81_hip_ternary_matmul_ws(which, x, x_dtype, w, c, m, n, k, alpha, beta, bias, nullptr,
                                     0, stream);
}

int t81_hip_ternary_matmul(const void *x, int x_dtype, const uint8_t *w, void *c, int64_t m,
                           int64_t n, int64_t k, float alpha, float beta, const float *bias,
                           void *stream) {
    return t81_hip_ternary_matmul_ws(0, x, x_dtype, w, c, m, n, k, alpha, beta, bias, nullptr, 0,
                                     stream);
}

int64_t t81_hip_ternary_matmul_workspace_size(int64_t m, int64_t n, int64_t k, int x_dtype) {
    if (m < 0 || n < 0 || k < 0 || m > INT_MAX / 2 || n > (int64_t(1) << 40) ||
        k > (int64_t(1) << 31))
        return 0;
    if (m <= 16) return t81hip::gemv_workspace_bytes(m, n, k, x_dtype);
    return t81hip::gemm_workspace_bytes(m, n, k, x_dtype);
}

// include/t81/linalg/gemm_gpu.hpp:171-190: dimension, K % 48 and (implicitly, through
// the caller's buffers) span checks; M == 0 or N == 0 is a no-op.
int t81_hip_gemm_ternary_limb(const uint8_t *a, const uint8_t *b, float *c, int m, int n, int k,
                              float alpha, float beta, void *stream) {
    if (m < 0 || n < 0 || k < 0)
        return fail(T81_HIP_EINVAL_SHAPE, "gemm_ternary dimensions must be non-negative");
    if (k % 48 != 0) return fail(T81_HIP_EINVAL_K48, "gemm_ternary requires K divisible by 48");
    if (m == 0 || n == 0) {
        g_last_error.clear();
        return T81_HIP_OK;
    }
    if (c == nullptr || (k > 0 && (a == nullptr || b == nullptr)))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (reinterpret_cast<uintptr_t>(a) % 16 != 0 || reinterpret_cast<uintptr_t>(b) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(c) % 4 != 0)
        return fail(T81_HIP_EINVAL_POINTER, "limb buffers must be 16-byte aligned");
    if (int rc = require_device("t81_hip_gemm_ternary_limb")) return rc;
    return finish(t81hip::launch_gemm_limb(a, b, c, m, n, k / 48, alpha, beta,
                                           static_cast<hipStream_t>(stream)),
                  "t81_hip_gemm_ternary_limb");
}

// src/linalg/gemm_dispatch.cpp:145-211: the CPU loops check matching lengths; here the
// caller passes one length, so only n >= 0 and the pointers are checked.
static int check_elementwise(int64_t n, std::initializer_list<const void *> ptrs) {
    if (n < 0) return fail(T81_HIP_EINVAL_SHAPE, "element count must be non-negative");
    if (n > 0)
        for (const void *p : ptrs) {
            if (p == nullptr)
                return fail(T81_HIP_EINVAL_POINTER,
                            "tensor metadata must provide a valid data pointer");
            if (reinterpret_cast<uintptr_t>(p) % 4 != 0)
                return fail(T81_HIP_EINVAL_POINTER, "float32 data must be 4-byte aligned");
        }
    return T81_HIP_OK;
}

int t81_hip_where(const float *cond, const float *x, const float *y, float *out, int64_t n,
                  void *stream) {
    if (int rc = check_elementwise(n, {cond, x, y, out})) return rc;
    if (int rc = require_device("t81_hip_where")) return rc;
    return finish(t81hip::launch_where(cond, x, y, out, n, static_cast<hipStream_t>(stream)),
                  "t81_hip_where");
}

int t81_hip_clamp(const float *in, float *out, int64_t n, float lo, float hi, void *stream) {
    if (int rc = check_elementwise(n, {in, out})) return rc;
    if (int rc = require_device("t81_hip_clamp")) return rc;
    return finish(t81hip::launch_clamp(in, out, n, lo, hi, static_cast<hipStream_t>(stream)),
                  "t81_hip_clamp");
}

int t81_hip_lerp(const float *start, const float *end, const float *weight, float *out,
                 int64_t n, void *stream) {
    if (int rc = check_elementwise(n, {start, end, weight, out})) return rc;
    if (int rc = require_device("t81_hip_lerp")) return rc;
    return finish(
        t81hip::launch_lerp(start, end, weight, out, n, static_cast<hipStream_t>(stream)),
        "t81_hip_lerp");
}

int t81_hip_addcmul(const float *in, const float *t1, const float *t2, float value, float *out,
                    int64_t n, void *stream) {
    if (int rc = check_elementwise(n, {in, t1, t2, out})) return rc;
    if (int rc = require_device("t81_hip_addcmul")) return rc;
    return finish(
        t81hip::launch_addcmul(in, t1, t2, value, out, n, static_cast<hipStream_t>(stream)),
        "t81_hip_addcmul");
}

int t81_hip_matmul_input_reference(const uint8_t *w, const void *x, int x_dtype, float *c,
                                   int64_t rows, int64_t tokens, int64_t k, float threshold,
                                   float alpha, float beta, void *stream) {
    if (int rc = check_threshold(threshold, T81_THR_TORCH)) return rc;
    if (rows < 0 || tokens < 0 || k < 0)
        return fail(T81_HIP_EINVAL_SHAPE, "gemm_ternary dimensions must be non-negative");
    if (rows > (int64_t{65535} * 16) || tokens > INT_MAX / 2 || k > (int64_t{1} << 31))
        return fail(T81_HIP_EINVAL_SHAPE, "matmul_input dimensions too large");
    if (!float_dtype(x_dtype)) return fail(T81_HIP_EINVAL_DTYPE, "input must be a float dtype");
    if (rows == 0 || tokens == 0) {
        g_last_error.clear();
        return T81_HIP_OK;
    }
    if (c == nullptr || (k > 0 && (w == nullptr || x == nullptr)))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (reinterpret_cast<uintptr_t>(w) % 16 != 0 || reinterpret_cast<uintptr_t>(c) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(x) % (x_dtype == T81_DTYPE_F32 ? 4 : 2) != 0)
        return fail(T81_HIP_EINVAL_POINTER, "misaligned weight, activation or output pointer");
    if (int rc = require_device("t81_hip_matmul_input_reference")) return rc;
    return finish(t81hip::launch_gemm_limb_fused(w, x, x_dtype, c, static_cast<int>(rows),
                                                 static_cast<int>(tokens), k, threshold, alpha,
                                                 beta, static_cast<hipStream_t>(stream)),
                  "t81_hip_matmul_input_reference");
}

int t81_hip_transpose_packed(const uint8_t *packed, uint8_t *out, int64_t rows, int64_t cols,
                             void *stream) {
    if (rows < 0 || cols < 0) return fail(T81_HIP_EINVAL_SHAPE, "rows and cols must be non-negative");
    if (cols > int64_t{48} * 4 * 65535 || rows > (int64_t{1} << 36))
        return fail(T81_HIP_EINVAL_SHAPE, "transpose_packed dimensions too large");
    if (rows > 0 && cols > 0 && (packed == nullptr || out == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (reinterpret_cast<uintptr_t>(packed) % 16 != 0 || reinterpret_cast<uintptr_t>(out) % 16 != 0)
        return fail(T81_HIP_EINVAL_POINTER, "packed limbs must be 16-byte aligned");
    if (int rc = require_device("t81_hip_transpose_packed")) return rc;
    return finish(t81hip::launch_transpose_packed(packed, out, rows, cols,
                                                  static_cast<hipStream_t>(stream)),
                  "t81_hip_transpose_packed");
}

int t81_hip_tq_block_bytes(int quant) {
    if (quant == T81_TQ1_0) return 54;
    if (quant == T81_TQ2_0) return 66;
    return fail(T81_HIP_EINVAL_DTYPE, "quant must be T81_TQ1_0 (34) or T81_TQ2_0 (35)");
}

int t81_hip_tq_quantize(const float *src, uint8_t *dst, int64_t rows, int64_t cols,
                        float threshold, int quant, void *stream) {
    if (quant != T81_TQ1_0 && quant != T81_TQ2_0)
        return fail(T81_HIP_EINVAL_DTYPE, "quant must be T81_TQ1_0 (34) or T81_TQ2_0 (35)");
    if (rows < 0 || cols < 0) return fail(T81_HIP_EINVAL_SHAPE, "rows and cols must be non-negative");
    if (too_many(rows, cols)) return fail(T81_HIP_EINVAL_SHAPE, "rows x cols too large");
    if (rows > 0 && cols > 0 && (src == nullptr || dst == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (reinterpret_cast<uintptr_t>(src) % 4 != 0)
        return fail(T81_HIP_EINVAL_POINTER, "float32 data must be 4-byte aligned");
    // t81/gguf.py:675-676: np.clip(threshold, 0, 1); a threshold of 0 selects rounding
    float thr = threshold < 0.0f ? 0.0f : (threshold > 1.0f ? 1.0f : threshold);
    if (threshold != threshold) thr = threshold;
    const int use_thr = thr > 0.0f ? 1 : 0;
    if (int rc = require_device("t81_hip_tq_quantize")) return rc;
    return finish(t81hip::launch_tq_quantize(src, dst, rows, cols, thr, use_thr, quant,
                                             static_cast<hipStream_t>(stream)),
                  "t81_hip_tq_quantize");
}

int t81_hip_tq_dequantize(const uint8_t *src, float *dst, int64_t rows, int64_t cols, int quant,
                          void *stream) {
    if (quant != T81_TQ1_0 && quant != T81_TQ2_0)
        return fail(T81_HIP_EINVAL_DTYPE, "quant must be T81_TQ1_0 (34) or T81_TQ2_0 (35)");
    if (rows < 0 || cols < 0) return fail(T81_HIP_EINVAL_SHAPE, "rows and cols must be non-negative");
    if (too_many(rows, cols)) return fail(T81_HIP_EINVAL_SHAPE, "rows x cols too large");
    if (rows > 0 && cols > 0 && (src == nullptr || dst == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (reinterpret_cast<uintptr_t>(dst) % 4 != 0)
        return fail(T81_HIP_EINVAL_POINTER, "float32 data must be 4-byte aligned");
    if (int rc = require_device("t81_hip_tq_dequantize")) return rc;
    return finish(t81hip::launch_tq_dequantize(src, dst, rows, cols, quant,
                                               static_cast<hipStream_t>(stream)),
                  "t81_hip_tq_dequantize");
}

// ---- the TQ1_0 row codec of src/t81/core/gguf_quants.h and its tensor payload ----
int t81_hip_tq1_quantize_rows(const float *values, int64_t rows, int64_t cols, float threshold,
                              const float *scales_in, float *scales_out, uint16_t *dst,
                              void *stream) {
    if (rows < 0 || cols < 0) return fail(T81_HIP_EINVAL_SHAPE, "rows and cols must be non-negative");
    if (too_many(rows, cols) || rows > INT_MAX) return fail(T81_HIP_EINVAL_SHAPE, "rows x cols too large");
    if (rows > 0 && cols > 0 && (values == nullptr || dst == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (reinterpret_cast<uintptr_t>(values) % 4 != 0 || reinterpret_cast<uintptr_t>(dst) % 2 != 0 ||
        reinterpret_cast<uintptr_t>(scales_in) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(scales_out) % 4 != 0)
        return fail(T81_HIP_EINVAL_POINTER, "misaligned values, words or scales pointer");
    if (int rc = require_device("t81_hip_tq1_quantize_rows")) return rc;
    return finish(t81hip::launch_tq1r_quantize_rows(values, rows, cols, threshold, scales_in,
                                                    scales_out, dst,
                                                    static_cast<hipStream_t>(stream)),
                  "t81_hip_tq1_quantize_rows");
}

int t81_hip_tq1_dequantize_rows(const uint16_t *src, int64_t rows, int64_t cols,
                                const float *scales, float *dst, void *stream) {
    if (rows < 0 || cols < 0) return fail(T81_HIP_EINVAL_SHAPE, "rows and cols must be non-negative");
    if (too_many(rows, cols)) return fail(T81_HIP_EINVAL_SHAPE, "rows x cols too large");
    if (rows > 0 && cols > 0 && (src == nullptr || dst == nullptr || scales == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (reinterpret_cast<uintptr_t>(src) % 2 != 0 || reinterpret_cast<uintptr_t>(dst) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(scales) % 4 != 0)
        return fail(T81_HIP_EINVAL_POINTER, "misaligned words, output or scales pointer");
    if (int rc = require_device("t81_hip_tq1_dequantize_rows")) return rc;
    return finish(t81hip::launch_tq1r_dequantize_rows(src, rows, cols, scales, dst,
                                                      static_cast<hipStream_t>(stream)),
                  "t81_hip_tq1_dequantize_rows");
}

int64_t t81_hip_tq1_payload_bytes(int64_t rows, int64_t cols, int64_t block_rows,
                                  int refinements) {
    if (rows < 0 || cols < 0) return fail(T81_HIP_EINVAL_SHAPE, "rows and cols must be non-negative");
    if (too_many(rows, cols)) return fail(T81_HIP_EINVAL_SHAPE, "rows x cols too large");
    return t81hip::tq1r_payload_bytes(rows, cols, block_rows, refinements != 0);
}

int t81_hip_tq1_quantize_payload(const float *values, int64_t rows, int64_t cols,
                                 int64_t block_rows, int refinements, float threshold,
                                 uint8_t *payload, void *stream) {
    if (rows < 0 || cols < 0) return fail(T81_HIP_EINVAL_SHAPE, "rows and cols must be non-negative");
    if (too_many(rows, cols) || rows > INT_MAX) return fail(T81_HIP_EINVAL_SHAPE, "rows x cols too large");
    if (rows > 0 && (payload == nullptr || (cols > 0 && values == nullptr)))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (reinterpret_cast<uintptr_t>(values) % 4 != 0)
        return fail(T81_HIP_EINVAL_POINTER, "float32 data must be 4-byte aligned");
    if (int rc = require_device("t81_hip_tq1_quantize_payload")) return rc;
    return finish(t81hip::launch_tq1r_quantize_payload(values, rows, cols, block_rows,
                                                       refinements != 0, threshold, payload,
                                                       static_cast<hipStream_t>(stream)),
                  "t81_hip_tq1_quantize_payload");
}

// python/bindings.cpp:561-638: the binding's checks, in its order and with its messages.
int t81_hip_tq1_dequantize_payload(const uint8_t *payload, int64_t payload_bytes, int64_t rows,
                                   int64_t cols, int64_t block_rows, int refinements, float *dst,
                                   void *stream) {
    if (rows < 0 || cols < 0) return fail(T81_HIP_EINVAL_SHAPE, "rows and cols must be non-negative");
    if (payload_bytes < 0) return fail(T81_HIP_EINVAL_SHAPE, "payload size must be non-negative");
    if (payload == nullptr && payload_bytes > 0)
        return fail(T81_HIP_EINVAL_POINTER, "buffer pointer is null");
    if (too_many(rows, cols)) return fail(T81_HIP_EINVAL_SHAPE, "rows x cols too large");
    switch (t81hip::tq1r_payload_check(payload_bytes, rows, cols, block_rows, refinements != 0)) {
        case 1: return fail(T81_HIP_EINVAL_SHAPE, "buffer truncated while reading scale");
        case 2: return fail(T81_HIP_EINVAL_SHAPE, "buffer truncated while skipping refinement bytes");
        case 3: return fail(T81_HIP_EINVAL_SHAPE, "buffer truncated while reading quantized rows");
        default: break;
    }
    if (rows > 0 && cols > 0 && dst == nullptr) return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (reinterpret_cast<uintptr_t>(dst) % 4 != 0)
        return fail(T81_HIP_EINVAL_POINTER, "float32 data must be 4-byte aligned");
    if (int rc = require_device("t81_hip_tq1_dequantize_payload")) return rc;
    return finish(t81hip::launch_tq1r_dequantize_payload(payload, rows, cols, block_rows,
                                                         refinements != 0, dst,
                                                         static_cast<hipStream_t>(stream)),
                  "t81_hip_tq1_dequantize_payload");
}

int t81_hip_tq2_matmul(const void *x, int x_dtype, const uint8_t *w, float *c, int64_t m,
                       int64_t n, int64_t k, float alpha, float beta, const float *bias,
                       void *stream) {
    if (m < 0 || n < 0 || k < 0)
        return fail(T81_HIP_EINVAL_SHAPE, "tq2_matmul dimensions must be non-negative");
    if (m > INT_MAX / 2 || k > (int64_t(1) << 31) || (n > 0 && !t81hip::tq2_matmul_fits(n, k)))
        return fail(T81_HIP_EINVAL_SHAPE, "tq2_matmul dimensions too large");
    if (x_dtype != T81_DTYPE_F32 && x_dtype != T81_DTYPE_BF16 && x_dtype != T81_DTYPE_I8)
        return fail(T81_HIP_EINVAL_DTYPE, "activations must be float32, bfloat16 or int8");
    if ((m > 0 && k > 0 && x == nullptr) || (n > 0 && k > 0 && w == nullptr) ||
        (m > 0 && n > 0 && c == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    const uintptr_t elem = x_dtype == T81_DTYPE_F32 ? 4 : (x_dtype == T81_DTYPE_BF16 ? 2 : 1);
    if (reinterpret_cast<uintptr_t>(w) % 4 != 0 || reinterpret_cast<uintptr_t>(x) % elem != 0 ||
        reinterpret_cast<uintptr_t>(c) % 4 != 0 || reinterpret_cast<uintptr_t>(bias) % 4 != 0)
        return fail(T81_HIP_EINVAL_POINTER, "misaligned weight, activation, output or bias pointer");
    if (int rc = require_device("t81_hip_tq2_matmul")) return rc;
    if (m == 0 || n == 0) return T81_HIP_OK;
    // k == 0: no blocks; the kernel still writes beta * c + bias (empty sums)
    return finish(t81hip::launch_tq2_matmul(x, x_dtype, w, c, m, n, k, alpha, beta, bias,
                                            static_cast<hipStream_t>(stream)),
                  "t81_hip_tq2_matmul");
}

}  // extern "C"

struct t81_hip_spmm_plan {
    int rows = 0;
    int cols = 0;
    int64_t nnz = 0;         // entries stored (those before the first bad one)
    int32_t *row_ptr = nullptr;  // rows + 1
    int32_t *col = nullptr;      // nnz, sorted by row, list order within a row
    double *val = nullptr;       // nnz
};

namespace {

void spmm_free(t81_hip_spmm_plan *p) {
    if (!p) return;
    (void)hipFree(p->row_ptr);
    (void)hipFree(p->col);
    (void)hipFree(p->val);
    delete p;
}

}  // namespace

extern "C" {

int t81_hip_spmm_plan_create(const int64_t *values, const int32_t *row_idx,
                             const int32_t *col_idx, int64_t nnz, int rows, int cols,
                             t81_hip_spmm_plan **plan, int64_t *first_bad, void *stream) {
    const char *where = "t81_hip_spmm_plan_create";
    if (plan == nullptr) return fail(T81_HIP_EINVAL_POINTER, "null plan pointer");
    *plan = nullptr;
    if (first_bad) *first_bad = -1;
    // python/bindings.cpp:903-905, simple.hpp:46-48
    if (rows < 0 || cols < 0) return fail(T81_HIP_EINVAL_SHAPE, "Matrix dimensions must be non-negative");
    if (nnz < 0 || nnz > INT32_MAX)
        return fail(T81_HIP_EINVAL_SHAPE, "entry count must be in [0, 2^31 - 1]");
    if (nnz > 0 && (values == nullptr || row_idx == nullptr || col_idx == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (reinterpret_cast<uintptr_t>(values) % 8 != 0 || reinterpret_cast<uintptr_t>(row_idx) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(col_idx) % 4 != 0)
        return fail(T81_HIP_EINVAL_POINTER, "misaligned entry arrays");
    if (int rc = require_device(where)) return rc;
    const hipStream_t s = static_cast<hipStream_t>(stream);

    auto *p = new (std::nothrow) t81_hip_spmm_plan;
    if (!p) return fail(T81_HIP_EHIP, "out of host memory");
    p->rows = rows;
    p->cols = cols;
    unsigned long long *bad_dev = nullptr;
    void *scratch = nullptr;
    auto cleanup = [&](int rc) {
        (void)hipFree(bad_dev);
        (void)hipFree(scratch);
        if (rc != T81_HIP_OK && rc != T81_HIP_EINVAL_INDEX) spmm_free(p);
        return rc;
    };
    hipError_t e = hipMalloc(&bad_dev, sizeof(unsigned long long));
    if (e != hipSuccess) return cleanup(hip_fail(e, where));
    e = t81hip::launch_spmm_first_bad(row_idx, col_idx, nnz, rows, cols, bad_dev, s);
    unsigned long long bad = 0;
    if (e == hipSuccess) e = hipMemcpyAsync(&bad, bad_dev, sizeof(bad), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return cleanup(hip_fail(e, where));
    const int64_t n = static_cast<int64_t>(bad < static_cast<unsigned long long>(nnz) ? bad : nnz);
    p->nnz = n;

    e = hipMalloc(&p->row_ptr, (static_cast<size_t>(rows) + 1) * sizeof(int32_t));
    if (e == hipSuccess && n > 0) e = hipMalloc(&p->col, static_cast<size_t>(n) * sizeof(int32_t));
    if (e == hipSuccess && n > 0) e = hipMalloc(&p->val, static_cast<size_t>(n) * sizeof(double));
    if (e == hipSuccess && n > 0) e = hipMalloc(&scratch, t81hip::spmm_sort_scratch_bytes(n));
    if (e == hipSuccess)
        e = t81hip::launch_spmm_build(values, row_idx, col_idx, n, rows, scratch, p->row_ptr, p->col,
                                      p->val, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);  // scratch is freed next
    if (e != hipSuccess) return cleanup(hip_fail(e, where));

    *plan = p;
    if (n < nnz) {
        // simple.hpp:79-84: the row check comes first
        int32_t r = 0;
        e = hipMemcpy(&r, row_idx + n, sizeof(r), hipMemcpyDeviceToHost);
        if (e != hipSuccess) {
            *plan = nullptr;
            return cleanup(hip_fail(e, where));  // frees p
        }
        if (first_bad) *first_bad = n;
        return cleanup(fail(T81_HIP_EINVAL_INDEX, r < 0 || r >= rows ? "Row index out of bounds"
                                                                     : "Column index out of bounds"));
    }
    g_last_error.clear();
    return cleanup(T81_HIP_OK);
}

int t81_hip_spmm_plan_apply(const t81_hip_spmm_plan *plan, const float *B, float *C, int N,
                            float alpha, float beta, void *stream) {
    if (plan == nullptr) return fail(T81_HIP_EINVAL_POINTER, "null plan");
    if (N < 0) return fail(T81_HIP_EINVAL_SHAPE, "Feature dimension N must be non-negative");  // bindings.cpp:906-908
    if ((plan->rows > 0 && N > 0 && C == nullptr) || (plan->cols > 0 && N > 0 && B == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    if (reinterpret_cast<uintptr_t>(B) % 4 != 0 || reinterpret_cast<uintptr_t>(C) % 4 != 0)
        return fail(T81_HIP_EINVAL_POINTER, "float32 data must be 4-byte aligned");
    if (int rc = require_device("t81_hip_spmm_plan_apply")) return rc;
    return finish(t81hip::launch_spmm_apply(plan->row_ptr, plan->col, plan->val, B, C, plan->rows, N,
                                            alpha, beta, static_cast<hipStream_t>(stream)),
                  "t81_hip_spmm_plan_apply");
}

int t81_hip_spmm_plan_info(const t81_hip_spmm_plan *plan, int *rows, int *cols, int64_t *nnz) {
    if (plan == nullptr) return fail(T81_HIP_EINVAL_POINTER, "null plan");
    if (rows) *rows = plan->rows;
    if (cols) *cols = plan->cols;
    if (nnz) *nnz = plan->nnz;
    return T81_HIP_OK;
}

void t81_hip_spmm_plan_destroy(t81_hip_spmm_plan *plan) { spmm_free(plan); }

int t81_hip_spmm_simple(const int64_t *values, const int32_t *row_idx, const int32_t *col_idx,
                        int64_t nnz, int rows, int cols, const float *B, float *C, int N,
                        float alpha, float beta, void *stream) {
    if (N < 0) return fail(T81_HIP_EINVAL_SHAPE, "Feature dimension N must be non-negative");
    if (rows < 0 || cols < 0) return fail(T81_HIP_EINVAL_SHAPE, "Matrix dimensions must be non-negative");
    if (reinterpret_cast<uintptr_t>(B) % 4 != 0 || reinterpret_cast<uintptr_t>(C) % 4 != 0)
        return fail(T81_HIP_EINVAL_POINTER, "float32 data must be 4-byte aligned");
    if ((rows > 0 && N > 0 && C == nullptr) || (cols > 0 && N > 0 && B == nullptr))
        return fail(T81_HIP_EINVAL_POINTER, "null data pointer");
    t81_hip_spmm_plan *plan = nullptr;
    int64_t bad = -1;
    const int rc = t81_hip_spmm_plan_create(values, row_idx, col_idx, nnz, rows, cols, &plan, &bad,
                                            stream);
    if (rc != T81_HIP_OK && rc != T81_HIP_EINVAL_INDEX) return rc;
    const std::string msg = g_last_error;
    int rc2 = t81_hip_spmm_plan_apply(plan, B, C, N, alpha, beta, stream);
    if (rc2 == T81_HIP_OK) {
        const hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
        if (e != hipSuccess) rc2 = hip_fail(e, "t81_hip_spmm_simple");
    }
    spmm_free(plan);
    if (rc2 != T81_HIP_OK) return rc2;
    if (rc == T81_HIP_EINVAL_INDEX) return fail(rc, msg);
    g_last_error.clear();
    return T81_HIP_OK;
}

void t81_hip_limb_tryte_table(double *out) { t81hip::host_tryte_table(out); }

}  // extern "C"

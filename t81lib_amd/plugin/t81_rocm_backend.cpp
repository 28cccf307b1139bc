// t81lib_amd/plugin/t81_rocm_backend.cpp -- the ROCm backend of t81lib's C++ dispatch,
// implemented over libt81_hip.so (include/t81_hip.h).
//
// A t81lib build configured with T81LIB_USE_ROCM=1 expects six symbols in
// t81::linalg::detail (include/t81/linalg/gemm_gpu.hpp:70-72, 80-85, 131-140,
// 233-249).  This file defines them; it is compiled inside that build, against
// t81lib's own headers, and linked with libt81_hip.so and the HIP runtime.
//
// Contract kept from the reference dispatch:
//  * synchronous: every call has finished, and its outputs are visible to the
//    host, when it returns;
//  * rocm_gemm_ternary has the semantics of gemm_ternary_cpu_impl
//    (src/linalg/gemm_cpu.cpp:8-71), bit for bit (K4); its caller,
//    gemm_ternary_dispatch (gemm_gpu.hpp:162-214), has already checked the sizes;
//  * the elementwise ops check what cpu_where / cpu_clamp / cpu_lerp /
//    cpu_addcmul check (src/linalg/gemm_dispatch.cpp:43-90, 145-211), with the
//    same exception types and messages, and compute the same values;
//  * errors from the library become std::invalid_argument (argument codes) or
//    std::runtime_error (HIP / device codes), as in src/linalg/gemm_rocm.cpp:22-27.
// Difference: buffers already in device memory (hipPointerGetAttributes says so)
// are used in place; host buffers are staged through temporary device copies.
//
// It also defines the trit-dot overload of gemm_ternary declared in t81_rocm_trit.hpp
// (X times the packed trit matrix, on the decode GEMV / prefill GEMM kernels), which the
// reference has no counterpart for: its C++ gemm_ternary multiplies limb integers only.
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <span>
#include <stdexcept>
#include <string>

#include <t81/linalg/gemm_gpu.hpp>
#include <t81/tensor_metadata.hpp>

#include "t81_hip.h"
#include "t81_rocm_trit.hpp"

namespace t81::linalg::detail {

namespace {

void check_rc(int rc) {
    if (rc == T81_HIP_OK) return;
    const std::string msg = t81_hip_last_error();
    if (rc == T81_HIP_EHIP || rc == T81_HIP_ENODEV) throw std::runtime_error(msg);
    throw std::invalid_argument(msg);
}

void check_hip(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

bool is_device_pointer(const void *p) {
    if (p == nullptr) return false;
    hipPointerAttribute_t attr{};
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();  // unknown to HIP: ordinary host memory
        return false;
    }
    return attr.type == hipMemoryTypeDevice;
}

// A device view of `bytes` bytes at `host_or_device`: the pointer itself when it is
// device memory, else a temporary device copy (copied in if `copy_in`, and back by
// `write_back()`).
class DeviceView {
  public:
    DeviceView(const void *p, std::size_t bytes, bool copy_in)
        : host_(const_cast<void *>(p)), bytes_(bytes) {
        if (bytes == 0 || is_device_pointer(p)) {
            dev_ = host_;
            return;
        }
        check_hip(hipMalloc(&dev_, bytes), "hipMalloc");
        owned_ = true;
        if (copy_in) check_hip(hipMemcpy(dev_, p, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
    }
    DeviceView(const DeviceView &) = delete;
    DeviceView &operator=(const DeviceView &) = delete;
    ~DeviceView() {
        if (owned_) (void)hipFree(dev_);
    }
    void *get() const { return dev_; }
    bool staged() const { return owned_; }
    void write_back() {
        check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
        if (owned_) check_hip(hipMemcpy(host_, dev_, bytes_, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    }

  private:
    void *host_ = nullptr;
    void *dev_ = nullptr;
    std::size_t bytes_ = 0;
    bool owned_ = false;
};

// The float32 view checks of gemm_dispatch.cpp:43-90.
float *float_data(const TensorMetadata &meta) {
    if (!meta.dtype_is_float32())
        throw std::invalid_argument("tensor metadata must describe float32 data");
    if (meta.data_ptr == nullptr)
        throw std::invalid_argument("tensor metadata must provide a valid data pointer");
    if (!meta.is_contiguous())
        throw std::invalid_argument("tensor metadata must describe contiguous storage");
    const std::int64_t offset = meta.storage_offset > 0 ? meta.storage_offset : 0;
    return reinterpret_cast<float *>(static_cast<std::uint8_t *>(meta.data_ptr) +
                                     static_cast<std::size_t>(offset) * sizeof(float));
}

}  // namespace

bool rocm_available() noexcept { return t81_hip_available() != 0; }

void rocm_gemm_ternary(std::span<const core::limb> A, std::span<const core::limb> B,
                       std::span<float> C, int M, int N, int K, float alpha, float beta) {
    if (M == 0 || N == 0) return;
    DeviceView a(A.data(), A.size_bytes(), true);
    DeviceView b(B.data(), B.size_bytes(), true);
    DeviceView c(C.data(), C.size_bytes(), true);
    check_rc(t81_hip_gemm_ternary_limb(static_cast<const std::uint8_t *>(a.get()),
                                       static_cast<const std::uint8_t *>(b.get()),
                                       static_cast<float *>(c.get()), M, N, K, alpha, beta,
                                       nullptr));
    c.write_back();
}

void rocm_where(const TensorMetadata &condition, const TensorMetadata &x,
                const TensorMetadata &y, TensorMetadata &out) {
    const float *pc = float_data(condition), *px = float_data(x), *py = float_data(y);
    float *po = float_data(out);
    const std::size_t n = out.numel();
    if (condition.numel() != n || x.numel() != n || y.numel() != n)
        throw std::invalid_argument("input shapes must match on the CPU path");
    DeviceView dc(pc, n * 4, true), dx(px, n * 4, true), dy(py, n * 4, true), dout(po, n * 4, false);
    check_rc(t81_hip_where(static_cast<const float *>(dc.get()), static_cast<const float *>(dx.get()),
                           static_cast<const float *>(dy.get()), static_cast<float *>(dout.get()),
                           static_cast<std::int64_t>(n), nullptr));
    dout.write_back();
}

void rocm_clamp(const TensorMetadata &input, TensorMetadata &out, float min_value,
                float max_value) {
    const float *pi = float_data(input);
    float *po = float_data(out);
    const std::size_t n = out.numel();
    if (input.numel() != n) throw std::invalid_argument("input/output lengths must match for clamp");
    DeviceView di(pi, n * 4, true), dout(po, n * 4, false);
    check_rc(t81_hip_clamp(static_cast<const float *>(di.get()), static_cast<float *>(dout.get()),
                           static_cast<std::int64_t>(n), min_value, max_value, nullptr));
    dout.write_back();
}

void rocm_lerp(const TensorMetadata &start, const TensorMetadata &end,
               const TensorMetadata &weight, TensorMetadata &out) {
    const float *ps = float_data(start), *pe = float_data(end), *pw = float_data(weight);
    float *po = float_data(out);
    const std::size_t n = out.numel();
    if (start.numel() != n || end.numel() != n || weight.numel() != n)
        throw std::invalid_argument("inputs for lerp must match output length");
    DeviceView ds(ps, n * 4, true), de(pe, n * 4, true), dw(pw, n * 4, true), dout(po, n * 4, false);
    check_rc(t81_hip_lerp(static_cast<const float *>(ds.get()), static_cast<const float *>(de.get()),
                          static_cast<const float *>(dw.get()), static_cast<float *>(dout.get()),
                          static_cast<std::int64_t>(n), nullptr));
    dout.write_back();
}

void rocm_addcmul(const TensorMetadata &input, const TensorMetadata &tensor1,
                  const TensorMetadata &tensor2, float value, TensorMetadata &out) {
    const float *pi = float_data(input), *p1 = float_data(tensor1), *p2 = float_data(tensor2);
    float *po = float_data(out);
    const std::size_t n = out.numel();
    if (input.numel() != n || tensor1.numel() != n || tensor2.numel() != n)
        throw std::invalid_argument("inputs for addcmul must align with output");
    DeviceView di(pi, n * 4, true), d1(p1, n * 4, true), d2(p2, n * 4, true), dout(po, n * 4, false);
    check_rc(t81_hip_addcmul(static_cast<const float *>(di.get()), static_cast<const float *>(d1.get()),
                             static_cast<const float *>(d2.get()), value,
                             static_cast<float *>(dout.get()), static_cast<std::int64_t>(n),
                             nullptr));
    dout.write_back();
}

// ---------------------------------------------------------------- trit-dot --
namespace {

int dtype_code(TritActivation t) {
    switch (t) {
        case TritActivation::Float32: return T81_DTYPE_F32;
        case TritActivation::BFloat16: return T81_DTYPE_BF16;
        case TritActivation::Int8: return T81_DTYPE_I8;
    }
    throw std::invalid_argument("unknown activation type");
}

std::size_t dtype_bytes(TritActivation t) {
    return t == TritActivation::Float32 ? 4 : (t == TritActivation::BFloat16 ? 2 : 1);
}

// rank-2 contiguous metadata -> (rows, cols, first element)
struct Matrix2 {
    std::int64_t rows, cols;
    std::uint8_t *data;
};

Matrix2 matrix2(const TensorMetadata &m, std::size_t elem, const char *name) {
    if (m.sizes.size() != 2)
        throw std::invalid_argument(std::string(name) + " must be a rank-2 tensor");
    if (m.data_ptr == nullptr && m.numel() > 0)
        throw std::invalid_argument("tensor metadata must provide a valid data pointer");
    if (!m.is_contiguous())
        throw std::invalid_argument("tensor metadata must describe contiguous storage");
    if (m.sizes[0] < 0 || m.sizes[1] < 0)
        throw std::invalid_argument("gemm_ternary dimensions must be non-negative");
    const std::int64_t offset = m.storage_offset > 0 ? m.storage_offset : 0;
    return {m.sizes[0], m.sizes[1],
            static_cast<std::uint8_t *>(m.data_ptr) + static_cast<std::size_t>(offset) * elem};
}

}  // namespace

}  // namespace t81::linalg::detail

namespace t81::linalg {

void gemm_ternary(const void *X, TritActivation x_type, std::span<const core::limb> W, void *C,
                  int M, int N, int K, float alpha, float beta, const float *bias,
                  void *stream) {
    if (M < 0 || N < 0 || K < 0)
        throw std::invalid_argument("gemm_ternary dimensions must be non-negative");
    const std::size_t L = (static_cast<std::size_t>(K) + core::limb::TRITS - 1) / core::limb::TRITS;
    if (static_cast<std::size_t>(N) * L != W.size())
        throw std::invalid_argument("W span size does not match (N, ceil(K / 48))");
    const int code = detail::dtype_code(x_type);
    if (M == 0 || N == 0) return;
    if (!detail::rocm_available())
        throw std::runtime_error("the trit-dot gemm_ternary needs a gfx950 device");
    const std::size_t xb = static_cast<std::size_t>(M) * static_cast<std::size_t>(K) *
                           detail::dtype_bytes(x_type);
    const std::size_t cb = static_cast<std::size_t>(M) * static_cast<std::size_t>(N) * 4;
    detail::DeviceView x(X, xb, true), w(W.data(), W.size_bytes(), true);
    detail::DeviceView c(C, cb, beta != 0.0f), b(bias, bias ? static_cast<std::size_t>(N) * 4 : 0, true);
    hipStream_t s = static_cast<hipStream_t>(stream);
    // K3's split-K workspace for shapes with few output tiles, from the stream-ordered pool
    // (a pool allocation, freed in stream order): calls on different streams may run at the
    // same time, which t81_hip_ternary_matmul_noalloc's one static scratch per device does
    // not allow
    const std::int64_t wsb = t81_hip_ternary_matmul_workspace_size(M, N, K, code);
    void *ws = nullptr;
    if (wsb > 0) detail::check_hip(hipMallocAsync(&ws, static_cast<std::size_t>(wsb), s), "hipMallocAsync");
    const int rc = t81_hip_ternary_matmul_ws(0, x.get(), code,
                                             static_cast<const std::uint8_t *>(w.get()), c.get(),
                                             M, N, K, alpha, beta,
                                             static_cast<const float *>(b.get()), ws, wsb, s);
    if (ws != nullptr) (void)hipFreeAsync(ws, s);
    detail::check_rc(rc);
    if (stream == nullptr || x.staged() || w.staged() || c.staged() || b.staged()) c.write_back();
}

namespace detail {

void gemm_ternary_trit(const TensorMetadata &X, const TensorMetadata &W, TensorMetadata &C,
                       float alpha, float beta, const TensorMetadata *bias) {
    TritActivation xt;
    switch (X.dtype) {
        case ScalarType::Float: xt = TritActivation::Float32; break;
        case ScalarType::BFloat16: xt = TritActivation::BFloat16; break;
        case ScalarType::Char: xt = TritActivation::Int8; break;
        default: throw std::invalid_argument("activations must be float32, bfloat16 or int8");
    }
    if (!W.dtype_is_ternary_limb())
        throw std::invalid_argument("packed weights must be TernaryLimb metadata");
    const ScalarType c_type = xt == TritActivation::Int8 ? ScalarType::Int : ScalarType::Float;
    if (C.dtype != c_type)
        throw std::invalid_argument(xt == TritActivation::Int8
                                        ? "C must be int32 for int8 activations"
                                        : "tensor metadata must describe float32 data");
    const Matrix2 x = matrix2(X, dtype_bytes(xt), "X");
    const Matrix2 w = matrix2(W, sizeof(core::limb), "W");
    const Matrix2 c = matrix2(C, 4, "C");
    const std::int64_t L = (x.cols + core::limb::TRITS - 1) / core::limb::TRITS;
    if (w.cols != L)
        throw std::invalid_argument("W shape must match the ceil(K / 48) dimension of X");
    if (c.rows != x.rows || c.cols != w.rows)
        throw std::invalid_argument("C shape must match the output dimensions");
    const float *bp = nullptr;
    if (bias != nullptr) {
        if (!bias->dtype_is_float32() || bias->numel() != static_cast<std::size_t>(w.rows))
            throw std::invalid_argument("bias must hold N float32 values");
        bp = float_data(*bias);
    }
    if (x.rows > INT32_MAX || w.rows > INT32_MAX || x.cols > INT32_MAX)
        throw std::invalid_argument("gemm_ternary dimensions too large");
    gemm_ternary(x.data, xt,
                 std::span<const core::limb>(reinterpret_cast<const core::limb *>(w.data),
                                             static_cast<std::size_t>(w.rows * w.cols)),
                 c.data, static_cast<int>(x.rows), static_cast<int>(w.rows),
                 static_cast<int>(x.cols), alpha, beta, bp, nullptr);
}

}  // namespace detail
}  // namespace t81::linalg

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
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <span>
#include <stdexcept>
#include <string>

#include <t81/linalg/gemm_gpu.hpp>
#include <t81/tensor_metadata.hpp>

#include "t81_hip.h"

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

}  // namespace t81::linalg::detail

// t81lib_amd/csrc/noalloc.hip -- t81_hip_ternary_matmul_noalloc: the trit-dot matmul with
// its workspace (K3's split-K partial tiles, K2's partials for 9..16 tokens over a long K
// with float32 or int8 activations, the bf16 planes of float32 activations past 64 tokens)
// taken from a static device array, for callers that cannot allocate device memory (code
// under HIP graph capture, serving loops that forbid it).
//
// `scratch` is a file-scope device array, reserved when the code object is loaded on a
// device and held until the process ends, one copy per device at its own address.  In
// host code its name is only a registration handle, so each device's address is looked
// up once with hipGetSymbolAddress (that device current) and that pointer is what the
// kernels receive.  Every call on a device shares the array: calls that overlap on one
// device (different streams, or threads) race and must be serialised by the caller.
// Nothing in it needs to start at zero -- a split launch writes every partial it later
// reads, the planes path every plane value -- so the last call's contents are simply
// overwritten.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "../../include/t81_hip.h"
#include "t81_kernels.hpp"

namespace {

constexpr int64_t kScratchBytes = int64_t{64} << 20;   // 64 MiB
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mutex;
void *g_scratch[kMaxDevices];   // non-null once a device's lookup has succeeded

// The current device's address of `scratch`.  Only a successful lookup is kept: a failed
// one (for instance under a capture that refuses it) is reported and tried again on the
// next call.
int scratch_address(void **out) {
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return t81hip::report_error(T81_HIP_EHIP, (std::string("t81_hip_ternary_matmul_noalloc: ") +
                                                   hipGetErrorString(e)).c_str());
    if (dev < 0 || dev >= kMaxDevices)
        return t81hip::report_error(T81_HIP_ENODEV, "device index out of range");
    std::lock_guard<std::mutex> lock(g_mutex);
    if (g_scratch[dev] == nullptr) {
        void *p = nullptr;
        const hipError_t le = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (le != hipSuccess || p == nullptr)
            return t81hip::report_error(
                T81_HIP_EHIP, (std::string("t81_hip_ternary_matmul_noalloc: scratch lookup: ") +
                               hipGetErrorString(le)).c_str());
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return T81_HIP_OK;
}

}  // namespace

extern "C" {

int t81_hip_ternary_matmul_noalloc(int which, const void *x, int x_dtype, const uint8_t *w,
                                   void *c, int64_t m, int64_t n, int64_t k, float alpha,
                                   float beta, const float *bias, void *stream) {
    // the arguments first, with the messages of t81_hip_ternary_matmul_ws
    if (int rc = t81hip::check_matmul_args(which, x, x_dtype, w, c, m, n, k, alpha, beta, bias))
        return rc;
    // Same workspace as t81_hip_ternary_matmul_ws is given by its callers (exactly
    // t81_hip_ternary_matmul_workspace_size bytes), so the split plan -- and with it the
    // order of every sum -- is the same, and so are the results, bit for bit.
    const int64_t need = t81_hip_ternary_matmul_workspace_size(m, n, k, x_dtype);
    if (need > kScratchBytes)
        return t81hip::report_error(
            T81_HIP_EINVAL_SHAPE,
            ("t81_hip_ternary_matmul_noalloc: this shape splits K over " + std::to_string(need) +
             " bytes of workspace, more than the " + std::to_string(kScratchBytes) +
             "-byte static scratch; use t81_hip_ternary_matmul_ws")
                .c_str());
    void *ws = nullptr;
    if (need > 0) {
        if (int rc = scratch_address(&ws)) return rc;
    }
    return t81_hip_ternary_matmul_ws(which, x, x_dtype, w, c, m, n, k, alpha, beta, bias, ws,
                                     need, stream);
}

}  // extern "C"

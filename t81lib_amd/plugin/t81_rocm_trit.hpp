// t81lib_amd/plugin/t81_rocm_trit.hpp -- the trit-dot overload of t81::linalg::gemm_ternary
// that a T81LIB_USE_ROCM build of t81lib gains from t81lib_amd/plugin/t81_rocm_backend.cpp.
//
// The reference's gemm_ternary (include/t81/linalg/gemm.hpp:68-77, gemm_gpu.hpp:113-140)
// multiplies two packed operands as 48-trit limb integers.  Every other consumer of the
// packed weights -- TernaryTensor's backward, t8.nn.Linear's training forward, the GGUF
// dequantisers -- reads them as a trit matrix T and multiplies it with float or integer
// activations.  This overload is that product, on the decode GEMV (M <= 16) and prefill
// GEMM kernels of libt81_hip.so:
//
//   C[m, n] = alpha * sum_{k < K} X[m, k] * T[n, k] + beta * C[m, n] + bias[n]
//
//   X     M x K row-major activations of type x_type;
//   W     N rows x ceil(K / 48) limbs, the layout pack_dense_matrix / from_float produce
//         (trits past K are zero);
//   C     M x N row-major float32 -- int32 for Int8 activations, exact (alpha must be 1,
//         beta 0 or 1, bias null, K <= 131071);
//   bias  N floats or null.
//
// Pointers may be host or device memory (device buffers are used in place, host buffers
// staged).  stream == nullptr: the call has finished, and C is visible to the host, when it
// returns (the reference's synchronous contract); otherwise work is ordered on `stream`
// and device-resident outputs are complete once the stream is (host buffers are still
// written back before the call returns).  Errors: std::invalid_argument for arguments,
// std::runtime_error for device failures or a missing gfx950.
#pragma once

#include <span>

#include <t81/core/limb.hpp>
#include <t81/tensor_metadata.hpp>

namespace t81::linalg {

enum class TritActivation { Float32, BFloat16, Int8 };

void gemm_ternary(const void *X, TritActivation x_type, std::span<const core::limb> W, void *C,
                  int M, int N, int K, float alpha = 1.0f, float beta = 0.0f,
                  const float *bias = nullptr, void *stream = nullptr);

namespace detail {

// The same product on TensorMetadata (the route of gemm_dispatch.cpp:325-344): X rank-2
// (M, K) Float / BFloat16 / Char, W rank-2 (N, ceil(K / 48)) TernaryLimb, C rank-2 (M, N)
// Float (Int for Char activations), bias rank-1 (N) Float or null; all contiguous;
// storage_offset in elements.  Synchronous.
void gemm_ternary_trit(const TensorMetadata &X, const TensorMetadata &W, TensorMetadata &C,
                       float alpha, float beta, const TensorMetadata *bias = nullptr);

}  // namespace detail
}  // namespace t81::linalg

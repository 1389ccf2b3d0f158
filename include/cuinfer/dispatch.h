// dispatch.h -- per-tensor weight format -> fused matmul.
//
// Mirrors matmul_dispatch (ref:src/model.cu:797-825, copied at
// ref:src/attention.cu:744-771) for the six formats of this library; the
// reference's FP32 branch calls matmul_tiled with pre-transposed [K,N]
// weights, which is outside this library and throws std::invalid_argument.
#pragma once

#include <hip/hip_runtime_api.h>

#include "tensor.h"

namespace cuinfer {

// ref:include/cuinfer/model.h:34-42
enum class WeightFormat { FP32, FP16, Q8_0, Q4_0, Q5_0, Q4_K, Q6_K };

const char* weight_format_name(WeightFormat fmt);
// Format of a weight tensor's dtype (Q4_K_M files mix Q4_K and Q6_K tensors).
WeightFormat weight_format_of(DType dtype);

// C[M,N] = A[M,K] * dequant(weight[N,K])^T on `stream`.
void matmul_dispatch(const float* A, const Tensor& weight, float* C, int M, int N, int K, WeightFormat format,
                     hipStream_t stream = 0);

// Decode-batch (M <= 16) forms with the neighbouring elementwise work folded into the
// matmul's activation staging (no counterpart in the reference; see cri_matmul_rmsnorm /
// cri_matmul_swiglu in cri.h):
//   C = RMSNorm(hidden + residual) * weight^T, hidden + residual also written to hidden_out
//   (not null, not overlapping hidden/residual) -- replaces rmsnorm_residual + matmul_dispatch;
//   C = (silu(gate) * up) * weight^T, gate/up rows ld floats apart -- replaces silu + multiply + matmul_dispatch.
void matmul_dispatch_rmsnorm(const float* hidden, const float* residual, const float* norm_weight, float* hidden_out,
                             const Tensor& weight, float* C, int M, int N, int K, WeightFormat format, float eps,
                             hipStream_t stream = 0);
void matmul_dispatch_swiglu(const float* gate, const float* up, int ld, const Tensor& weight, float* C, int M, int N,
                            int K, WeightFormat format, hipStream_t stream = 0);

}  // namespace cuinfer

// embedding.h -- the transposed-B matmul used by the LM head.
#pragma once

#include <hip/hip_runtime_api.h>

namespace cuinfer {

// C[M,N] = A[M,K] * B[N,K]^T, all fp32 device pointers
// (ref:include/cuinfer/embedding.h:136-137).
void matmul_transposed_b(const float* A, const float* B, float* C, int M, int N, int K, hipStream_t stream = 0);

}  // namespace cuinfer

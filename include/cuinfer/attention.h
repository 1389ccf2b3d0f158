// attention.h -- GQA-broadcast batched matmul.
#pragma once

#include <hip/hip_runtime_api.h>

namespace cuinfer {

// C[h] = A[h] * B[h / (n_heads / n_kv_heads)]; A [n_heads,M,K], B [n_kv_heads,K,N],
// C [n_heads,M,N], fp32 device pointers (ref:include/cuinfer/attention.h:79-82).
void batched_matmul_gqa(const float* A, const float* B, float* C, int n_heads, int n_kv_heads, int M, int N, int K,
                        hipStream_t stream = 0);

}  // namespace cuinfer

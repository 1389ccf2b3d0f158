// attention.h -- GQA-broadcast batched matmul and fused decode attention.
#pragma once

#include <hip/hip_runtime_api.h>

namespace cuinfer {

// C[h] = A[h] * B[h / (n_heads / n_kv_heads)]; A [n_heads,M,K], B [n_kv_heads,K,N],
// C [n_heads,M,N], fp32 device pointers (ref:include/cuinfer/attention.h:79-82).
void batched_matmul_gqa(const float* A, const float* B, float* C, int n_heads, int n_kv_heads, int M, int N, int K,
                        hipStream_t stream = 0);

// Decode attention of one query token: output[h] = softmax(scale * Q[h] . K[t, h / G]) V[t, h / G]
// over t < kv_len, G = n_heads / n_kv_heads; Q and output [n_heads * head_dim], K_cache and V_cache
// in the cache layout [kv_len, n_kv_heads, head_dim], fp32 device pointers
// (ref:include/cuinfer/attention.h:161-167).  Throws std::runtime_error for kv_len == 0,
// head_dim > 256 or n_heads % n_kv_heads != 0.
void fused_decode_attention(const float* Q, const float* K_cache, const float* V_cache, float* output, int n_heads,
                            int n_kv_heads, int head_dim, int kv_len, float scale, hipStream_t stream = 0);

// Prompt attention (the prefill branch of ref:src/attention.cu:809-871 after the cache append):
// M rotated query rows at Q + m * ldq at positions pos .. pos + M - 1, row m attending to cache
// positions [0, pos + m]; output [M, n_heads * head_dim].  Allocates its workspace for the call
// (cri_prefill_attention takes a caller's).  Throws std::runtime_error on an unsupported shape.
void prefill_attention(const float* Q, int ldq, const float* K_cache, const float* V_cache, float* output, int M,
                       int n_heads, int n_kv_heads, int head_dim, int pos, float scale, hipStream_t stream = 0);

}  // namespace cuinfer

// matmul_quant.h -- fused dequantize + matmul, C[M,N] = A[M,K] * dequant(B[N,K])^T.
//
// Same signatures and argument meaning as ref:include/cuinfer/kernels/matmul_quant.h:37-105,
// with hipStream_t in place of cudaStream_t.  A, C fp32 row-major device
// pointers; B GGUF-native [N,K] rows of K/block_size blocks.  C is overwritten.
// K must be a multiple of 32 (Q8_0, Q4_0, Q5_0, FP16) or 256 (Q4_K, Q6_K);
// violations throw std::runtime_error instead of truncating.
#pragma once

#include <hip/hip_runtime_api.h>

namespace cuinfer {

void matmul_q8_0(const float* A, const void* B_quant, float* C, int M, int N, int K, hipStream_t stream = 0);
void matmul_q4_0(const float* A, const void* B_quant, float* C, int M, int N, int K, hipStream_t stream = 0);
void matmul_q5_0(const float* A, const void* B_quant, float* C, int M, int N, int K, hipStream_t stream = 0);
void matmul_q4_k(const float* A, const void* B_quant, float* C, int M, int N, int K, hipStream_t stream = 0);
void matmul_q6_k(const float* A, const void* B_quant, float* C, int M, int N, int K, hipStream_t stream = 0);
void matmul_fp16(const float* A, const void* B_fp16, float* C, int M, int N, int K, hipStream_t stream = 0);

}  // namespace cuinfer

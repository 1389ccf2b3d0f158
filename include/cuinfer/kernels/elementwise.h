// elementwise.h -- the two elementwise neighbours of the fused matmuls.
//
// rmsnorm_residual keeps the reference's signature
// (ref:include/cuinfer/kernels/elementwise.h:107-110); silu_mul is the
// reference's silu then multiply pair (:23, :75) as one launch, the way the
// quantized FFN uses them (ref:src/model.cu:996-997).
#pragma once

#include <hip/hip_runtime_api.h>

namespace cuinfer {

// output = input + residual; normed = output * weight * rsqrt(mean(output^2) + eps), per row of n.
// output may alias input; residual may be null.
void rmsnorm_residual(const float* input, const float* residual, const float* weight, float* output, float* normed,
                      int rows, int n, float eps = 1e-5f, hipStream_t stream = 0);

// out = silu(gate) * up over n elements (out may alias gate or up).
void silu_mul(const float* gate, const float* up, float* out, long long n, hipStream_t stream = 0);

}  // namespace cuinfer

// generic.hip -- any-M fused dequant matmul with element-wise decode.
//
// C[M,N] = A[M,K] * dequant(B[N,K])^T for every format and every shape the
// ABI accepts, including rows that are not dword aligned.  This is the
// correctness backstop used when no specialised kernel applies; it follows
// the reference's structure (dequantised B tile in LDS, fp32 FMA from LDS,
// ref:src/kernels/matmul_quant.cu:64-119) with a 64x32 output tile per
// 256-thread block and 8 outputs per thread.
#include "common.hpp"
#include "decode.hpp"
#include "internal.hpp"

namespace cri {
namespace dev {

constexpr int kGTN = 64;  // weight rows per tile
constexpr int kGTM = 32;  // activation rows per tile
constexpr int kGTK = 32;  // k per LDS stage

__global__ __launch_bounds__(256) void generic_matmul_kernel(int fmt, const float* __restrict__ A,
                                                             const uint8_t* __restrict__ B, float* __restrict__ C,
                                                             int M, int N, int K, long rbytes) {
    __shared__ float bs[kGTK][kGTN + 1];
    __shared__ float as[kGTM][kGTK + 1];
    const int tid = threadIdx.x;
    const int n0 = blockIdx.x * kGTN, m0 = blockIdx.y * kGTM;
    const int tx = tid & 63;      // output column (weight row) in tile
    const int ty = tid >> 6;      // 0..3 -> output rows ty*8 .. ty*8+7
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};

    // B-tile fill: thread -> (row tid/4, 8 consecutive k); A-tile fill: 4 floats
    const int br = tid >> 2, bk = (tid & 3) * 8;
    const int ar = tid >> 3, ak = (tid & 7) * 4;
    for (int k0 = 0; k0 < K; k0 += kGTK) {
        {
            const int n = n0 + br;
            const uint8_t* row = B + static_cast<long>(n < N ? n : 0) * rbytes;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int k = k0 + bk + i;
                bs[bk + i][br] = (n < N && k < K) ? decode_row_elem(fmt, row, k) : 0.0f;
            }
        }
        {
            const int m = m0 + ar;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int k = k0 + ak + i;
                as[ar][ak + i] = (m < M && k < K) ? A[static_cast<long>(m) * K + k] : 0.0f;
            }
        }
        __syncthreads();
#pragma unroll 8
        for (int k = 0; k < kGTK; ++k) {
            const float b = bs[k][tx];
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = __builtin_fmaf(as[ty * 8 + i][k], b, acc[i]);
        }
        __syncthreads();
    }
    const int n = n0 + tx;
    if (n < N) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int m = m0 + ty * 8 + i;
            if (m < M) C[static_cast<long>(m) * N + n] = acc[i];
        }
    }
}

}  // namespace dev

namespace detail {

int launch_generic_matmul(int fmt, const float* A, const void* B, float* C, int M, int N, int K,
                          hipStream_t stream) {
    const dim3 grid((N + dev::kGTN - 1) / dev::kGTN, (M + dev::kGTM - 1) / dev::kGTM);
    hipLaunchKernelGGL(dev::generic_matmul_kernel, grid, dim3(256), 0, stream, fmt, A,
                       static_cast<const uint8_t*>(B), C, M, N, K, row_bytes(fmt, K));
    return 0;
}

}  // namespace detail
}  // namespace cri

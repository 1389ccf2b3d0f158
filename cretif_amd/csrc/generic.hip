// generic.hip -- any-M fused dequant matmul with element-wise decode.
//
// C[M,N] = A[M,K] * dequant(B[N,K])^T for every format and every shape the
// ABI accepts, including rows that are not dword aligned.  This is the
// correctness backstop used when no specialised kernel applies; it follows
// the reference's structure (dequantised B tile in LDS, fp32 FMA from LDS,
// ref:src/kernels/matmul_quant.cu:64-119) with a 64x32 output tile per
// 256-thread block and 8 outputs per thread.  MODE (see ActIn) computes the
// activations as they are tiled (SwiGLU, or RMSNorm with the row factor from
// per-thread sums of squares reduced over the 8 threads that tile a row).
#include "act.hpp"
#include "common.hpp"
#include "decode.hpp"
#include "internal.hpp"

namespace cri {
namespace dev {

constexpr int kGTN = 64;  // weight rows per tile
constexpr int kGTM = 32;  // activation rows per tile
constexpr int kGTK = 32;  // k per LDS stage

template <int MODE>
__global__ __launch_bounds__(256) void generic_matmul_kernel(int fmt, const ActIn P, const uint8_t* __restrict__ B,
                                                             float* __restrict__ C, int M, int N, int K,
                                                             long rbytes) {
    __shared__ float bs[kGTK][kGTN + 1];
    __shared__ float as[kGTM][kGTK + 1];
    __shared__ float rfac[kGTM];
    float ss = 0.0f;  // RMSNorm: this thread's part of its tile row's sum of v^2
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
            const int k = k0 + ak;
            f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
            if (m < M && k + 4 <= K) {
                ActRaw<MODE> raw;
                act_load<MODE>(raw, P, m, k, MODE == kActPlain ? K : P.lda);
                v = act_finish<MODE>(raw, P, m, k, K, ss, blockIdx.x == 0);
            } else if (m < M) {
                // ragged K: one element at a time (the four-wide form needs k + 4 <= K)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (k + i >= K) break;
                    const long off = static_cast<long>(m) * (MODE == kActPlain ? K : P.lda) + k + i;
                    float x;
                    if constexpr (MODE == kActPlain) {
                        x = P.a[off];
                    } else if constexpr (MODE == kActSwiGLU) {
                        x = silu_f(P.a[off]) * P.b[off];
                    } else {
                        const float h = P.a[off] + (P.b ? P.b[off] : 0.0f);
                        ss = __builtin_fmaf(h, h, ss);
                        if (blockIdx.x == 0 && P.h_out) P.h_out[static_cast<long>(m) * K + k + i] = h;
                        x = h * P.w[k + i];
                    }
                    v[i] = x;
                }
            }
            as[ar][ak] = v.x;
            as[ar][ak + 1] = v.y;
            as[ar][ak + 2] = v.z;
            as[ar][ak + 3] = v.w;
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
    if constexpr (MODE == kActRMSNorm) {
        // the 8 threads tiling row ar are lanes 8 ar' .. 8 ar' + 7 of one wave
        ss = group_sum_t<3>(ss);
        if ((tid & 7) == 0) rfac[ar] = rms_factor(ss, K, P.eps);
        __syncthreads();
    }
    const int n = n0 + tx;
    if (n < N) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int m = m0 + ty * 8 + i;
            if (m < M) C[static_cast<long>(m) * N + n] = MODE == kActRMSNorm ? acc[i] * rfac[ty * 8 + i] : acc[i];
        }
    }
}

}  // namespace dev

namespace detail {

int launch_generic_matmul_act(int mode, int fmt, const ActIn& act, const void* B, float* C, int M, int N, int K,
                              hipStream_t stream) {
    const dim3 grid((N + dev::kGTN - 1) / dev::kGTN, (M + dev::kGTM - 1) / dev::kGTM);
    const uint8_t* Bb = static_cast<const uint8_t*>(B);
    const long rb = row_bytes(fmt, K);
    switch (mode) {
        case kActPlain:
            hipLaunchKernelGGL(dev::generic_matmul_kernel<kActPlain>, grid, dim3(256), 0, stream, fmt, act, Bb, C, M,
                               N, K, rb);
            return 0;
        case kActSwiGLU:
            hipLaunchKernelGGL(dev::generic_matmul_kernel<kActSwiGLU>, grid, dim3(256), 0, stream, fmt, act, Bb, C,
                               M, N, K, rb);
            return 0;
        case kActRMSNorm:
            hipLaunchKernelGGL(dev::generic_matmul_kernel<kActRMSNorm>, grid, dim3(256), 0, stream, fmt, act, Bb, C,
                               M, N, K, rb);
            return 0;
    }
    return -1;
}

int launch_generic_matmul(int fmt, const float* A, const void* B, float* C, int M, int N, int K,
                          hipStream_t stream) {
    const ActIn act{A, nullptr, nullptr, nullptr, K, 0.0f};
    return launch_generic_matmul_act(kActPlain, fmt, act, B, C, M, N, K, stream);
}

}  // namespace detail
}  // namespace cri

// step_kernels.hip -- the small neighbours of the matmuls in one decode step:
// RoPE with the KV-cache append, the greedy token choice, and the device-side
// position counter that lets a captured step be replayed token after token.
//
// The position lives in device memory and every kernel that needs it reads it
// there, so a HIP graph of the step stays valid as the sequence grows: the
// counter is advanced by the last kernel of the step.
#include <cmath>

#include "common.hpp"
#include "internal.hpp"

namespace cri {
namespace dev {

// One thread per rotated pair (q heads, then k heads) plus one per v element
// pair of a row; grid.y = row.  The rotation is the reference's
// (ref:src/kernels/elementwise.cu:232-257): pair i of a head (elements 2i and
// 2i+1) turns by pos * theta^(-2i / head_dim), with the same fp32 expression
// for the angle.  Rotated k and the unchanged v go to cache row pos, as
// KVCache::append copies them (ref:src/kv_cache.cu:181-196).
__global__ __launch_bounds__(256) void rope_append_kernel(float* __restrict__ q, long ldq, const float* __restrict__ k,
                                                          long ldk, const float* __restrict__ v, long ldv, int n_heads,
                                                          int n_kv_heads, int head_dim, float theta,
                                                          const int* __restrict__ pos_dev, float* __restrict__ kc,
                                                          float* __restrict__ vc) {
    const int m = blockIdx.y;
    const int pos = *pos_dev + m;
    const int half = head_dim / 2;
    const int qpairs = n_heads * half, kpairs = n_kv_heads * half;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const long kvd = static_cast<long>(n_kv_heads) * head_dim;
    float* krow = kc + static_cast<long>(pos) * kvd;
    if (i < qpairs + kpairs) {
        const bool isq = i < qpairs;
        const int pi = isq ? i : i - qpairs;
        const int head = pi / half, lp = pi - head * half;
        // theta^e, cos and sin are evaluated in double and rounded once to fp32, i.e. the
        // correctly rounded values the fp32 expressions stand for (the position amplifies a
        // one-ulp difference in the frequency ~pos times); the angle and the rotation are the
        // reference's fp32 operations, the products rounded separately (no contraction)
        const float e = (2.0f * static_cast<float>(lp)) / static_cast<float>(head_dim);
        const float freq = 1.0f / static_cast<float>(pow(static_cast<double>(theta), static_cast<double>(e)));
        const float ang = static_cast<float>(pos) * freq;
        const float cs = static_cast<float>(cos(static_cast<double>(ang)));
        const float sn = static_cast<float>(sin(static_cast<double>(ang)));
        const long off = static_cast<long>(head) * head_dim + 2 * lp;
        const float* src = isq ? q + m * ldq + off : k + m * ldk + off;
        const float x0 = src[0], x1 = src[1];
        const float y0 = __fsub_rn(__fmul_rn(x0, cs), __fmul_rn(x1, sn));
        const float y1 = __fadd_rn(__fmul_rn(x0, sn), __fmul_rn(x1, cs));
        float* dst = isq ? q + m * ldq + off : krow + off;
        dst[0] = y0;
        dst[1] = y1;
    } else if (i < qpairs + kpairs + (kvd + 1) / 2) {
        const long e = 2L * (i - qpairs - kpairs);
        float* vrow = vc + static_cast<long>(pos) * kvd;
        vrow[e] = v[m * ldv + e];
        if (e + 1 < kvd) vrow[e + 1] = v[m * ldv + e + 1];
    }
}

// One workgroup of 1024 threads per row.  A thread keeps the first index of
// its strided elements' maximum (the comparison v > best skips NaN and keeps
// the earlier index on ties); the workgroup then merges (value, index) pairs
// preferring the larger value, then the smaller index -- the reference's
// kernel_argmax (ref:src/embedding.cu:155-200), whose start value -FLT_MAX at
// index 0 is kept too.
constexpr int kArgmaxThreads = 1024;

__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(const float* __restrict__ logits, long ld, int n,
                                                                     int* __restrict__ out) {
    __shared__ float sv[kArgmaxThreads / 64];
    __shared__ int si[kArgmaxThreads / 64];
    const float* row = logits + blockIdx.x * ld;
    float best = -3.402823466e38f;
    int bi = 0;
    for (int j = threadIdx.x; j < n; j += kArgmaxThreads) {
        const float x = row[j];
        if (x > best) {
            best = x;
            bi = j;
        }
    }
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) {
        const float ov = __shfl_xor(best, s);
        const int oi = __shfl_xor(bi, s);
        argmax_merge(best, bi, ov, oi);
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[wave] = best;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kArgmaxThreads / 64; ++w) argmax_merge(best, bi, sv[w], si[w]);
        out[blockIdx.x] = bi;
    }
}

__global__ void pos_update_kernel(int* pos, int value, int add) {
    if (threadIdx.x == 0) *pos = add ? *pos + value : value;
}

}  // namespace dev

namespace detail {

int launch_rope_append(float* q, long ldq, const float* k, long ldk, const float* v, long ldv, int rows, int n_heads,
                       int n_kv_heads, int head_dim, float theta, const int* pos, float* k_cache, float* v_cache,
                       hipStream_t stream) {
    if (rows < 1 || rows > 65535 || head_dim < 2 || head_dim % 2 != 0) return kDeclined;
    const long kvd = static_cast<long>(n_kv_heads) * head_dim;
    const long work = static_cast<long>(n_heads + n_kv_heads) * (head_dim / 2) + (kvd + 1) / 2;
    const long blocks = (work + 255) / 256;
    if (blocks > 0x7FFFFFFFL) return kDeclined;
    hipLaunchKernelGGL(dev::rope_append_kernel, dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(rows)),
                       dim3(256), 0, stream, q, ldq, k, ldk, v, ldv, n_heads, n_kv_heads, head_dim, theta, pos, k_cache,
                       v_cache);
    return 0;
}

int launch_argmax_rows(const float* logits, long ld, int rows, int n, int* out, hipStream_t stream) {
    if (rows < 1 || n < 1) return kDeclined;
    hipLaunchKernelGGL(dev::argmax_rows_kernel, dim3(static_cast<unsigned>(rows)), dim3(dev::kArgmaxThreads), 0, stream,
                       logits, ld, n, out);
    return 0;
}

int launch_pos_add(int* pos, int delta, hipStream_t stream) {
    hipLaunchKernelGGL(dev::pos_update_kernel, dim3(1), dim3(64), 0, stream, pos, delta, 1);
    return 0;
}

int launch_pos_set(int* pos, int value, hipStream_t stream) {
    hipLaunchKernelGGL(dev::pos_update_kernel, dim3(1), dim3(64), 0, stream, pos, value, 0);
    return 0;
}

}  // namespace detail
}  // namespace cri

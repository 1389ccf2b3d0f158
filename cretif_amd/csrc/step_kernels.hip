// step_kernels.hip -- the small neighbours of the matmuls in one decode step:
// RoPE with the KV-cache append, the greedy token choice, and the device-side
// position counter that lets a captured step be replayed token after token.
//
// The position lives in device memory and every kernel that needs it reads it
// there, so a HIP graph of the step stays valid as the sequence grows: the
// counter is advanced by the last kernel of the step.
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "internal.hpp"
#include "split.hpp"

namespace cri {
namespace dev {

// One thread per rotated pair (q heads, then k heads) plus one per v element
// pair of a row; grid.y = row.  The rotation is the reference's
// (ref:src/kernels/elementwise.cu:232-257): pair i of a head (elements 2i and
// 2i+1) turns by the angle pos * theta^(-2i / head_dim).  Its cosine and sine
// come from `rot`, a [max_seq, head_dim / 2] table of (cos, sin) built once on
// the host with the reference's fp32 expressions for the frequency and the
// angle and cos/sin rounded once to fp32 (the position amplifies a one-ulp
// difference in the frequency ~pos times, so these are computed exactly rather
// than with fast device approximations).  The products are rounded separately
// (no contraction), as in the reference's fp32 expression.  Rotated k and the
// unchanged v go to cache row pos, as KVCache::append copies them
// (ref:src/kv_cache.cu:181-196).  With qkv.S > 0 the q/k/v projection arrives
// as its unreduced partial sums: q, k and v are its columns [0, ..), [kcol, ..)
// and [vcol, ..), reduced here exactly as the reduction kernel would, and the
// rotated q is written to q.
__global__ __launch_bounds__(256) void rope_append_kernel(float* __restrict__ q, long ldq, const float* __restrict__ k,
                                                          long ldk, const float* __restrict__ v, long ldv, int n_heads,
                                                          int n_kv_heads, int head_dim, const f32x2* __restrict__ rot,
                                                          const int* __restrict__ pos_dev, float* __restrict__ kc,
                                                          float* __restrict__ vc, const SplitSums qkv, int kcol,
                                                          int vcol) {
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
        const f32x2 cs = rot[static_cast<long>(pos) * half + lp];
        const long off = static_cast<long>(head) * head_dim + 2 * lp;
        float x0, x1;
        if (qkv.S) {
            const long e = static_cast<long>(m) * qkv.N + (isq ? 0 : kcol) + off;
            const float f = split_factor(qkv, m);
            x0 = split_sum(qkv, e) * f;
            x1 = split_sum(qkv, e + 1) * f;
        } else {
            const float* src = isq ? q + m * ldq + off : k + m * ldk + off;
            x0 = src[0];
            x1 = src[1];
        }
        const float y0 = __fsub_rn(__fmul_rn(x0, cs.x), __fmul_rn(x1, cs.y));
        const float y1 = __fadd_rn(__fmul_rn(x0, cs.y), __fmul_rn(x1, cs.x));
        float* dst = isq ? q + m * ldq + off : krow + off;
        dst[0] = y0;
        dst[1] = y1;
    } else if (i < qpairs + kpairs + (kvd + 1) / 2) {
        const long e = 2L * (i - qpairs - kpairs);
        float* vrow = vc + static_cast<long>(pos) * kvd;
        if (qkv.S) {
            const long o = static_cast<long>(m) * qkv.N + vcol + e;
            const float f = split_factor(qkv, m);
            vrow[e] = split_sum(qkv, o) * f;
            if (e + 1 < kvd) vrow[e + 1] = split_sum(qkv, o + 1) * f;
        } else {
            vrow[e] = v[m * ldv + e];
            if (e + 1 < kvd) vrow[e + 1] = v[m * ldv + e + 1];
        }
    }
}

// Greedy token of each row, kernel_argmax's rule (ref:src/embedding.cu:155-200):
// the largest value (a comparison v > best, so NaN never wins), the smallest
// index among equal maxima, starting from (-FLT_MAX, 0).  The rule is a total
// order on (value, index), so any merge order gives the same answer.  Each
// row is cut into gridDim.x slices; a workgroup reduces its slice and writes
// (value, index) to `part`; the last workgroup of the row (release / acquire
// fences around a counter, reset afterwards) merges the slices.  The last
// workgroup of row 0 also advances the position counter by `pos_add` when
// `pos` is not null (the step's final kernel).
constexpr int kArgmaxThreads = 256;

__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

__device__ __forceinline__ void argmax_block(float& best, int& bi) {
    __shared__ float sv[kArgmaxThreads / 64];
    __shared__ int si[kArgmaxThreads / 64];
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
    best = sv[0];
    bi = si[0];
    for (int w = 1; w < kArgmaxThreads / 64; ++w) argmax_merge(best, bi, sv[w], si[w]);
}

// vec (rows 16-byte aligned): the slice is read as 16-byte loads, eight per thread issued
// before any is compared (a loop of dependent scalar loads took ~14 us for one 128256-logit
// row); slices start on multiples of four.
__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(const float* __restrict__ logits, long ld, int n,
                                                                     int* __restrict__ out, f32x2* __restrict__ part,
                                                                     unsigned* __restrict__ counters,
                                                                     int* __restrict__ pos, int pos_add, int vec) {
    const int row = blockIdx.y, nb = gridDim.x, b = blockIdx.x;
    const float* r = logits + row * ld;
    const int per = ((n + nb - 1) / nb + 3) & ~3;
    const int j0 = min(n, b * per), j1 = min(n, j0 + per);
    float best = -3.402823466e38f;
    int bi = 0;
    int js = j0;  // first element of the scalar tail
    if (vec) {
        constexpr int kBatch = 8;
        const int nv = (j1 - j0) >> 2;  // whole 16-byte groups of the slice
        for (int q0 = 0; q0 < nv; q0 += kBatch * kArgmaxThreads) {
            f32x4 x[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {  // clamped, so every load is in bounds and unconditional
                const int q = min(q0 + u * kArgmaxThreads + static_cast<int>(threadIdx.x), nv - 1);
                x[u] = *reinterpret_cast<const f32x4*>(r + j0 + 4 * q);
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int q = q0 + u * kArgmaxThreads + static_cast<int>(threadIdx.x);
                if (q < nv) {
                    const int j = j0 + 4 * q;
                    argmax_merge(best, bi, x[u].x, j);
                    argmax_merge(best, bi, x[u].y, j + 1);
                    argmax_merge(best, bi, x[u].z, j + 2);
                    argmax_merge(best, bi, x[u].w, j + 3);
                }
            }
        }
        js = j0 + 4 * nv;
    }
    for (int j = js + threadIdx.x; j < j1; j += kArgmaxThreads) argmax_merge(best, bi, r[j], j);
    argmax_block(best, bi);
    __shared__ int last;
    if (threadIdx.x == 0) {
        part[static_cast<long>(row) * nb + b] = f32x2{best, __int_as_float(bi)};
        // release: the slice result before the count (a release alone: no L2 invalidate here)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        last = atomicAdd(&counters[row], 1u) == static_cast<unsigned>(nb - 1);
    }
    __syncthreads();
    if (!last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // acquire: every slice's result
    best = -3.402823466e38f;
    bi = 0;
    for (int s = threadIdx.x; s < nb; s += kArgmaxThreads) {
        const f32x2 p = part[static_cast<long>(row) * nb + s];
        argmax_merge(best, bi, p.x, __float_as_int(p.y));
    }
    argmax_block(best, bi);
    if (threadIdx.x == 0) {
        out[row] = bi;
        counters[row] = 0u;
        if (pos && row == 0) *pos += pos_add;
    }
}

// The residual stream entering a layer, for a step's layer taps: out = h + (the pending
// residual: its partial sums added in split order, as the next RMSNorm prologue adds them).
__global__ __launch_bounds__(256) void hidden_tap_kernel(const float* __restrict__ h, const SplitSums r,
                                                         float* __restrict__ out, int rows, int n) {
    const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= static_cast<long>(rows) * n) return;
    float v = h[i];
    if (r.S) {
        const long row = i / n, col = i - row * n;
        const float* src = r.part + row * r.N + col;
        float t = src[0];
        for (int s = 1; s < r.S; ++s) t += src[s * r.stride];
        v += t;
    }
    out[i] = v;
}

__global__ void pos_update_kernel(int* pos, int value, int add) {
    if (threadIdx.x == 0) *pos = add ? *pos + value : value;
}

}  // namespace dev

namespace detail {

int launch_rope_append(float* q, long ldq, const float* k, long ldk, const float* v, long ldv, int rows, int n_heads,
                       int n_kv_heads, int head_dim, const float* rot, const int* pos, float* k_cache, float* v_cache,
                       hipStream_t stream, const SplitSums* qkv, int kcol, int vcol) {
    if (rows < 1 || rows > 65535 || head_dim < 2 || head_dim % 2 != 0) return kDeclined;
    const SplitSums none;
    if (qkv && qkv->S > dev::kSplitMaxS) return kDeclined;
    const long kvd = static_cast<long>(n_kv_heads) * head_dim;
    const long work = static_cast<long>(n_heads + n_kv_heads) * (head_dim / 2) + (kvd + 1) / 2;
    const long blocks = (work + 255) / 256;
    if (blocks > 0x7FFFFFFFL) return kDeclined;
    hipLaunchKernelGGL(dev::rope_append_kernel, dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(rows)),
                       dim3(256), 0, stream, q, ldq, k, ldk, v, ldv, n_heads, n_kv_heads, head_dim,
                       reinterpret_cast<const dev::f32x2*>(rot), pos, k_cache, v_cache, qkv ? *qkv : none, kcol, vcol);
    return 0;
}

int argmax_slices(int n) { return static_cast<int>(std::min<long>(64, std::max<long>(1, (n + 8191) / 8192))); }

int launch_argmax_rows(const float* logits, long ld, int rows, int n, int* out, float* part, unsigned* counters,
                       int* pos, int pos_add, hipStream_t stream) {
    if (rows < 1 || rows > 65535 || n < 1) return kDeclined;
    const int vec = (reinterpret_cast<uintptr_t>(logits) & 15u) == 0 && ld % 4 == 0;
    hipLaunchKernelGGL(dev::argmax_rows_kernel, dim3(static_cast<unsigned>(argmax_slices(n)), static_cast<unsigned>(rows)),
                       dim3(dev::kArgmaxThreads), 0, stream, logits, ld, n, out, reinterpret_cast<dev::f32x2*>(part),
                       counters, pos, pos_add, vec);
    return 0;
}

int launch_pos_add(int* pos, int delta, hipStream_t stream) {
    hipLaunchKernelGGL(dev::pos_update_kernel, dim3(1), dim3(64), 0, stream, pos, delta, 1);
    return 0;
}

int launch_hidden_tap(const float* h, const SplitSums& r, float* out, int rows, int n, hipStream_t stream) {
    const long total = static_cast<long>(rows) * n;
    if (total <= 0) return 0;
    hipLaunchKernelGGL(dev::hidden_tap_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream,
                       h, r, out, rows, n);
    return 0;
}

int launch_pos_set(int* pos, int value, hipStream_t stream) {
    hipLaunchKernelGGL(dev::pos_update_kernel, dim3(1), dim3(64), 0, stream, pos, value, 0);
    return 0;
}

}  // namespace detail
}  // namespace cri

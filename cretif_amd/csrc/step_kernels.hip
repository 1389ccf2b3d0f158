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
            x0 = split_sum_any(qkv, e) * f;
            x1 = split_sum_any(qkv, e + 1) * f;
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
            vrow[e] = split_sum_any(qkv, o) * f;
            if (e + 1 < kvd) vrow[e + 1] = split_sum_any(qkv, o + 1) * f;
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

// ---- prompt attention through batched_matmul_gqa (the reference's prefill, ref:src/attention.cu:809-871)
// Every kernel reads the position from device memory: rows t >= kv_len = pos + M of a cache operand
// are written as zeros and score columns past row m's causal limit pos + m + 1 are masked, so the
// padded width T4 (a multiple of 4, >= kv_len) may exceed kv_len -- a captured step uses the cache's
// full length and stays correct at every position it is replayed at.

// q rows [M][ldq] (head h at columns h D .. h D + D - 1) -> qh [H][M][D] (transpose_seq_heads)
__global__ __launch_bounds__(256) void heads_from_rows_kernel(const float* __restrict__ q, long ldq,
                                                              float* __restrict__ qh, int M, int H, int D) {
    const long i = (static_cast<long>(blockIdx.x) * 256 + threadIdx.x) * 4;  // element of qh
    if (i >= static_cast<long>(H) * M * D) return;
    const int d = static_cast<int>(i % D);
    const long hm = i / D;
    const int m = static_cast<int>(hm % M), h = static_cast<int>(hm / M);
    *reinterpret_cast<f32x4*>(qh + i) = ld_f32x4(q + m * ldq + h * D + d);
}

// o [H][M][D] -> ctx rows [M][H D] (transpose_heads_seq)
__global__ __launch_bounds__(256) void rows_from_heads_kernel(const float* __restrict__ o, float* __restrict__ ctx,
                                                              int M, int H, int D) {
    const long i = (static_cast<long>(blockIdx.x) * 256 + threadIdx.x) * 4;  // element of ctx
    if (i >= static_cast<long>(H) * M * D) return;
    const int hd = static_cast<int>(i % (static_cast<long>(H) * D));
    const int m = static_cast<int>(i / (static_cast<long>(H) * D));
    const int h = hd / D, d = hd % D;
    *reinterpret_cast<f32x4*>(ctx + i) = *reinterpret_cast<const f32x4*>(o + (static_cast<long>(h) * M + m) * D + d);
}

// cache [T][Hkv][D] -> vh [Hkv][T4][D] (rows t >= pos + kv_rows zero)
__global__ __launch_bounds__(256) void v_heads_kernel(const float* __restrict__ vc, float* __restrict__ vh, int Hkv,
                                                      int D, int T4, const int* __restrict__ pos, int kv_rows) {
    const long i = (static_cast<long>(blockIdx.x) * 256 + threadIdx.x) * 4;  // element of vh
    if (i >= static_cast<long>(Hkv) * T4 * D) return;
    const int kv_len = *pos + kv_rows;
    const int d = static_cast<int>(i % D);
    const long kt = i / D;
    const int t = static_cast<int>(kt % T4), kv = static_cast<int>(kt / T4);
    f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    if (t < kv_len) v = *reinterpret_cast<const f32x4*>(vc + (static_cast<long>(t) * Hkv + kv) * D + d);
    *reinterpret_cast<f32x4*>(vh + i) = v;
}

// cache [T][Hkv][D] -> kt [Hkv][D][T4] (transpose_seq_heads + transpose_k; columns t >= pos +
// kv_rows zero): a 64-position x D tile through LDS per workgroup, read along d and written along t
__global__ __launch_bounds__(256) void k_transpose_kernel(const float* __restrict__ kc, float* __restrict__ kt,
                                                          int Hkv, int D, int T4, const int* __restrict__ pos,
                                                          int kv_rows) {
    __shared__ float tile[64][detail::kDecodeAttnSplitMaxHeadDim + 1];
    const int kv = blockIdx.y, t0 = blockIdx.x * 64;
    const int kv_len = *pos + kv_rows;
    for (int e = threadIdx.x; e < 64 * D; e += 256) {
        const int tt = e / D, d = e % D, t = t0 + tt;
        tile[tt][d] = t < kv_len && t < T4 ? kc[(static_cast<long>(t) * Hkv + kv) * D + d] : 0.0f;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * D; e += 256) {
        const int d = e / 64, tt = e % 64, t = t0 + tt;
        if (t < T4) kt[(static_cast<long>(kv) * D + d) * T4 + t] = tile[tt][d];
    }
}

// s [H][M][T4] in place: row (h, m) keeps columns j < pos + m0 + m + 1, scaled (scale) and softmax-ed
// (max subtracted, exponentiated, divided by the row sum; ref:src/attention.cu:849-855 runs scale,
// causal_mask and softmax as three kernels), the others set to 0.  One workgroup per row.
__global__ __launch_bounds__(256) void causal_softmax_kernel(float* __restrict__ s, int M, int T4, float scale,
                                                             const int* __restrict__ pos, int m0) {
    __shared__ float red[4];
    const long row = blockIdx.x;
    const int m = static_cast<int>(row % M);
    const int valid = min(*pos + m0 + m + 1, T4);
    float* r = s + row * T4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float mx = -INFINITY;
    for (int j = threadIdx.x; j < valid; j += 256) mx = fmaxf(mx, r[j] * scale);
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float sum = 0.0f;
    for (int j = threadIdx.x; j < valid; j += 256) sum += expf(r[j] * scale - mx);
    sum = group_sum_t<6>(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    const float inv = 1.0f / (((red[0] + red[1]) + red[2]) + red[3]);
    for (int j = threadIdx.x; j < T4; j += 256) r[j] = j < valid ? expf(r[j] * scale - mx) * inv : 0.0f;
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

int launch_prefill_attention(const float* q, long ldq, const float* kc, const float* vc, float* ctx, int m0, int M,
                             int H, int Hkv, int D, int T4, const int* pos, float scale, float* qh, float* kt,
                             float* vh, float* sc, float* oh, hipStream_t stream) {
    if (M < 1 || D % 4 != 0 || D > kDecodeAttnSplitMaxHeadDim || T4 % 4 != 0 || T4 < 4 || H % Hkv != 0 ||
        ldq % 4 != 0)
        return kDeclined;
    auto grid4 = [](long n) { return dim3(static_cast<unsigned>((n / 4 + 255) / 256)); };
    const long nq = static_cast<long>(H) * M * D;
    hipLaunchKernelGGL(dev::heads_from_rows_kernel, grid4(nq), dim3(256), 0, stream, q, ldq, qh, M, H, D);
    hipLaunchKernelGGL(dev::k_transpose_kernel, dim3(static_cast<unsigned>((T4 + 63) / 64), Hkv), dim3(256), 0, stream,
                       kc, kt, Hkv, D, T4, pos, m0 + M);
    hipLaunchKernelGGL(dev::v_heads_kernel, grid4(static_cast<long>(Hkv) * T4 * D), dim3(256), 0, stream, vc, vh, Hkv,
                       D, T4, pos, m0 + M);
    // scores = Q K^T per KV head, [H][M][T4] (batched_matmul_gqa, ref:src/attention.cu:837-841)
    int rc = launch_gqa(qh, kt, sc, H, Hkv, M, T4, D, stream);
    if (rc != 0) return rc;
    hipLaunchKernelGGL(dev::causal_softmax_kernel, dim3(static_cast<unsigned>(static_cast<long>(H) * M)), dim3(256), 0,
                       stream, sc, M, T4, scale, pos, m0);
    // out = P V, [H][M][D] (ref:src/attention.cu:857-861)
    rc = launch_gqa(sc, vh, oh, H, Hkv, M, D, T4, stream);
    if (rc != 0) return rc;
    hipLaunchKernelGGL(dev::rows_from_heads_kernel, grid4(nq), dim3(256), 0, stream, oh, ctx, M, H, D);
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

// elementwise.hip -- the path's two elementwise neighbours as standalone
// kernels, for callers that do not fuse them into the next matmul (prefill
// batches, or any other consumer).
//
// rmsnorm_residual (ref:src/kernels/elementwise.cu:463-513): per row,
//   v = input + residual; output = v; normed = v * weight * rsqrt(mean(v^2) + eps).
//   One workgroup per row; output may alias input (each element is read
//   before it is written, by the same thread).  residual may be null.
// silu_mul (ref:src/kernels/elementwise.cu:93-99 then :300-305, the pair the
//   quantized FFN calls at ref:src/model.cu:996-997): out = silu(gate) * up.
#include "act.hpp"
#include "common.hpp"
#include "internal.hpp"
#include "split.hpp"

namespace cri {
namespace dev {

__global__ __launch_bounds__(256) void rmsnorm_residual_kernel(const float* input, const float* residual,
                                                               const float* __restrict__ weight, float* output,
                                                               float* __restrict__ normed, int n, float eps) {
    __shared__ float part[4];
    const long row = blockIdx.x;
    const float* in = input + row * n;
    const float* res = residual ? residual + row * n : nullptr;
    float* out = output + row * n;
    float* nrm = normed + row * n;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = in[i] + (res ? res[i] : 0.0f);
        out[i] = v;
        ss = __builtin_fmaf(v, v, ss);
    }
    ss = group_sum_t<6>(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float f = rms_factor(((part[0] + part[1]) + part[2]) + part[3], n, eps);
    for (int i = threadIdx.x; i < n; i += 256) nrm[i] = out[i] * weight[i] * f;
}

// Rows of up to 4096 floats, 16-byte aligned: every load of the row (input,
// residual and weight, 16 bytes each) is issued before the reduction and the
// values stay in registers, so the row takes one memory round trip (the loop
// form above re-reads `output` after the barrier).  `output` is the same; the
// sum of squares is accumulated in another order, so `normed` can differ from
// the loop form in the last bits.
__global__ __launch_bounds__(256) void rmsnorm_residual_vec_kernel(const float* input, const float* residual,
                                                                   const float* __restrict__ weight, float* output,
                                                                   float* __restrict__ normed, int n, float eps) {
    __shared__ float part[4];
    const long row = blockIdx.x;
    const float* in = input + row * n;
    const float* res = residual ? residual + row * n : nullptr;
    float* out = output + row * n;
    float* nrm = normed + row * n;
    f32x4 v[4], w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = 4 * (threadIdx.x + 256 * j);
        if (i < n) {
            v[j] = *reinterpret_cast<const f32x4*>(in + i);
            if (res) v[j] += *reinterpret_cast<const f32x4*>(res + i);
            w[j] = *reinterpret_cast<const f32x4*>(weight + i);
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = 4 * (threadIdx.x + 256 * j);
        if (i < n) {
            *reinterpret_cast<f32x4*>(out + i) = v[j];
            ss = __builtin_fmaf(v[j].x, v[j].x, ss);
            ss = __builtin_fmaf(v[j].y, v[j].y, ss);
            ss = __builtin_fmaf(v[j].z, v[j].z, ss);
            ss = __builtin_fmaf(v[j].w, v[j].w, ss);
        }
    }
    ss = group_sum_t<6>(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float f = rms_factor(((part[0] + part[1]) + part[2]) + part[3], n, eps);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = 4 * (threadIdx.x + 256 * j);
        if (i < n) *reinterpret_cast<f32x4*>(nrm + i) = v[j] * w[j] * f;
    }
}

// rmsnorm_residual_vec_kernel with the residual given as the partial sums of a decode-batch
// matmul whose K was split over workgroups (SplitSums r, no row factor; r.S = 0: no residual):
// they are added in split order (split.hpp's steps, so h_out equals what the reduction
// kernel followed by rmsnorm_residual would give), then output = h + r and normed as above.
// With row_ss, normed = v * weight without the row factor: workgroup (g, row) takes columns
// [g n / G, (g + 1) n / G) of the row (G = gridDim.x parts, more workgroups reading the partial
// sums) and writes their sum of v^2 to row_ss[16 g + row], for consumers that apply the factor
// to their fp32 outputs (SplitSums.ssq).  Without it G = 1.  Parts of up to 4096 floats,
// 16-byte aligned.  output may be h (each thread reads its elements before writing them).
__global__ __launch_bounds__(256) void split_norm_kernel(const float* h, const SplitSums r,
                                                         const float* __restrict__ weight, float* output,
                                                         float* __restrict__ normed, int n, float eps,
                                                         float* __restrict__ row_ss) {
    __shared__ float part[4];
    const long row = blockIdx.y;
    const int cw = n / static_cast<int>(gridDim.x), c0 = static_cast<int>(blockIdx.x) * cw;
    f32x4 v[4], w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int o = 4 * (threadIdx.x + 256 * j), i = c0 + o;
        if (o < cw) {
            v[j] = *reinterpret_cast<const f32x4*>(h + row * n + i);
            if (r.S) v[j] += split_sum4_any(r.part + row * r.N + i, r.stride, r.S);
            w[j] = *reinterpret_cast<const f32x4*>(weight + i);
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int o = 4 * (threadIdx.x + 256 * j), i = c0 + o;
        if (o < cw) {
            *reinterpret_cast<f32x4*>(output + row * n + i) = v[j];
            ss = __builtin_fmaf(v[j].x, v[j].x, ss);
            ss = __builtin_fmaf(v[j].y, v[j].y, ss);
            ss = __builtin_fmaf(v[j].z, v[j].z, ss);
            ss = __builtin_fmaf(v[j].w, v[j].w, ss);
        }
    }
    ss = group_sum_t<6>(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float sum = ((part[0] + part[1]) + part[2]) + part[3];
    const float f = row_ss ? 1.0f : rms_factor(sum, n, eps);
    if (row_ss && threadIdx.x == 0) row_ss[16 * blockIdx.x + row] = sum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int o = 4 * (threadIdx.x + 256 * j), i = c0 + o;
        if (o < cw) {
            const f32x4 x = v[j] * w[j];
            *reinterpret_cast<f32x4*>(normed + row * n + i) = row_ss ? x : x * f;
        }
    }
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const float* gate, const float* up, float* out, long n) {
    const long stride = static_cast<long>(gridDim.x) * 256;
    for (long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride)
        out[i] = silu_f(gate[i]) * up[i];
}

}  // namespace dev

namespace detail {

int launch_rmsnorm_residual(const float* input, const float* residual, const float* weight, float* output,
                            float* normed, int rows, int n, float eps, hipStream_t stream) {
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (n <= 4096 && n % 4 == 0 && a16(input) && a16(residual) && a16(weight) && a16(output) && a16(normed))
        hipLaunchKernelGGL(dev::rmsnorm_residual_vec_kernel, dim3(rows), dim3(256), 0, stream, input, residual, weight,
                           output, normed, n, eps);
    else
        hipLaunchKernelGGL(dev::rmsnorm_residual_kernel, dim3(rows), dim3(256), 0, stream, input, residual, weight,
                           output, normed, n, eps);
    return 0;
}

int launch_split_norm(const float* h, const SplitSums& r, const float* weight, float* output, float* normed, int rows,
                      int n, float eps, hipStream_t stream, float* row_ss) {
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    const int parts = row_ss ? kNormParts : 1;
    // row_ss holds 16 rows; without it any number of rows (a prompt's)
    if (rows < 1 || rows > (row_ss ? 16 : 65535) || n % (4 * parts) != 0 || n / parts > 4096 || !a16(h) || !a16(weight) ||
        !a16(output) || !a16(normed))
        return kDeclined;
    if (r.S && (r.S > dev::kSplitMaxS || r.N % 4 != 0 || r.stride % 4 != 0 || !a16(r.part))) return kDeclined;
    hipLaunchKernelGGL(dev::split_norm_kernel, dim3(parts, rows), dim3(256), 0, stream, h, r, weight, output, normed, n,
                       eps, row_ss);
    return 0;
}

int launch_silu_mul(const float* gate, const float* up, float* out, long n, hipStream_t stream) {
    long blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(dev::silu_mul_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, gate, up, out,
                       n);
    return 0;
}

}  // namespace detail
}  // namespace cri

// ---- embedding rows from a (quantized) table -------------------------------------
#include "decode.hpp"

namespace cri {
namespace dev {

// One workgroup per token: out[i][k] = decode(table row ids[i], k), the
// reference's per-element dequant (so bit-identical to dequantize + gather).
// U elements per thread (dim <= 256 U), the format fixed: every element's loads (at a
// clamped, in-bounds column) are issued before any is stored, one memory round trip for
// the row (a loop over the columns took one per element: ~7 us for one 2048-wide row).
template <int FMT, int U>
__device__ __forceinline__ void embed_row(const uint8_t* row, float* o, int dim, bool ok) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = decode_row_elem(FMT, row, min(static_cast<int>(threadIdx.x) + 256 * u, dim - 1));
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int k = threadIdx.x + 256 * u;
        if (k < dim) o[k] = ok ? v[u] : 0.0f;
    }
}

template <int FMT>
__device__ __forceinline__ void embed_row_any(const uint8_t* row, float* o, int dim, bool ok) {
    if (dim <= 256 * 8)
        embed_row<FMT, 8>(row, o, dim, ok);
    else if (dim <= 256 * 16)
        embed_row<FMT, 16>(row, o, dim, ok);
    else
        for (int k = threadIdx.x; k < dim; k += 256) o[k] = ok ? decode_row_elem(FMT, row, k) : 0.0f;
}

__global__ __launch_bounds__(256) void embedding_rows_kernel(int fmt, const uint8_t* __restrict__ table,
                                                             const int* __restrict__ ids, float* __restrict__ out,
                                                             int dim, int vocab, long rbytes) {
    const long i = blockIdx.x;
    const int id = ids[i];
    const bool ok = id >= 0 && id < vocab;
    const uint8_t* row = table + (ok ? static_cast<long>(id) : 0) * rbytes;
    float* o = out + i * dim;
    switch (fmt) {
        case kFmtQ8_0: embed_row_any<kFmtQ8_0>(row, o, dim, ok); break;
        case kFmtQ4_0: embed_row_any<kFmtQ4_0>(row, o, dim, ok); break;
        case kFmtQ5_0: embed_row_any<kFmtQ5_0>(row, o, dim, ok); break;
        case kFmtQ4_K: embed_row_any<kFmtQ4_K>(row, o, dim, ok); break;
        case kFmtQ6_K: embed_row_any<kFmtQ6_K>(row, o, dim, ok); break;
        case kFmtF16: embed_row_any<kFmtF16>(row, o, dim, ok); break;
        case kFmtF32: embed_row_any<kFmtF32>(row, o, dim, ok); break;
    }
}

}  // namespace dev

namespace detail {

int launch_embedding_rows(int fmt, const void* table, const int* ids, float* out, int n_ids, int dim, int vocab,
                          hipStream_t stream) {
    if (n_ids < 1 || dim < 1) return 0;  // the kernel reads column dim - 1
    hipLaunchKernelGGL(dev::embedding_rows_kernel, dim3(n_ids), dim3(256), 0, stream, fmt,
                       static_cast<const uint8_t*>(table), ids, out, dim, vocab, row_bytes(fmt, dim));
    return 0;
}

}  // namespace detail
}  // namespace cri

// gemv.hip -- batch-1 fused dequant GEMV, y[N] = W[N,K] x[K], for gfx950.
//
// Replaces the M == 1 case of the reference's fused kernels
// (ref:src/kernels/matmul_quant.cu:64-119 and siblings), which use one
// 32x32 thread block per 32 outputs and leave 31/32 of the lanes idle at M=1.
//
// Work decomposition (wave64):
//   * a row of K weights is cut into K/64 "units" of 64 weights;
//   * LPR = 2^lpr_log2 lanes share a row (LPR >= units per row), each lane owns
//     units {u0, u0+LPR, ...} (UPL of them) in every row it visits, so its 64*UPL
//     activations live in VGPRs for the whole kernel;
//   * a wave covers 64/LPR rows at a time and strides over rows by
//     (waves in grid) * (64/LPR), prefetching the next rows' bytes into a second
//     register set while it decodes the current ones;
//   * partial sums are reduced over the LPR lanes with DPP/swizzle and the
//     first lane of the row writes y.
// Weights are read once from HBM with dword-aligned 16-byte loads; the lanes of
// a row read adjacent bytes, so a wave's loads of one row cover whole cache lines.
#include "common.hpp"
#include "gemv_formats.hpp"
#include "internal.hpp"

namespace cri {
namespace dev {

template <class F, int UPL>
__global__ __launch_bounds__(256) void gemv_kernel(const float* __restrict__ x, const uint8_t* __restrict__ W,
                                                   float* __restrict__ y, int N, int units, long row_bytes,
                                                   int lpr_log2) {
    const int lane = threadIdx.x & 63;
    const int lpr = 1 << lpr_log2;
    const int u0 = lane & (lpr - 1);
    const int rsub = lane >> lpr_log2;
    const int rows_per_iter = 64 >> lpr_log2;
    const int gwave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int nwaves = (gridDim.x * blockDim.x) >> 6;
    const int stride = nwaves * rows_per_iter;

    typename F::Xr xr[UPL];
    int unit[UPL];
    bool valid[UPL];
#pragma unroll
    for (int u = 0; u < UPL; ++u) {
        const int un = u0 + u * lpr;
        valid[u] = un < units;
        unit[u] = valid[u] ? un : 0;  // idle lanes decode a real unit and discard it
        F::load_x(xr[u], x, unit[u]);
    }

    int base = gwave * rows_per_iter;
    if (base >= N) return;  // whole wave idle (uniform)

    // Ping-pong register sets: decode one while the next rows' bytes arrive.
    typename F::Data buf0[UPL], buf1[UPL];
    auto load_rows = [&](typename F::Data(&dst)[UPL], int b) {
        const int r = min(b + rsub, N - 1);
        const uint8_t* rp = W + static_cast<long>(r) * row_bytes;
#pragma unroll
        for (int u = 0; u < UPL; ++u) F::load(dst[u], rp, unit[u]);
    };
    auto finish = [&](const typename F::Data(&src)[UPL], int b) {
        float acc = 0.0f;
#pragma unroll
        for (int u = 0; u < UPL; ++u) {
            const float p = F::dot(src[u], xr[u], unit[u]);
            acc += valid[u] ? p : 0.0f;
        }
        acc = group_sum(acc, lpr_log2);
        const int r = b + rsub;
        if (u0 == 0 && r < N) y[r] = acc;
    };
    load_rows(buf0, base);
    for (;;) {
        if (base + stride < N) load_rows(buf1, base + stride);
        finish(buf0, base);
        base += stride;
        if (base >= N) break;
        if (base + stride < N) load_rows(buf0, base + stride);
        finish(buf1, base);
        base += stride;
        if (base >= N) break;
    }
}

}  // namespace dev

namespace detail {

template <class F, int UPL>
static void launch_gemv_t(const float* x, const void* W, float* y, int N, int units, long row_bytes, int lpr_log2,
                          int blocks, hipStream_t stream) {
    hipLaunchKernelGGL((dev::gemv_kernel<F, UPL>), dim3(blocks), dim3(256), 0, stream, x,
                       static_cast<const uint8_t*>(W), y, N, units, row_bytes, lpr_log2);
}

template <class F>
static int launch_gemv_f(const float* x, const void* W, float* y, int N, int K, long row_bytes,
                         hipStream_t stream) {
    const int units = K / 64;
    int lpr_log2 = 0;
    while ((1 << lpr_log2) < units && lpr_log2 < 6) ++lpr_log2;
    const int lpr = 1 << lpr_log2;
    const int upl = (units + lpr - 1) / lpr;
    const int rows_per_iter = 64 / lpr;
    const long wave_iters = (static_cast<long>(N) + rows_per_iter - 1) / rows_per_iter;
    // Enough waves to keep ~8 per CU in flight on a 256-CU part, but give each
    // wave several rows so the activation load is amortised.
    long waves = wave_iters < kGemvTargetWaves ? wave_iters : kGemvTargetWaves;
    if (waves < 1) waves = 1;
    const int blocks = static_cast<int>((waves + 3) / 4);
    switch (upl) {
        case 1: launch_gemv_t<F, 1>(x, W, y, N, units, row_bytes, lpr_log2, blocks, stream); break;
        case 2: launch_gemv_t<F, 2>(x, W, y, N, units, row_bytes, lpr_log2, blocks, stream); break;
        case 3:
        case 4: launch_gemv_t<F, 4>(x, W, y, N, units, row_bytes, lpr_log2, blocks, stream); break;
        default: return -1;
    }
    return 0;
}

bool gemv_supported(int fmt, int K, const void* W) {
    (void)fmt;
    if (K % 64 != 0 || K / 64 > 256) return false;
    return (reinterpret_cast<uintptr_t>(W) & 3u) == 0;  // dword-aligned vector loads
}

int launch_gemv(int fmt, const float* x, const void* W, float* y, int N, int K, hipStream_t stream) {
    switch (fmt) {
        case kFmtQ8_0: return launch_gemv_f<dev::GemvQ8_0>(x, W, y, N, K, (K / 32) * 34L, stream);
        case kFmtQ4_0: return launch_gemv_f<dev::GemvQ4_0>(x, W, y, N, K, (K / 32) * 18L, stream);
        case kFmtQ5_0: return launch_gemv_f<dev::GemvQ5_0>(x, W, y, N, K, (K / 32) * 22L, stream);
        case kFmtQ4_K: return launch_gemv_f<dev::GemvQ4K>(x, W, y, N, K, (K / 256) * 144L, stream);
        case kFmtQ6_K: return launch_gemv_f<dev::GemvQ6K>(x, W, y, N, K, (K / 256) * 210L, stream);
        case kFmtF16: return launch_gemv_f<dev::GemvF16>(x, W, y, N, K, K * 2L, stream);
        case kFmtF32: return launch_gemv_f<dev::GemvF32>(x, W, y, N, K, K * 4L, stream);
    }
    return -1;
}

}  // namespace detail
}  // namespace cri

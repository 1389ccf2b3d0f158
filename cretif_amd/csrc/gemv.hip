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
//
// MODE (see ActIn): the activations are computed while staged -- SwiGLU of the
// gate/up outputs, or RMSNorm of hidden + residual (the row factor multiplies
// y, the workgroup-wide sum of squares is reduced through LDS).
#include <atomic>
#include <type_traits>

#include "act.hpp"
#include "common.hpp"
#include "gemv_formats.hpp"
#include "internal.hpp"
#include "rope.hpp"

namespace cri {
namespace dev {

// PREF row-groups of weight bytes are kept in flight per wave: a wave issues
// the loads of its first PREF row-groups before anything else, then stages
// the activations, so the HBM latency of the weights overlaps the activation
// fetch; afterwards every decoded row-group is immediately replaced by the
// row-group PREF steps ahead.
// The activation prologue comes last in the arguments (the first 16 argument
// dwords are preloaded into SGPRs; P.a still falls inside them).
// MR activation rows (1, or 2 for plain activations): each decoded unit of
// weights is multiplied with both rows, so a batch of two streams the weights once.
// Workgroup row blockIdx.y takes activation rows MR y .. MR y + MR - 1 of mrows
// (past the last row: the last row again, not stored).
// ROPE: the fused q/k/v projection of one token (RopeOut).  A wave's rows b .. b + 64 / LPR - 1
// start at an even b (rows per iteration and the stride are even for LPR <= 32), so the
// rotated pair (2i, 2i + 1) sits in lane groups rsub and rsub ^ 1, one shuffle apart; the
// rotation is the RoPE kernel's (same table, products rounded separately).
// KSPLIT: K is cut into gridDim.y parts; workgroup row blockIdx.y takes columns
// [K blockIdx.y, K (blockIdx.y + 1)) of the weights (K, units: one part's) and of the
// activations, and writes its partial sums to y + blockIdx.y N.
// BLK: threads per workgroup (256 or 512); every workgroup stages the whole activation vector.
template <class F, int UPL, int PREF, int MODE, int MR = 1, bool ROPE = false, bool KSPLIT = false, int BLK = 256>
__global__ __launch_bounds__(BLK) void gemv_kernel(const uint8_t* __restrict__ W, float* __restrict__ y, int N, int K,
                                                   int units, long row_bytes, int lpr_log2, int nblocks,
                                                   const ActIn Pin, int mrows, const RopeOut R) {
    constexpr bool kRms = MODE == kActRMSNorm || MODE == kActRMSNormS;
    static_assert(MR == 1 || MODE == kActPlain, "two activation rows: plain activations only");
    static_assert(!ROPE || (MR == 1 && kRms), "RoPE epilogue: the one-row RMSNorm GEMV");
    static_assert(!KSPLIT || (MR == 1 && !kRms && !ROPE), "K split: one row, no row factor");
    ActIn P = Pin;
    const int kp = KSPLIT ? static_cast<int>(blockIdx.y) : 0;
    if constexpr (KSPLIT) {
        P.a += static_cast<long>(kp) * K;
        if (P.b) P.b += static_cast<long>(kp) * K;
        y += static_cast<long>(kp) * N;
    }
    extern __shared__ float xs[];  // MR x K activations (padded, xpad), staged once per workgroup (+ one partial sum per wave)
    const int lane = threadIdx.x & 63;
    const int lpr = 1 << lpr_log2;
    const int u0 = lane & (lpr - 1);
    const int rsub = lane >> lpr_log2;
    const int rows_per_iter = 64 >> lpr_log2;
    // the weight addresses depend only on arguments among the first 16 dwords (preloaded into
    // SGPRs) and on compile-time constants: no hidden argument (blockDim, gridDim) is read
    const int gwave = (static_cast<int>(blockIdx.x) * BLK + static_cast<int>(threadIdx.x)) >> 6;
    const int nwaves = (nblocks * BLK) >> 6;
    const int stride = nwaves * rows_per_iter;  // rows between a wave's consecutive row-groups

    int unit[UPL], wunit[UPL];  // unit inside the staged activations / the weight row
    bool valid[UPL];
#pragma unroll
    for (int u = 0; u < UPL; ++u) {
        const int un = u0 + u * lpr;
        valid[u] = un < units;
        unit[u] = valid[u] ? un : 0;  // idle lanes decode a real unit and discard it
        wunit[u] = unit[u] + kp * units;  // a part starts on a 256-column boundary: unit % 4 is kept
    }

    // 1. activations: global -> registers (issued first, tiny), weights in flight behind them
    constexpr int kXI = 1024 / BLK;  // 16-byte activation loads per thread covering K <= 4096
    ActRaw<MODE> xv[MR][kXI];
    const int nx4 = K >> 2;
    const int xrow = xpad(K);  // LDS floats per staged activation row
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int i = 0; i < kXI; ++i) {
            const int j = threadIdx.x + BLK * i;
            if (j < nx4) act_load<MODE>(xv[m][i], P, min(MR * (KSPLIT ? 0 : static_cast<int>(blockIdx.y)) + m, mrows - 1), 4 * j, P.lda);
        }
    typename F::Data buf[PREF][UPL];
    const int base0 = gwave * rows_per_iter;
    // Row-group b past the end is a placeholder read: every lane takes unit 0 of row 0, so the
    // unconditional prefetch after a wave's last row-group costs one cache line per instruction.
    auto load_rows = [&](typename F::Data(&dst)[UPL], int b) {
        const bool real = b < N;
        const int r = min(b + rsub, N - 1);
        const uint8_t* rp = real ? W + static_cast<long>(r) * row_bytes : W;
#pragma unroll
        for (int u = 0; u < UPL; ++u) F::load(dst[u], rp, real ? wunit[u] : 0);
    };
    // Every prefetch is issued unconditionally (row-groups past the end are
    // placeholder reads): a load under a condition leaves the compiler unsure how
    // many loads are in flight, and it then waits for all of them before decoding
    // the oldest row-group.
#pragma unroll
    for (int p = 0; p < PREF; ++p) load_rows(buf[p], base0 + p * stride);

    // 2. stage activations in LDS (K <= 4096 is covered by the loads above)
    float ss = 0.0f;
    const bool write_h = blockIdx.x == 0;
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int i = 0; i < kXI; ++i) {
            const int j = threadIdx.x + BLK * i;
            if (j < nx4)
                *reinterpret_cast<f32x4*>(xs + m * xrow + xpad(4 * j)) =
                    act_finish<MODE>(xv[m][i], P, m, 4 * j, K, ss, write_h);
        }
    for (int j = threadIdx.x + 1024; j < nx4; j += BLK)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            ActRaw<MODE> raw;
            act_load<MODE>(raw, P, min(MR * (KSPLIT ? 0 : static_cast<int>(blockIdx.y)) + m, mrows - 1), 4 * j, P.lda);
            *reinterpret_cast<f32x4*>(xs + m * xrow + xpad(4 * j)) = act_finish<MODE>(raw, P, m, 4 * j, K, ss, write_h);
        }
    if constexpr (kRms) {
        ss = group_sum_t<6>(ss);
        if (lane == 0) xs[xpad(K) + (threadIdx.x >> 6)] = ss;
    }
    __syncthreads();
    float rs = 1.0f;
    if constexpr (kRms) {
        const float* part = xs + xpad(K);
        float t = part[0];
#pragma unroll
        for (int w = 1; w < BLK / 64; ++w) t += part[w];  // in wave order
        rs = rms_factor(t, K, P.eps);
    }
    typename F::Xr xr[MR][UPL];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int u = 0; u < UPL; ++u) F::load_x(xr[m][u], xs + m * xrow, unit[u]);

    // 3. stream the wave's row-groups
    auto finish = [&](const typename F::Data(&src)[UPL], int b) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float acc = 0.0f;
#pragma unroll
            for (int u = 0; u < UPL; ++u) {
                const float p = F::dot(src[u], xr[m][u], unit[u]);
                acc += valid[u] ? p : 0.0f;
            }
            acc = group_sum(acc, lpr_log2);
            const int r = b + rsub;
            const int orow = MR * (KSPLIT ? 0 : static_cast<int>(blockIdx.y)) + m;
            if constexpr (ROPE) {
                const float x = acc * rs;
                const float xp = __shfl_xor(x, 1 << lpr_log2);  // row r ^ 1 (every lane takes part)
                if (u0 == 0 && r < N) rope_out(R, y, r, x, xp);
            } else {
                if (u0 == 0 && r < N && orow < mrows)
                    y[static_cast<long>(orow) * N + r] = kRms ? acc * rs : acc;
            }
        }
    };
    for (int b = base0; b < N; b += PREF * stride) {
#pragma unroll
        for (int p = 0; p < PREF; ++p) {
            const int bp = b + p * stride;
            if (bp < N) finish(buf[p], bp);
            load_rows(buf[p], bp + PREF * stride);
        }
    }
}

}  // namespace dev

namespace detail {

template <class F, int UPL, int PREF, int MODE, int MR, bool ROPE, bool KSPLIT, int BLK>
static int launch_gemv_blk(const ActIn& act, const void* W, float* y, int N, int K, int units, long row_bytes,
                           int lpr_log2, hipStream_t stream, int mrows, const RopeOut& rope, int splits, long waves) {
    constexpr int kW = BLK / 64;  // waves per workgroup
    const int blocks = static_cast<int>((waves + kW - 1) / kW);
    constexpr bool kRms = MODE == kActRMSNorm || MODE == kActRMSNormS;
    const int lds = (MR * dev::xpad(K) + (kRms ? kW : 0)) * static_cast<int>(sizeof(float));
    if (lds > 65536) {  // beyond the default dynamic-LDS limit: raise it once per kernel and device
        constexpr int kMaxDevices = 64;
        static std::atomic<bool> ready[kMaxDevices];
        int devid = 0;
        if (hipGetDevice(&devid) != hipSuccess || devid < 0 || devid >= kMaxDevices) return kFailed;
        if (!ready[devid].load(std::memory_order_acquire)) {
            const void* fn = reinterpret_cast<const void*>(&dev::gemv_kernel<F, UPL, PREF, MODE, MR, ROPE, KSPLIT, BLK>);
            if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
                return kFailed;
            ready[devid].store(true, std::memory_order_release);
        }
    }
    const unsigned gy = KSPLIT ? static_cast<unsigned>(splits) : static_cast<unsigned>((mrows + MR - 1) / MR);
    hipLaunchKernelGGL((dev::gemv_kernel<F, UPL, PREF, MODE, MR, ROPE, KSPLIT, BLK>), dim3(blocks, gy), dim3(BLK), lds,
                       stream, static_cast<const uint8_t*>(W), y, N, K, units, row_bytes, lpr_log2, blocks, act, mrows,
                       rope);
    return 0;
}

template <class F, int UPL, int PREF, int MODE, int MR = 1, bool ROPE = false, bool KSPLIT = false>
static int launch_gemv_t(const ActIn& act, const void* W, float* y, int N, int K, int units, long row_bytes,
                          int lpr_log2, hipStream_t stream, int mrows = 1, const RopeOut& rope = RopeOut{},
                          int splits = 1) {
    const int rows_per_iter = 64 >> lpr_log2;
    const long groups = (static_cast<long>(N) + rows_per_iter - 1) / rows_per_iter;
    // one wave per PREF row-groups (all of a small matrix is requested at once),
    // capped at the resident-wave budget of the GPU for large N.  With one unit
    // per lane and no more row groups than that budget, one wave per row group
    // instead: the short matrices of a decode step (Q6_K 2048 x 2048 5.23 ->
    // 4.08 us, 512 x 2048 5.14 -> 3.90, Q8_0 1536 x 576 3.11 -> 2.81) are bound
    // by each wave's serial chain, not by bytes in flight
    long waves = (UPL == 1 && (F::kSpread || groups <= kGemvTargetWaves)) ? groups : (groups + PREF - 1) / PREF;
    const long budget = KSPLIT ? kGemvTargetWaves / splits : kGemvTargetWaves;  // over all K parts
    if (waves > budget) waves = budget;
    // 512-thread workgroups (one per CU at the wave budget, so each CU stages the activations
    // once) for the plain GEMVs that measured faster that way: Q8_0 at 2048 waves (8192 x 2048
    // 5.90 -> 5.52 us) and the long activation vectors (2048 x 8192 Q4_K 6.44 -> 6.24 us); Q4_K
    // 8192 x 2048 is even, short matrices (fewer CUs in use) and the RMSNorm prologue are slower
    // (at most two units per lane and not FP32: wider variants spill at 256 registers per lane)
    if constexpr (MODE == kActPlain && MR == 1 && !ROPE && !KSPLIT && UPL <= 2 && !std::is_same<F, dev::GemvF32>::value)
        if (waves >= kGemvTargetWaves && (std::is_same<F, dev::GemvQ8_0>::value || K >= 4096))
            return launch_gemv_blk<F, UPL, PREF, MODE, MR, ROPE, KSPLIT, 512>(act, W, y, N, K, units, row_bytes,
                                                                               lpr_log2, stream, mrows, rope, splits,
                                                                               waves);
    return launch_gemv_blk<F, UPL, PREF, MODE, MR, ROPE, KSPLIT, 256>(act, W, y, N, K, units, row_bytes, lpr_log2,
                                                                       stream, mrows, rope, splits, waves);
}

template <class F, int MODE, int MR = 1>
static int launch_gemv_f(const ActIn& x, const void* W, float* y, int N, int K, long row_bytes,
                         hipStream_t stream, int mrows = 1) {
    const int units = K / 64;
    int lpr_log2 = 0;
    while ((1 << lpr_log2) < units && lpr_log2 < 6) ++lpr_log2;
    // Q4_K, Q4_0, Q5_0 on long matrices: 16 lanes per row, two units each (fewer lanes to reduce
    // over, twice the rows per wave iteration)
    if (F::kPairUnits && MR == 1 && units == 32 && N >= 8192) lpr_log2 = 4;
    const int lpr = 1 << lpr_log2;
    const int upl = (units + lpr - 1) / lpr;
    switch (upl) {
        case 1:
            // one row group per wave (a short matrix): nothing to prefetch behind it
            if constexpr (F::kPref1 > 1)
                if (static_cast<long>(N) <= kGemvTargetWaves * (64 >> lpr_log2))
                    return launch_gemv_t<F, 1, 1, MODE, MR>(x, W, y, N, K, units, row_bytes, lpr_log2, stream, mrows);
            return launch_gemv_t<F, 1, F::kPref1, MODE, MR>(x, W, y, N, K, units, row_bytes, lpr_log2, stream, mrows);
        case 2:
            if constexpr (MR > 1) return -1;  // two activation rows: one unit per lane (K <= 4096)
            // one row group in flight: fewer registers, twice the waves (2048 x 8192: Q8_0 7.68 ->
            // 7.36 us, Q4_0 6.27 -> 6.09, Q5_0 7.24 -> 6.93, FP16 11.13 -> 10.25 against two)
            return launch_gemv_t<F, 2, 1, MODE>(x, W, y, N, K, units, row_bytes, lpr_log2, stream);
        case 3:
        case 4:
            if constexpr (MR > 1) return -1;
            return launch_gemv_t<F, 4, 1, MODE>(x, W, y, N, K, units, row_bytes, lpr_log2, stream);
        default: return -1;
    }
    return 0;
}

bool gemv_supported(int fmt, int K, const void* W) {
    (void)fmt;
    if (K % 64 != 0 || K / 64 > 256) return false;
    return (reinterpret_cast<uintptr_t>(W) & 3u) == 0;  // dword-aligned vector loads
}

template <int MODE>
static int launch_gemv_m(int fmt, const ActIn& x, const void* W, float* y, int N, int K, hipStream_t stream) {
    switch (fmt) {
        case kFmtQ8_0: return launch_gemv_f<dev::GemvQ8_0, MODE>(x, W, y, N, K, (K / 32) * 34L, stream);
        case kFmtQ4_0: return launch_gemv_f<dev::GemvQ4_0, MODE>(x, W, y, N, K, (K / 32) * 18L, stream);
        case kFmtQ5_0: return launch_gemv_f<dev::GemvQ5_0, MODE>(x, W, y, N, K, (K / 32) * 22L, stream);
        case kFmtQ4_K: return launch_gemv_f<dev::GemvQ4K, MODE>(x, W, y, N, K, (K / 256) * 144L, stream);
        case kFmtQ6_K: return launch_gemv_f<dev::GemvQ6K, MODE>(x, W, y, N, K, (K / 256) * 210L, stream);
        case kFmtF16: return launch_gemv_f<dev::GemvF16, MODE>(x, W, y, N, K, K * 2L, stream);
        case kFmtF32:
            if constexpr (MODE == kActPlain) return launch_gemv_f<dev::GemvF32, MODE>(x, W, y, N, K, K * 4L, stream);
            break;
    }
    return -1;
}

// Two activation rows (a batch of two decode tokens) for the 32-element formats and
// Q6_K: the weights are decoded once and streamed once for both rows.  K <= 4096.
// M rows (up to 16) run as ceil(M / 2) row pairs, one per grid row.
// (Q4_K and FP16 at M = 2 measured faster on the skinny MFMA kernel: 5.1 against
// 6.9 us and 8.9 against 9.7 us at 8192 x 2048.)
int launch_gemv2(int fmt, const float* x, const void* W, float* y, int M, int N, int K, hipStream_t stream) {
    const ActIn act{x, nullptr, nullptr, nullptr, K, 0.0f};
    if (K / 64 > 64 || M < 1 || M > 16) return -1;
    switch (fmt) {
        case kFmtQ8_0: return launch_gemv_f<dev::GemvQ8_0, kActPlain, 2>(act, W, y, N, K, (K / 32) * 34L, stream, M);
        case kFmtQ4_0: return launch_gemv_f<dev::GemvQ4_0, kActPlain, 2>(act, W, y, N, K, (K / 32) * 18L, stream, M);
        case kFmtQ5_0: return launch_gemv_f<dev::GemvQ5_0, kActPlain, 2>(act, W, y, N, K, (K / 32) * 22L, stream, M);
        case kFmtQ6_K: return launch_gemv_f<dev::GemvQ6K, kActPlain, 2>(act, W, y, N, K, (K / 256) * 210L, stream, M);
    }
    return -1;
}

int launch_gemv(int fmt, const float* x, const void* W, float* y, int N, int K, hipStream_t stream) {
    const ActIn act{x, nullptr, nullptr, nullptr, K, 0.0f};
    return launch_gemv_m<kActPlain>(fmt, act, W, y, N, K, stream);
}

// The RoPE epilogue needs each rotated pair inside one wave: at most 32 lanes per row (K <= 2048
// at one unit per lane), which also keeps one unit per lane.
template <class F>
static int launch_gemv_rope_f(const ActIn& x, const void* W, float* q_out, int N, int K, long row_bytes,
                              const RopeOut& rope, hipStream_t stream, bool split_res) {
    const int units = K / 64;
    int lpr_log2 = 0;
    while ((1 << lpr_log2) < units && lpr_log2 < 6) ++lpr_log2;
    if (units > 32 || lpr_log2 > 5) return kDeclined;
    if (split_res)
        return launch_gemv_t<F, 1, F::kPref1, kActRMSNormS, 1, true>(x, W, q_out, N, K, units, row_bytes, lpr_log2,
                                                                      stream, 1, rope);
    return launch_gemv_t<F, 1, F::kPref1, kActRMSNorm, 1, true>(x, W, q_out, N, K, units, row_bytes, lpr_log2, stream,
                                                                 1, rope);
}

// K split: one unit per lane where it fits (the part's units <= 64)
template <class F, int MODE>
static int launch_gemv_ksplit_f(const ActIn& x, const void* W, float* y, int N, int K, long row_bytes, int splits,
                                hipStream_t stream) {
    const int Ks = K / splits, units = Ks / 64;
    int lpr_log2 = 0;
    while ((1 << lpr_log2) < units && lpr_log2 < 6) ++lpr_log2;
    if (units > 64) return kDeclined;
    return launch_gemv_t<F, 1, F::kPref1, MODE, 1, false, true>(x, W, y, N, Ks, units, row_bytes, lpr_log2, stream, 1,
                                                                 RopeOut{}, splits);
}

template <int MODE>
static int launch_gemv_ksplit_m(int fmt, const ActIn& act, const void* W, float* y, int N, int K, int splits,
                                hipStream_t stream) {
    switch (fmt) {
        case kFmtQ8_0: return launch_gemv_ksplit_f<dev::GemvQ8_0, MODE>(act, W, y, N, K, (K / 32) * 34L, splits, stream);
        case kFmtQ4_0: return launch_gemv_ksplit_f<dev::GemvQ4_0, MODE>(act, W, y, N, K, (K / 32) * 18L, splits, stream);
        case kFmtQ5_0: return launch_gemv_ksplit_f<dev::GemvQ5_0, MODE>(act, W, y, N, K, (K / 32) * 22L, splits, stream);
        case kFmtQ4_K: return launch_gemv_ksplit_f<dev::GemvQ4K, MODE>(act, W, y, N, K, (K / 256) * 144L, splits, stream);
        case kFmtQ6_K: return launch_gemv_ksplit_f<dev::GemvQ6K, MODE>(act, W, y, N, K, (K / 256) * 210L, splits, stream);
        case kFmtF16: return launch_gemv_ksplit_f<dev::GemvF16, MODE>(act, W, y, N, K, K * 2L, splits, stream);
    }
    return kDeclined;
}

int launch_gemv_ksplit(int mode, int fmt, const ActIn& act, const void* W, float* y, int N, int K, int splits,
                       hipStream_t stream) {
    if (splits < 2 || splits > kResMaxSplits || K % (256 * splits) != 0 || !gemv_supported(fmt, K, W)) return kDeclined;
    if ((dev::xpad(K / splits) + 8) * 4 > 160 * 1024) return kDeclined;
    switch (mode) {
        case kActPlain: return launch_gemv_ksplit_m<kActPlain>(fmt, act, W, y, N, K, splits, stream);
        case kActSwiGLU: return launch_gemv_ksplit_m<kActSwiGLU>(fmt, act, W, y, N, K, splits, stream);
    }
    return kDeclined;
}

int launch_gemv_rope(int fmt, const ActIn& act, const void* W, float* q_out, int N, int K, const RopeOut& rope,
                     hipStream_t stream, bool split_res) {
    if ((dev::xpad(K) + 8) * 4 > 160 * 1024 || !gemv_supported(fmt, K, W)) return kDeclined;
    if (rope.qd % 2 || rope.kvd % 2 || rope.half < 1 || rope.qd % (2 * rope.half) || rope.kvd % (2 * rope.half) ||
        N != rope.qd + 2 * rope.kvd)
        return kDeclined;
    switch (fmt) {
        case kFmtQ8_0: return launch_gemv_rope_f<dev::GemvQ8_0>(act, W, q_out, N, K, (K / 32) * 34L, rope, stream, split_res);
        case kFmtQ4_0: return launch_gemv_rope_f<dev::GemvQ4_0>(act, W, q_out, N, K, (K / 32) * 18L, rope, stream, split_res);
        case kFmtQ5_0: return launch_gemv_rope_f<dev::GemvQ5_0>(act, W, q_out, N, K, (K / 32) * 22L, rope, stream, split_res);
        case kFmtQ4_K: return launch_gemv_rope_f<dev::GemvQ4K>(act, W, q_out, N, K, (K / 256) * 144L, rope, stream, split_res);
        case kFmtQ6_K: return launch_gemv_rope_f<dev::GemvQ6K>(act, W, q_out, N, K, (K / 256) * 210L, rope, stream, split_res);
        case kFmtF16: return launch_gemv_rope_f<dev::GemvF16>(act, W, q_out, N, K, K * 2L, rope, stream, split_res);
    }
    return kDeclined;
}

int launch_gemv_act(int mode, int fmt, const ActIn& act, const void* W, float* y, int N, int K, hipStream_t stream) {
    if ((dev::xpad(K) + 8) * 4 > 160 * 1024) return -1;  // the staged activations (+ one partial sum per wave) fit in LDS
    switch (mode) {
        case kActPlain: return launch_gemv_m<kActPlain>(fmt, act, W, y, N, K, stream);
        case kActSwiGLU: return launch_gemv_m<kActSwiGLU>(fmt, act, W, y, N, K, stream);
        case kActRMSNorm: return launch_gemv_m<kActRMSNorm>(fmt, act, W, y, N, K, stream);
        case kActRMSNormS: return launch_gemv_m<kActRMSNormS>(fmt, act, W, y, N, K, stream);
    }
    return -1;
}

}  // namespace detail
}  // namespace cri

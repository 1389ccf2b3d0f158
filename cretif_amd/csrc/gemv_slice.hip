// gemv_slice.hip -- batch-1 GEMV y[N] = W[N,K] x[K] with K sliced over the waves of a
// workgroup (four for Q4_K, eight for the 32-element formats), for Q4_K weights and Q8_0, Q4_0
// and Q5_0 ones at K = 8192: the C ABI's M = 1 case (plain activations, and SwiGLU ones at
// K = 8192, the FFN down projection).
//
// Replaces the M == 1 case of ref:src/kernels/matmul_quant.cu:309-397 (one 32x32 thread
// block per 32 outputs, 31/32 of the lanes idle at M = 1).
//
// Work decomposition (wave64, W = F::kWaves waves per workgroup):
//   * a workgroup owns R consecutive rows; wave w owns K slice [K w / W, K (w + 1) / W) of
//     all of them, so the W waves' partial sums meet once, through LDS, at the end;
//   * a "piece" is 32 weights of one row (half of a 64-element Q4_K chunk: 16 bytes of qs,
//     low nibbles = 16 elements, high nibbles = the 16 elements 32 further on; one Q8_0,
//     Q4_0 or Q5_0 block); L = K / (32 W) lanes share a row (L pieces = one K slice), so a wave takes
//     64 / L rows per step and IT steps (R = IT * 64 / L);
//   * a lane's 32 activations stay in VGPRs for all of its IT rows (computed from the
//     prologue's inputs when MODE is not plain), loaded straight from global memory: every
//     wave of the grid reads the same K floats, which the L1/L2 serve; LDS staging, with its
//     barrier and 4x-replicated reads, measured slower;
//   * every weight load of the wave is issued at kernel entry, before the activation loads
//     (which are L2 hits and would otherwise delay the HBM requests behind them), two row
//     steps ahead of them so the first steps' decode can start while later rows stream in;
//   * every argument is a plain scalar in the first kernel-argument dwords, which the
//     hardware preloads into SGPRs: no load waits on a kernel-argument fetch (an aggregate
//     argument is fetched with scalar loads), and the kernel reads no hidden argument
//     (blockDim, gridDim) at all.
// Per piece a lane loads the 16-byte super-block header (d, dmin, 12 scale bytes; the 8 lanes
// of one super-block read the same 16 bytes in one instruction) and its 16 quant bytes, both
// 16-byte aligned; consecutive lanes read consecutive quant bytes.
//
// MODE (see ActIn): kActPlain or kActSwiGLU.  Each lane computes the prologue of its own 32
// activations, so at L < 64 lanes per row the 64 / L row groups of a wave compute the same
// values; with an RMSNorm prologue (three loads per activation, a workgroup reduction) that
// costs more than staging once per workgroup, and the batch-1 GEMV of gemv.hip takes those.
#include "act.hpp"
#include "common.hpp"
#include "internal.hpp"

namespace cri {
namespace dev {

// Q4_K piece p of a row: super-block p >> 3, chunk j = (p >> 1) & 3, half h = p & 1.  Quant
// bytes 16 + 32 j + 16 h .. +16 of the super-block; low nibble of byte i = element
// 64 j + 16 h + i, high nibble = element 64 j + 32 + 16 h + i (ref:src/kernels/dequantize.cu:307-319).
// WAVES: waves per workgroup (K slices).  Four from 8192 x 2048 on (eight measured slower, 3.96
// -> 4.80 us; two 4.82 us, and 5.81 against 4.05 at 2048 x 8192); two up to 2048 x 2048, where
// they halve the number of waves (2048 x 2048 2.70 -> 2.57 us, 512 x 2048 2.15 -> 2.09).
template <int WAVES>
struct SliceQ4KW {
    static constexpr int kFmt = kFmtQ4_K;
    static constexpr int kXb = 32;        // xb: elements x_first + 32 .. +16
    static constexpr int kMaxSteps = 8;   // row steps per workgroup at most
    static constexpr int kWaves = WAVES;
    struct Data {
        u32x4 hd, q;
    };
    static __device__ __forceinline__ int x_first(int p) { return (p >> 3) * 256 + 64 * ((p >> 1) & 3) + 16 * (p & 1); }
    static __device__ __forceinline__ void load(Data& d, const uint8_t* __restrict__ row, int p) {
        const uint8_t* sb = row + (p >> 3) * 144;
        d.hd = ld_u32x4(sb);
        d.q = ld_u32x4(sb + 16 + 32 * ((p >> 1) & 3) + 16 * (p & 1));
    }
    // sum over the piece of w * x, xa = elements x_first .. +16, xb = x_first + 32 .. +16,
    // sa / sb their sums (for the -dmin * mn term)
    static __device__ __forceinline__ float dot(const Data& d, const float (&xa)[16], const float (&xb)[16],
                                                float sa, float sb, int p) {
        // 6-bit scale and min of sub-blocks 2j (low nibbles) and 2j + 1 (high nibbles)
        // (ref:src/kernels/dequantize.cu:298-305):
        //   j < 2:  sc = s[sb] & 63, mn = s[sb + 4] & 63
        //   j >= 2: sc = (s[sb + 4] & 15) | (s[sb - 4] >> 6) << 4, mn = (s[sb + 4] >> 4) | (s[sb] >> 6) << 4
        const int j = (p >> 1) & 3;
        const bool low = j < 2;
        const uint32_t o = (j & 1) * 16;
        const uint32_t h1 = d.hd.y, h2 = d.hd.z, h3 = d.hd.w;
        const uint32_t a_sc = low ? h1 : h3;
        const uint32_t a_mn = low ? h2 : h3;
        const uint32_t wa = low ? 6 : 4;
        const uint32_t wb = low ? 0 : 2;
        const uint32_t om = low ? 0 : 4;
        const uint32_t sc_lo = ubfe(a_sc, o, wa) | (ubfe(h1, o + 6, wb) << 4);
        const uint32_t mn_lo = ubfe(a_mn, o + om, wa) | (ubfe(h2, o + 6, wb) << 4);
        const uint32_t sc_hi = ubfe(a_sc, o + 8, wa) | (ubfe(h1, o + 14, wb) << 4);
        const uint32_t mn_hi = ubfe(a_mn, o + 8 + om, wa) | (ubfe(h2, o + 14, wb) << 4);
        // nibbles as binary16 subnormals q * 2^-24 in the halves of a dword: one v_fma_mix_f32 each
        float l0 = 0.f, l1 = 0.f, g0 = 0.f, g1 = 0.f;
        const uint32_t q[4] = {d.q.x, d.q.y, d.q.z, d.q.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t w = q[t], u = w >> 8;
            const uint32_t a = w & 0x000F000Fu;  // low nibbles of bytes 4t, 4t + 2
            const uint32_t b = w & 0x00F000F0u;  // 16 * high nibbles of bytes 4t, 4t + 2
            const uint32_t e = u & 0x000F000Fu;  // low nibbles of bytes 4t + 1, 4t + 3
            const uint32_t f = u & 0x00F000F0u;  // 16 * high nibbles of bytes 4t + 1, 4t + 3
            l0 = __builtin_fmaf(h_lo(a), xa[4 * t + 0], l0);
            l1 = __builtin_fmaf(h_lo(e), xa[4 * t + 1], l1);
            l0 = __builtin_fmaf(h_hi(a), xa[4 * t + 2], l0);
            l1 = __builtin_fmaf(h_hi(e), xa[4 * t + 3], l1);
            g0 = __builtin_fmaf(h_lo(b), xb[4 * t + 0], g0);
            g1 = __builtin_fmaf(h_lo(f), xb[4 * t + 1], g1);
            g0 = __builtin_fmaf(h_hi(b), xb[4 * t + 2], g0);
            g1 = __builtin_fmaf(h_hi(f), xb[4 * t + 3], g1);
        }
        const float dd = h_lo(d.hd.x), dmin = h_hi(d.hd.x);
        const float t = (l0 + l1) * static_cast<float>(sc_lo) + (g0 + g1) * (static_cast<float>(sc_hi) * 0.0625f);
        const float m = static_cast<float>(mn_lo) * sa + static_cast<float>(mn_hi) * sb;
        return (dd * kTwo24) * t - dmin * m;
    }
};
using SliceQ4K = SliceQ4KW<4>;
using SliceQ4K2 = SliceQ4KW<2>;

// Q8_0 piece p of a row: block p (34 bytes: fp16 d, 32 int8 quants; ref:src/kernels/dequantize.cu:60-70),
// elements 32 p .. +32.  Blocks start at 34 p: dword aligned for even p, two bytes past a dword
// boundary for odd p, so a lane loads the nine dwords from the one holding d (34 p - 2 (p & 1)) and
// realigns the quants in registers; with an even number of blocks per row the nine dwords end
// inside the row.  Quants enter as q + 128 (bytes xor 0x80, converted with v_cvt_f32_ubyteN) and
// 128 sum(x) comes off at the end.
struct SliceQ80 {
    static constexpr int kFmt = kFmtQ8_0;
    static constexpr int kXb = 16;  // xb: elements x_first + 16 .. +16
    // 2048 x 8192, same box: eight waves (K slices of 1024) 6.12 us against 6.86 at four; four
    // row steps 6.12, eight 6.12, two 6.74 (the batch-1 GEMV: 7.42)
    static constexpr int kMaxSteps = 4;
    static constexpr int kWaves = 8;
    struct Data {
        u32x4 a, b;
        uint32_t c;
    };
    static __device__ __forceinline__ int x_first(int p) { return 32 * p; }
    static __device__ __forceinline__ void load(Data& d, const uint8_t* __restrict__ row, int p) {
        const uint8_t* s = row + 34 * p - 2 * (p & 1);
        d.a = ld_u32x4(s);
        d.b = ld_u32x4(s + 16);
        d.c = ld_u32(s + 32);
    }
    static __device__ __forceinline__ float dot(const Data& d, const float (&xa)[16], const float (&xb)[16],
                                                float sa, float sb, int p) {
        const bool odd = p & 1;
        const uint32_t D[9] = {d.a.x, d.a.y, d.a.z, d.a.w, d.b.x, d.b.y, d.b.z, d.b.w, d.c};
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            // quant bytes 4 k .. 4 k + 3 of the block (block bytes 2 + 4 k ..)
            const uint32_t q = (odd ? D[k + 1] : align_bytes(D[k + 1], D[k], 2)) ^ 0x80808080u;
            const float* x = k < 4 ? xa + 4 * k : xb + 4 * (k - 4);
            s0 = __builtin_fmaf(static_cast<float>(q & 0xFFu), x[0], s0);
            s1 = __builtin_fmaf(static_cast<float>((q >> 8) & 0xFFu), x[1], s1);
            s0 = __builtin_fmaf(static_cast<float>((q >> 16) & 0xFFu), x[2], s0);
            s1 = __builtin_fmaf(static_cast<float>(q >> 24), x[3], s1);
        }
        const float dd = odd ? h_hi(D[0]) : h_lo(D[0]);
        return dd * ((s0 + s1) - 128.0f * (sa + sb));
    }
};

// Q4_0 piece p of a row: block p (18 bytes: fp16 d, 16 quant bytes; ref:src/kernels/dequantize.cu:73-101),
// element i <- quant byte i / 2, low nibble for even i; x = d (q - 8).  Blocks start at 18 p: dword
// aligned for even p, two bytes off for odd p; a lane loads the five dwords from the one holding d
// (the extra two bytes of an even block are the next block's d: rows hold an even number of blocks).
struct SliceQ40 {
    static constexpr int kFmt = kFmtQ4_0;
    static constexpr int kXb = 16;
    static constexpr int kMaxSteps = 8;
    static constexpr int kWaves = 8;  // 2048 x 8192: 4.67 us at eight, 5.20 at four (the batch-1 GEMV: 5.71)
    struct Data {
        u32x4 a;
        uint32_t b;
    };
    static __device__ __forceinline__ int x_first(int p) { return 32 * p; }
    static __device__ __forceinline__ void load(Data& d, const uint8_t* __restrict__ row, int p) {
        const uint8_t* s = row + 18 * p - 2 * (p & 1);
        d.a = ld_u32x4(s);
        d.b = ld_u32(s + 16);
    }
    static __device__ __forceinline__ float dot(const Data& d, const float (&xa)[16], const float (&xb)[16],
                                                float sa, float sb, int p) {
        const bool odd = p & 1;
        const uint32_t D[5] = {d.a.x, d.a.y, d.a.z, d.a.w, d.b};
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            // quant bytes 4 t .. 4 t + 3: elements 8 t + 2 b (low nibble) and 8 t + 2 b + 1 (high)
            const uint32_t w = odd ? D[t + 1] : align_bytes(D[t + 1], D[t], 2);
            const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
            const float* x = t < 2 ? xa + 8 * t : xb + 8 * (t - 2);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                s0 = __builtin_fmaf(ubyte(lo, b), x[2 * b], s0);
                s1 = __builtin_fmaf(ubyte(hi, b), x[2 * b + 1], s1);
            }
        }
        const float dd = odd ? h_hi(D[0]) : h_lo(D[0]);
        return dd * ((s0 + s1) - 8.0f * (sa + sb));
    }
};

// Q5_0 piece p of a row: block p (22 bytes: fp16 d, qh[4], qs[16]; ref:src/kernels/dequantize.cu:126-165),
// element i: low nibble of qs[i] (i < 16) or high nibble of qs[i - 16], bit i of qh as bit 4;
// x = d (q - 16).  Blocks start at 22 p (two bytes off for odd p): six dwords from the one holding d.
struct SliceQ50 {
    static constexpr int kFmt = kFmtQ5_0;
    static constexpr int kXb = 16;
    static constexpr int kMaxSteps = 8;
    static constexpr int kWaves = 8;  // 2048 x 8192: 5.08 us at eight, 7.11 at four (the batch-1 GEMV: 6.51)
    struct Data {
        u32x4 a;
        uint32_t b, c;
    };
    static __device__ __forceinline__ int x_first(int p) { return 32 * p; }
    static __device__ __forceinline__ void load(Data& d, const uint8_t* __restrict__ row, int p) {
        const uint8_t* s = row + 22 * p - 2 * (p & 1);
        d.a = ld_u32x4(s);
        d.b = ld_u32(s + 16);
        d.c = ld_u32(s + 20);
    }
    static __device__ __forceinline__ float dot(const Data& d, const float (&xa)[16], const float (&xb)[16],
                                                float sa, float sb, int p) {
        const bool odd = p & 1;
        const uint32_t D[6] = {d.a.x, d.a.y, d.a.z, d.a.w, d.b, d.c};
        const uint32_t qh = odd ? D[1] : align_bytes(D[1], D[0], 2);
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t w = odd ? D[t + 2] : align_bytes(D[t + 2], D[t + 1], 2);
            const uint32_t nlo = ubfe(qh, 4 * t, 4), nhi = ubfe(qh, 16 + 4 * t, 4);
            // the four high bits spread to bit 4 of each byte (no carries between the copies)
            const uint32_t lo = (w & 0x0F0F0F0Fu) | ((nlo * 0x02040810u) & 0x10101010u);
            const uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) | ((nhi * 0x02040810u) & 0x10101010u);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                s0 = __builtin_fmaf(ubyte(lo, b), xa[4 * t + b], s0);
                s1 = __builtin_fmaf(ubyte(hi, b), xb[4 * t + b], s1);
            }
        }
        const float dd = odd ? h_hi(D[0]) : h_lo(D[0]);
        return dd * ((s0 + s1) - 16.0f * (sa + sb));
    }
};

constexpr int kSliceMaxWaves = 8;  // waves per workgroup (F::kWaves), one K slice each
constexpr int kSliceXAfter = 2;    // row steps whose weight loads go before the activation loads

// The prologue's pointers and integers are separate scalar arguments (16 dwords up to kn), all
// preloaded into SGPRs: an aggregate argument is fetched with scalar loads, and activation loads
// waiting on that fetch would hold back the weight loads issued after them.
template <class F, int LG, int IT, int MODE>
__global__ __launch_bounds__(64 * F::kWaves) void slice_gemv_kernel(const uint8_t* __restrict__ W,
                                                                      float* __restrict__ y,
                                                                      const float* __restrict__ a,
                                                                      const float* __restrict__ b, int N,
                                                                      int row_bytes) {
    static_assert(MODE == kActPlain || MODE == kActSwiGLU, "plain or SwiGLU prologue");
    constexpr int L = 1 << LG, RPI = 64 / L, RW = IT * RPI;  // lanes per row, rows per step, rows per workgroup
    constexpr int kSliceWaves = F::kWaves;
    static_assert(kSliceWaves <= kSliceMaxWaves, "waves per workgroup");
    constexpr int K = kSliceWaves * L * 32;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int sub = lane & (L - 1), rsub = lane >> LG;
    const int p = wv * L + sub;  // piece index along the row
    const int row0 = blockIdx.x * RW;

    const ActIn P{a, b, nullptr, nullptr, 0, 0.0f};  // lda is not read: one activation row
    float xa[16], xb[16];
    float ss = 0.0f;  // (unused without RMSNorm)
    auto xload = [&]() {
        const int k0 = F::x_first(p);
        ActRaw<MODE> ra[4], rb[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            act_load<MODE>(ra[v], P, 0, k0 + 4 * v, P.lda);
            act_load<MODE>(rb[v], P, 0, k0 + F::kXb + 4 * v, P.lda);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const f32x4 a = act_finish<MODE>(ra[v], P, 0, k0 + 4 * v, K, ss, false);
            const f32x4 b = act_finish<MODE>(rb[v], P, 0, k0 + F::kXb + 4 * v, K, ss, false);
            xa[4 * v] = a.x; xa[4 * v + 1] = a.y; xa[4 * v + 2] = a.z; xa[4 * v + 3] = a.w;
            xb[4 * v] = b.x; xb[4 * v + 1] = b.y; xb[4 * v + 2] = b.z; xb[4 * v + 3] = b.w;
        }
    };
    typename F::Data buf[IT];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        if (it == kSliceXAfter) xload();
        // rows past the end read row N - 1 again (unconditional loads keep every request in flight)
        const uint8_t* rp = W + static_cast<long>(min(row0 + it * RPI + rsub, N - 1)) * row_bytes;
        F::load(buf[it], rp, p);
    }
    if constexpr (IT <= kSliceXAfter) xload();

    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        sa += xa[v];
        sb += xb[v];
    }
    float acc[IT];
#pragma unroll
    for (int it = 0; it < IT; ++it) acc[it] = group_sum_t<LG>(F::dot(buf[it], xa, xb, sa, sb, p));

    __shared__ float red[kSliceWaves][RW];
#pragma unroll
    for (int it = 0; it < IT; ++it)
        if (sub == 0) red[wv][it * RPI + rsub] = acc[it];
    __syncthreads();
    if (threadIdx.x < RW) {
        const int t = threadIdx.x;
        float v = red[0][t];
#pragma unroll
        for (int w = 1; w < kSliceWaves; ++w) v += red[w][t];  // in wave order
        if (row0 + t < N) y[row0 + t] = v;
    }
}

}  // namespace dev

namespace detail {

namespace {

// lanes per row = K / (32 waves) (K in {1024, 2048, 4096, 8192}); log2 of it, or -1
int slice_lg(int K, int waves) {
    int lg = -1;
    switch (K) {
        case 1024: lg = 5; break;
        case 2048: lg = 6; break;
        case 4096: lg = 7; break;
        case 8192: lg = 8; break;
    }
    if (lg < 0) return -1;
    lg -= waves == 8 ? 3 : (waves == 4 ? 2 : 1);  // K / 32 pieces over the waves
    return lg >= 2 && lg <= 6 ? lg : -1;
}

// Row steps per wave: IT rows per lane share one activation load, so the grid's activation reads
// are N K / (IT 64 / L) floats; IT = 8 measured fastest at the Llama-3.2-1B shapes (8192 x 2048:
// 256 workgroups of 32 rows, 3.94 us against 4.56 us on the unsliced GEMV; 2048 x 8192: 256 of
// 8 rows, 4.71 against 6.2 us).  Fewer for short matrices, so that ~256 workgroups still run.
int slice_steps(int N, int LG, int max_steps) {
    const long rows_per_step = 64 >> LG;
    int it = max_steps;
    while (it > 1 && (static_cast<long>(N) + it * rows_per_step - 1) / (it * rows_per_step) < 256) it >>= 1;
    return it;
}

template <class F, int LG, int IT, int MODE>
int launch_slice_t(const ActIn& act, const void* W, float* y, int N, int K, hipStream_t s) {
    constexpr int RW = IT * (64 >> LG);
    const int blocks = (N + RW - 1) / RW;
    const int rbytes = static_cast<int>(cri::row_bytes(F::kFmt, K));
    hipLaunchKernelGGL((dev::slice_gemv_kernel<F, LG, IT, MODE>), dim3(blocks), dim3(64 * F::kWaves), 0, s,
                       static_cast<const uint8_t*>(W), y, act.a, act.b, N, rbytes);
    return 0;
}

template <class F, int LG, int MODE>
int launch_slice_it(const ActIn& act, const void* W, float* y, int N, int K, hipStream_t s) {
    switch (slice_steps(N, LG, F::kMaxSteps)) {
        case 8: return launch_slice_t<F, LG, 8, MODE>(act, W, y, N, K, s);
        case 4: return launch_slice_t<F, LG, 4, MODE>(act, W, y, N, K, s);
        case 2: return launch_slice_t<F, LG, 2, MODE>(act, W, y, N, K, s);
        default: return launch_slice_t<F, LG, 1, MODE>(act, W, y, N, K, s);
    }
}

template <class F, int MODE>
int launch_slice_m(const ActIn& act, const void* W, float* y, int N, int K, hipStream_t s) {
    switch (slice_lg(K, F::kWaves)) {
        case 2: return launch_slice_it<F, 2, MODE>(act, W, y, N, K, s);
        case 3: return launch_slice_it<F, 3, MODE>(act, W, y, N, K, s);
        case 4: return launch_slice_it<F, 4, MODE>(act, W, y, N, K, s);
        case 5: return launch_slice_it<F, 5, MODE>(act, W, y, N, K, s);
        case 6: return launch_slice_it<F, 6, MODE>(act, W, y, N, K, s);
    }
    return kDeclined;
}

template <class F>
int launch_slice_f(int mode, const ActIn& act, const void* W, float* y, int N, int K, hipStream_t s) {
    switch (mode) {
        case kActPlain: return launch_slice_m<F, kActPlain>(act, W, y, N, K, s);
        case kActSwiGLU:
            // the up rows ld floats after the gate rows: the kernel reads one row, so ld is not needed
            return launch_slice_m<F, kActSwiGLU>(act, W, y, N, K, s);
    }
    return kDeclined;
}

}  // namespace

// Q8_0 only at K = 8192: at 8192 x 2048 the batch-1 GEMV of gemv.hip (two blocks per lane) is
// faster (5.51 us against 5.96 at four row steps, same box)
// Q8_0, Q4_0 and Q5_0 only at K = 8192 (the FFN down shape): at 8192 x 2048 the batch-1 GEMV of
// gemv.hip is faster for them (same box: Q8_0 5.18 against 5.96 / 6.06 us at four / eight waves,
// Q4_0 4.13 against 4.77, Q5_0 4.92 against 5.11 at eight waves)
static bool slice_fmt(int fmt, int K) {
    switch (fmt) {
        case kFmtQ4_K: return true;
        case kFmtQ8_0:
        case kFmtQ4_0:
        case kFmtQ5_0: return K == 8192;
    }
    return false;
}
// Q4_K up to 2048 x 2048 on two waves per workgroup
static bool q4k_two_waves(int N, int K) { return N <= 2048 && K <= 2048; }
static int slice_waves(int fmt, int N, int K) {
    switch (fmt) {
        case kFmtQ8_0: return dev::SliceQ80::kWaves;
        case kFmtQ4_0: return dev::SliceQ40::kWaves;
        case kFmtQ5_0: return dev::SliceQ50::kWaves;
    }
    return q4k_two_waves(N, K) ? dev::SliceQ4K2::kWaves : dev::SliceQ4K::kWaves;
}

bool slice_gemv_supported(int fmt, int N, int K, const void* W) {
    return slice_fmt(fmt, K) && slice_lg(K, slice_waves(fmt, N, K)) >= 0 && (reinterpret_cast<uintptr_t>(W) & 3u) == 0;
}

int launch_slice_gemv(int mode, int fmt, const ActIn& act, const void* W, float* y, int N, int K, hipStream_t s) {
    if (!slice_gemv_supported(fmt, N, K, W)) return kDeclined;
    switch (fmt) {
        case kFmtQ4_K:
            if (q4k_two_waves(N, K)) return launch_slice_f<dev::SliceQ4K2>(mode, act, W, y, N, K, s);
            return launch_slice_f<dev::SliceQ4K>(mode, act, W, y, N, K, s);
        case kFmtQ8_0: return launch_slice_f<dev::SliceQ80>(mode, act, W, y, N, K, s);
        case kFmtQ4_0: return launch_slice_f<dev::SliceQ40>(mode, act, W, y, N, K, s);
        case kFmtQ5_0: return launch_slice_f<dev::SliceQ50>(mode, act, W, y, N, K, s);
    }
    return kDeclined;
}

}  // namespace detail
}  // namespace cri

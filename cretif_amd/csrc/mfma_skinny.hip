// mfma_skinny.hip -- fused dequant GEMV / skinny GEMM on the matrix cores,
// C[M,N] = A[M,K] * dequant(B[N,K])^T for 1 <= M <= 16 (decode batch sizes).
// The ABI sends it 2 <= M <= 16 (the batch-1 GEMV of gemv.hip measured faster at
// M = 1 for every format, Q4_K included); M = 1 stays supported by the kernel.
//
// Q4_K (ref:src/kernels/matmul_quant.cu:309-386 computes the same product on
// fp32 FMA units).  gfx950 v_mfma_f32_16x16x32_f16 multiplies a 16(m) x 32(k)
// activation tile by a 32(k) x 16(n) weight tile:
//   * weights are the B operand as exact fp16 integers sc*q (6-bit scale times
//     4-bit code <= 945), unpacked from the nibbles with one and-or (the
//     1024 + q fp16 bit pattern) and one packed fma per two weights; the
//     super-block scale d (and the row's activation scale) is applied to the
//     fp32 accumulator once per 256 k;
//   * activations are the A operand, split x = hi + lo into two fp16 parts
//     (after a power-of-two scaling per row and super-block that keeps
//     hi < 2^15), so two MFMAs reproduce fp32-accurate products;
//   * the -dmin * mn offsets become one 16x16x16 MFMA per super-block between
//     the 6-bit mins and the per-sub-block activation sums (hi + lo, staged
//     times 2^-6 so that 32 values below 2^15 cannot overflow fp16);
// so the VALU only unpacks nibbles, and only the lanes that carry real rows
// (m < M) read activations from LDS.  Each 16-row weight tile is split over
// the waves of a workgroup by super-block and reduced through LDS at the end.
//
// Q6_K (ref:src/kernels/matmul_quant.cu:408-494) for 2 <= M <= 16 uses the
// same staging and tiling.  Its int8 sub-scale times the 6-bit code reaches
// 4096, beyond fp16's exact integers, so each weight sc * (q6 - 32) goes in as
// its fp16 rounding hi plus the exact remainder lo in {-1, 0, 1}: three MFMAs
// (x_hi * hi, x_lo * hi, x_hi * lo) per 32 k, the dropped x_lo * lo being
// 2^-11 of the smallest term; d is applied per super-block.
//
// MODE (see ActIn): the activations are computed while staged -- SwiGLU of the
// gate/up outputs, or RMSNorm of hidden + residual: per (row, super-block)
// sums of squares go to LDS next to the unscale factors, and the epilogue
// multiplies each output row by 1/sqrt(mean + eps).
#include <atomic>
#include <type_traits>

#include "act.hpp"
#include "common.hpp"
#include "internal.hpp"
#include "split.hpp"

namespace cri {
namespace dev {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

// Staging items per thread per load batch.
constexpr int kSkMaxItems = 6;
// Activation chunk bound: M * KC <= kSkChunk (fp16 hi + lo copies: 4 * kSkChunk bytes of LDS).
constexpr int kSkChunk = 32768;
// Workspace of a K split over workgroups (floats): the RMSNorm sums of squares [split][16 rows],
// then the partial sums [split][M][N].  Groups x splits <= 256 and a group is 128 columns, so
// N x splits <= 32768 and the partial sums take at most 32768 M floats.
constexpr int kSkMaxSplits = 16;
constexpr long kSkPartOff = kSkMaxSplits * 16;
static_assert(kSkMaxSplits <= kSplitMaxS, "the reduction reads up to kSplitMaxS splits");

// Order of the 8 k values of one k8 group inside an operand register set: the
// nibble unpack produces (0,2), (1,3), (4,6), (5,7) pairs.
__device__ constexpr int kPerm8[8] = {0, 2, 1, 3, 4, 6, 5, 7};

// (v & m) | o as one v_and_or_b32: gfx950 VOP3 takes no literal constants, so
// the mask comes from an SGPR and the or-constant from a VGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(m), "v"(o));
    return r;
}

__device__ __forceinline__ uint32_t pk_fma_f16(uint32_t a, uint32_t b, uint32_t c) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    h2 r = __builtin_elementwise_fma(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), __builtin_bit_cast(h2, c));
    return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ uint32_t f16x2_splat(float v) {
    const uint16_t h = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
    return static_cast<uint32_t>(h) | (static_cast<uint32_t>(h) << 16);
}

struct SkLds {
    // byte offsets inside the dynamic LDS block
    int xh, xl, xs, red, scl, ssq;
    int bytes;
};

// Row strides (in halves) of the staged activations and sub-block sums: one
// 16-byte (8-byte) pad per row puts the rows of a 16-lane operand fetch in
// different LDS banks.
__device__ __host__ inline int sk_xstride(int KC) { return KC + 8; }
__device__ __host__ inline int sk_sstride(int KC) { return KC / 16 + 4; }

__device__ __host__ inline SkLds sk_layout(int M, int KC, int nw, int K = 0, bool rms = false) {
    SkLds L;
    int o = 0;
    L.xh = o; o += M * sk_xstride(KC) * 2;
    L.xl = o; o += M * sk_xstride(KC) * 2;
    L.xs = o; o += M * sk_sstride(KC) * 2;  // per (m, sub-block pair): Xhi, Xhi, Xlo, Xlo
    o = (o + 15) & ~15;
    L.scl = o; o += (KC / 256) * 16 * 4;  // unscale[super-block][m] (16 m slots, zero beyond M)
    L.red = o; o += nw * 4 * 64 * 4;   // cross-wave reduction of k-split partials
    L.ssq = o; o += rms ? (K / 256) * 16 * 4 : 0;  // RMSNorm: sum of v^2 per [super-block of K][m]
    L.bytes = o;
    return L;
}

// Stage activations A[m][k0 .. k0+KC) (rows m < M) into LDS as fp16 hi/lo in
// the operand order.  Each (row, super-block) of 256 activations gets its own
// power-of-two scale that puts its max |x| just under 2^15 (the product of a
// super-block is rescaled anyway); the 32 k8 groups of one super-block sit in
// one half-wave, so the max is a DPP/swizzle reduction and needs no barrier.
// Per-sub-block sums (times 2^-6) feed the mins MFMA.  One barrier.
// Convert one staging item (row m, k8 group g8; live = it exists) into LDS:
// fp16 hi/lo in the operand order, the (row, super-block) unscale and the
// sub-block sums.  All 64 lanes of the wave must call it together (lane
// reductions); 32-lane groups hold one (row, super-block).
__device__ __forceinline__ void sk_convert_item(const f32x4 a, const f32x4 b, bool live, int m, int g8, int KC,
                                                _Float16* xh, _Float16* xl, _Float16* xs, float* unscale,
                                                float ss = 0.0f, float* ssq = nullptr) {
    if (ssq) {  // RMSNorm: the (row, super-block) sum of v^2 over the 32 lanes holding it, fixed order
        ss = group_sum_t<5>(ss);
        if (live && (g8 & 31) == 0) ssq[(g8 >> 5) * 16 + m] = ss;
    }
    float mx = fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                     fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
    mx = fmaxf(mx, dpp<kQuadPerm1032>(mx));
    mx = fmaxf(mx, dpp<kQuadPerm2301>(mx));
    mx = fmaxf(mx, dpp<kRowHalfMirror>(mx));
    mx = fmaxf(mx, dpp<kRowMirror>(mx));
    mx = fmaxf(mx, swizzle_xor16(mx));  // max over the 32 lanes = one super-block
    int ex = 0;
    if (mx > 0.0f) {
        frexpf(mx, &ex);
        ex -= 15;
        ex = ex < -100 ? -100 : (ex > 100 ? 100 : ex);
    }
    const float sc = ldexpf(1.0f, -ex);
    const float v[8] = {a.x * sc, a.y * sc, a.z * sc, a.w * sc, b.x * sc, b.y * sc, b.z * sc, b.w * sc};
    float sum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    if (live) {
        half8 hi, lo;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float x = v[kPerm8[i]];
            const _Float16 h = static_cast<_Float16>(x);
            hi[i] = h;
            lo[i] = static_cast<_Float16>(x - static_cast<float>(h));
        }
        *reinterpret_cast<half8*>(xh + m * sk_xstride(KC) + 8 * g8) = hi;
        *reinterpret_cast<half8*>(xl + m * sk_xstride(KC) + 8 * g8) = lo;
        if ((g8 & 31) == 0) unscale[(g8 >> 5) * 16 + m] = ldexpf(1.0f, ex);
    }
    // sub-block sum over the quad (fixed order -> deterministic), pair via row_shl:4
    sum = sum + dpp<kQuadPerm1032>(sum);
    sum = sum + dpp<kQuadPerm2301>(sum);
    const float next = dpp<0x104>(sum);  // row_shl:4: the quad above (sub-block 2p+1)
    if (live && (g8 & 7) == 0) {
        const float s0 = sum * 0.015625f, s1 = next * 0.015625f;  // 2^-6 keeps 32 * 2^15 in range
        const _Float16 h0 = static_cast<_Float16>(s0), h1 = static_cast<_Float16>(s1);
        half4 q;
        q[0] = h0;
        q[1] = h1;
        q[2] = static_cast<_Float16>(s0 - static_cast<float>(h0));
        q[3] = static_cast<_Float16>(s1 - static_cast<float>(h1));
        *reinterpret_cast<half4*>(xs + m * sk_sstride(KC) + 4 * (g8 >> 3)) = q;
    }
}

// Slots of unscale[] for rows m >= M (never written by the items) read as 0.
template <int NT>
__device__ __forceinline__ void sk_clear_unscale(int M, int KC, float* unscale) {
    const int nsb = KC / 256;
    for (int e = threadIdx.x; e < nsb * 16; e += NT)
        if ((e & 15) >= M) unscale[e] = 0.0f;
}

// Stage activations A[m][k0 .. k0+KC) (rows m < M) into LDS as fp16 hi/lo in
// the operand order.  Each (row, super-block) of 256 activations gets its own
// power-of-two scale that puts its max |x| just under 2^15 (the product of a
// super-block is rescaled anyway); (row, k8 group) items e = m * groups + g8
// are strided over the threads in batches of kSkMaxItems per thread, each
// batch's loads issued before any of its items is converted.  Per-sub-block
// sums (times 2^-6) feed the mins MFMA.  One barrier.
template <int MODE, int NT>
__device__ void sk_stage(const ActIn& P, int M, int K, int k0, int KC, char* lds, const SkLds& L, bool write_h) {
    const int tid = threadIdx.x;
    constexpr int nth = NT;
    const long lda = MODE == kActPlain ? K : P.lda;
    float* ssq = MODE == kActRMSNorm ? reinterpret_cast<float*>(lds + L.ssq) + (k0 >> 8) * 16 : nullptr;
    _Float16* xh = reinterpret_cast<_Float16*>(lds + L.xh);
    _Float16* xl = reinterpret_cast<_Float16*>(lds + L.xl);
    _Float16* xs = reinterpret_cast<_Float16*>(lds + L.xs);
    float* unscale = reinterpret_cast<float*>(lds + L.scl);
    const int groups = KC / 8;  // k8 groups per row; a multiple of 32
    sk_clear_unscale<NT>(M, KC, unscale);
    const int total = M * groups;  // a multiple of 32
    // items per load batch: the prologues hold 2x (SwiGLU), 3x (RMSNorm) or 4x (SwiGLU of two
    // partial sums) the raw values per item
    constexpr int kItems = MODE == kActPlain ? kSkMaxItems : (MODE == kActSwiGLU ? 4 : (MODE == kActRMSNorm ? 3 : 2));
    for (int e_batch = 0; e_batch < total; e_batch += kItems * nth) {
        ActRaw<MODE> ra[kItems], rb[kItems];
#pragma unroll
        for (int it = 0; it < kItems; ++it) {
            const int e = e_batch + it * nth + tid;
            if constexpr (MODE == kActPlain) ra[it].a = rb[it].a = f32x4{0.f, 0.f, 0.f, 0.f};
            if (e < total) {
                const int m = e / groups, g8 = e - m * groups;
                act_load<MODE>(ra[it], P, m, k0 + 8 * g8, lda);
                act_load<MODE>(rb[it], P, m, k0 + 8 * g8 + 4, lda);
            }
        }
#pragma unroll
        for (int it = 0; it < kItems; ++it) {
            const int e0 = e_batch + it * nth;
            if (e0 >= total) break;  // uniform over the workgroup
            const int e = e0 + tid;
            const bool live = e < total;
            const int m = live ? e / groups : 0, g8 = live ? e - m * groups : 0;
            if constexpr (MODE == kActPlain) {
                sk_convert_item(ra[it].a, rb[it].a, live, m, g8, KC, xh, xl, xs, unscale);
            } else {
                float ss = 0.0f;
                f32x4 va = f32x4{0.f, 0.f, 0.f, 0.f}, vb = va;
                if (live) {
                    va = act_finish<MODE>(ra[it], P, m, k0 + 8 * g8, K, ss, write_h);
                    vb = act_finish<MODE>(rb[it], P, m, k0 + 8 * g8 + 4, K, ss, write_h);
                }
                sk_convert_item(va, vb, live, m, g8, KC, xh, xl, xs, unscale, ss, ssq);
            }
        }
    }
    __syncthreads();
}

// When every thread has at most NPT items (M * KC / 8 <= NPT * threads), their
// loads are issued at kernel start, before the weight loads, and converted
// here: waiting for them does not wait for the weights.
template <int MODE, int NT, int NPT>
__device__ __forceinline__ void sk_load_few(const ActIn& P, int M, int K, int k0, int KC, ActRaw<MODE> (&a)[NPT],
                                            ActRaw<MODE> (&b)[NPT], bool none = false) {
    const int groups = KC / 8, total = M * groups;
    const long lda = MODE == kActPlain ? K : P.lda;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
        // an item past the end reads item 0 (every such lane the same address):
        // whole 32-lane groups are past the end, and they are not converted
        // none: a placeholder read (every lane item 0), whose registers go unused
        const int e0 = threadIdx.x + i * NT, e = e0 < total && !none ? e0 : 0;
        const int m = e / groups, g8 = e - m * groups;
        act_load<MODE>(a[i], P, m, k0 + 8 * g8, lda);
        act_load<MODE>(b[i], P, m, k0 + 8 * g8 + 4, lda);
    }
}
template <int MODE, int NT, int NPT>
__device__ __forceinline__ void sk_stage_few(const ActRaw<MODE> (&ra)[NPT], const ActRaw<MODE> (&rb)[NPT],
                                             const ActIn& P, int M, int K, int k0, int KC, char* lds, const SkLds& L,
                                             bool write_h) {
    _Float16* xh = reinterpret_cast<_Float16*>(lds + L.xh);
    _Float16* xl = reinterpret_cast<_Float16*>(lds + L.xl);
    _Float16* xs = reinterpret_cast<_Float16*>(lds + L.xs);
    float* unscale = reinterpret_cast<float*>(lds + L.scl);
    const int groups = KC / 8;
    sk_clear_unscale<NT>(M, KC, unscale);
    const int total = M * groups;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
        const int e = threadIdx.x + i * NT;
        if ((e & ~63) < total) {  // whole waves past the items skip (lane reductions need all 64 lanes)
            const bool live = e < total;
            const int m = live ? e / groups : 0, g8 = live ? e - m * groups : 0;
            if constexpr (MODE == kActPlain) {
                sk_convert_item(ra[i].a, rb[i].a, live, m, g8, KC, xh, xl, xs, unscale);
            } else {
                float ss = 0.0f;
                f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f}, b = a;
                if (live) {
                    a = act_finish<MODE>(ra[i], P, m, k0 + 8 * g8, K, ss, write_h);
                    b = act_finish<MODE>(rb[i], P, m, k0 + 8 * g8 + 4, K, ss, write_h);
                }
                float* ssq = MODE == kActRMSNorm ? reinterpret_cast<float*>(lds + L.ssq) + (k0 >> 8) * 16 : nullptr;
                sk_convert_item(a, b, live, m, g8, KC, xh, xl, xs, unscale, ss, ssq);
            }
        }
    }
    __syncthreads();
}

// The A operand of the skinny MFMAs.  Activation rows are staged as fp16 x_hi
// and x_lo (x_hi + x_lo = x to ~22 bits).  Two lane-row layouts:
//  - plain (M > 8): lane row m supplies x_hi of activation row m to one MFMA
//    chain and x_lo to a second one; output row m is the sum of both;
//  - paired (PAIR, M <= 8): lane row 2 i supplies x_hi and lane row 2 i + 1
//    x_lo of activation row i to the same MFMA, so one MFMA does the work of
//    two, and output rows 2 i and 2 i + 1 are added in the epilogue.
// Lane rows past the real ones read the last real row: an A row only feeds
// its own output row, and those are never stored (their unscale factor is 0).
// x0 / x1 point at the lane's hi / lo row (plain) or its one row (paired; x1
// unused); odd marks the lo rows of the paired layout.

// One Q4_K super-block of a 16-row tile, computed by one wave.
struct Q4KItem {
    u32x4 h, q0, q1;
};

// acc contribution of one super-block: lane (g = k slice, n) holds the row's
// 32 qs bytes of chunk g (sub-blocks 2g, 2g+1) and the 16-byte header; x0 / x1
// point at the lane's activation row(s) in LDS, super-block start + 64 g.
template <bool PAIR>
__device__ __forceinline__ f4 q4k_block(const Q4KItem& d, const _Float16* x0, const _Float16* x1,
                                        const _Float16* xsa, bool odd, int g, const float (&us)[4]) {
    // 6-bit scale / min of sub-blocks 2g, 2g+1 (ref:src/kernels/dequantize.cu:298-305)
    const bool low = g < 2;
    const uint32_t o = (g & 1) * 16;
    const uint32_t h1 = d.h.y, h2 = d.h.z, h3 = d.h.w;
    const uint32_t a_sc = low ? h1 : h3, a_mn = low ? h2 : h3;
    const uint32_t wa = low ? 6 : 4, wb = low ? 0 : 2, om = low ? 0 : 4;
    const uint32_t sc_lo = ubfe(a_sc, o, wa) | (ubfe(h1, o + 6, wb) << 4);
    const uint32_t mn_lo = ubfe(a_mn, o + om, wa) | (ubfe(h2, o + 6, wb) << 4);
    const uint32_t sc_hi = ubfe(a_sc, o + 8, wa) | (ubfe(h1, o + 14, wb) << 4);
    const uint32_t mn_hi = ubfe(a_mn, o + 8 + om, wa) | (ubfe(h2, o + 14, wb) << 4);
    // (1024 + q) * sc - 1024 * sc = q * sc exactly (q * sc <= 945); high nibbles
    // come out as 1024 + 16 q and use sc / 16
    const float fsl = static_cast<float>(sc_lo), fsh = static_cast<float>(sc_hi);
    const uint32_t mul_lo = f16x2_splat(fsl), add_lo = f16x2_splat(-1024.0f * fsl);
    const uint32_t mul_hi = f16x2_splat(fsh * 0.0625f), add_hi = f16x2_splat(-64.0f * fsh);
    const uint32_t q[8] = {d.q0.x, d.q0.y, d.q0.z, d.q0.w, d.q1.x, d.q1.y, d.q1.z, d.q1.w};
    half8 a0[8], a1[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {  // one batch of LDS reads per item
        a0[s] = *reinterpret_cast<const half8*>(x0 + 8 * s);
        if constexpr (!PAIR) a1[s] = *reinterpret_cast<const half8*>(x1 + 8 * s);
    }
    // sub-block sums (hi and lo parts); paired: they enter once, on the even row
    half4 as4 = *reinterpret_cast<const half4*>(xsa);
    if constexpr (PAIR) as4 = odd ? half4{0, 0, 0, 0} : as4;
    f4 P0 = f4{0.f, 0.f, 0.f, 0.f}, P1 = P0;  // two independent MFMA chains
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const uint32_t w0 = q[2 * (s & 3)], w1 = q[2 * (s & 3) + 1];
        const uint32_t m4 = s < 4 ? 0x000F000Fu : 0x00F000F0u;
        const uint32_t mul = s < 4 ? mul_lo : mul_hi, add = s < 4 ? add_lo : add_hi;
        typedef uint32_t u4 __attribute__((ext_vector_type(4)));
        const u4 b = u4{pk_fma_f16(and_or(w0, m4, 0x64006400u), mul, add),
                        pk_fma_f16(and_or(w0 >> 8, m4, 0x64006400u), mul, add),
                        pk_fma_f16(and_or(w1, m4, 0x64006400u), mul, add),
                        pk_fma_f16(and_or(w1 >> 8, m4, 0x64006400u), mul, add)};
        const half8 bw = __builtin_bit_cast(half8, b);
        if constexpr (PAIR) {
            if (s & 1) P1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0[s], bw, P1, 0, 0, 0);
            else P0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0[s], bw, P0, 0, 0, 0);
        } else {
            P0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0[s], bw, P0, 0, 0, 0);
            P1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1[s], bw, P1, 0, 0, 0);
        }
    }
    const f4 P = P0 + P1;
    // mins: sum over sub-blocks of mn * X on a 16x16x16 MFMA, slots (Xhi, Xhi, Xlo, Xlo)
    const uint32_t mnp = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(mn_lo))) |
                         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(mn_hi))) << 16);
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    const half4 bm = __builtin_bit_cast(half4, u2{mnp, mnp});
    const f4 Pm = __builtin_amdgcn_mfma_f32_16x16x16f16(as4, bm, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    const float dd = h_lo(d.h.x), dmin = h_hi(d.h.x) * 64.0f;  // sums were staged times 2^-6
    f4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = us[i] * (dd * P[i] - dmin * Pm[i]);
    return r;
}

// Format policies of the skinny kernel: the bytes one lane (k slice g of a
// 16-row tile, row nl) loads per super-block, and that super-block's
// contribution to the lane's four outputs.
struct SkQ4K {
    static constexpr int kBlockBytes = 144;
    static constexpr int kSliceStride = 64;  // lane group g holds k [64 g, 64 g + 64) of a super-block
    typedef Q4KItem Item;
    static __device__ __forceinline__ void load(Item& d, const uint8_t* sb, int g) {
        d.h = ld_u32x4_a16(sb);
        d.q0 = ld_u32x4_a16(sb + 16 + 32 * g);
        d.q1 = ld_u32x4_a16(sb + 32 + 32 * g);
    }
    template <bool PAIR>
    static __device__ __forceinline__ f4 block(const Item& d, const _Float16* x0, const _Float16* x1,
                                               const _Float16* xsa, bool odd, int g, const float (&us)[4]) {
        return q4k_block<PAIR>(d, x0, x1, xsa, odd, g, us);
    }
};

// Q6_K super-block (ref:src/kernels/dequantize.cu:215-243): element 128 c + e
// (e < 128) takes the low (e < 64) or high nibble of ql[64 c + (e % 64)] and
// bits 2 (e / 32) .. +1 of qh[32 c + e % 32]; int8 scale scales[8 c + e / 16];
// x = d * sc * (q6 - 32).  Lane slice g covers e in [64 (g & 1), +64) of chunk
// c = g >> 1, so MFMA slice s (8 k) needs ql bytes [8 s, 8 s + 8) and qh bytes
// [8 (s & 3), +8) of its chunk and one of four consecutive scales.  The
// super-blocks are only 2-byte aligned: the loads round down to a dword and
// funnel-shift.
struct Q6KItem {
    uint32_t ql[17], qh[9], sc[2];
    uint32_t d;      // fp16 bits of d
    uint32_t shift;  // byte offset of the super-block within its dword
};
struct SkQ6K {
    static constexpr int kBlockBytes = 210;
    static constexpr int kSliceStride = 64;
    typedef Q6KItem Item;
    static __device__ __forceinline__ void load(Item& d, const uint8_t* sb, int g) {
        const int c = g >> 1;
        const uintptr_t sh = reinterpret_cast<uintptr_t>(sb) & 3;
        const uint8_t* al = sb - sh + 64 * c;  // the runs below share sb's dword offset
        const uint8_t* ah = sb - sh + 128 + 32 * c;
        const uint8_t* as = sb - sh + 192 + 8 * c + 4 * (g & 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 v = ld_u32x4(al + 16 * i);
            d.ql[4 * i] = v.x; d.ql[4 * i + 1] = v.y; d.ql[4 * i + 2] = v.z; d.ql[4 * i + 3] = v.w;
        }
        d.ql[16] = ld_u32(al + 64);  // <= sb + 132
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const u32x4 v = ld_u32x4(ah + 16 * i);
            d.qh[4 * i] = v.x; d.qh[4 * i + 1] = v.y; d.qh[4 * i + 2] = v.z; d.qh[4 * i + 3] = v.w;
        }
        d.qh[8] = ld_u32(ah + 32);  // <= sb + 196
        d.sc[0] = ld_u32(as);
        d.sc[1] = ld_u32(as + (sh ? 4 : 0));  // second dword only when the scales straddle it (<= sb + 210)
        d.d = *reinterpret_cast<const uint16_t*>(sb + 208);
        d.shift = static_cast<uint32_t>(sh);
    }
    template <bool PAIR>
    static __device__ __forceinline__ f4 block(const Item& d, const _Float16* x0, const _Float16* x1,
                                               const _Float16*, bool, int g, const float (&us)[4]) {
        const uint32_t sh = d.shift;
        const uint32_t scs = __builtin_amdgcn_alignbyte(d.sc[1], d.sc[0], sh);
        uint32_t sc2[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) sc2[j] = f16x2_splat(static_cast<float>(static_cast<int8_t>(scs >> (8 * j))));
        const uint32_t bias = f16x2_splat(-1056.0f);  // (1024 + q6) - 1056 = q6 - 32
        const uint32_t lsh = 4 * (g & 1);
        half8 a0[8], a1[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            a0[s] = *reinterpret_cast<const half8*>(x0 + 8 * s);
            if constexpr (!PAIR) a1[s] = *reinterpret_cast<const half8*>(x1 + 8 * s);
        }
        // Ph: x_hi (paired: x_hi or x_lo) times the weights' hi part, Pc: times the
        // lo part (paired: for both rows, adding the tiny x_lo * lo term), Pl: x_lo
        // times the hi part (plain only)
        f4 Ph = f4{0.f, 0.f, 0.f, 0.f}, Pl = Ph, Pc = Ph;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint32_t hsh = 2 * (2 * (g & 1) + (s >> 2));
            uint32_t w[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t ql = __builtin_amdgcn_alignbyte(d.ql[2 * s + j + 1], d.ql[2 * s + j], sh);
                const uint32_t qh = __builtin_amdgcn_alignbyte(d.qh[2 * (s & 3) + j + 1], d.qh[2 * (s & 3) + j], sh);
                w[j] = ((ql >> lsh) & 0x0F0F0F0Fu) | (((qh >> hsh) & 0x03030303u) << 4);  // q6 bytes
            }
            const uint32_t sc = sc2[2 * (s >> 2) + ((s & 3) >> 1)];
            // register pairs (0,2), (1,3), (4,6), (5,7) of the slice, as the staged activations
            const uint32_t t[4] = {and_or(w[0], 0x00FF00FFu, 0x64006400u), and_or(w[0] >> 8, 0x00FF00FFu, 0x64006400u),
                                   and_or(w[1], 0x00FF00FFu, 0x64006400u), and_or(w[1] >> 8, 0x00FF00FFu, 0x64006400u)};
            typedef uint32_t u4 __attribute__((ext_vector_type(4)));
            u4 hi, lo;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // q6 - 32 exact; sc * (q6 - 32) = hi + lo with hi its fp16 rounding and
                // lo in {-1, 0, 1} (|sc * (q6 - 32)| <= 4096), both exact
                const uint32_t q = pk_fma_f16(t[r], 0x3C003C00u, bias);
                hi[r] = pk_fma_f16(q, sc, 0u);
                lo[r] = pk_fma_f16(q, sc, hi[r] ^ 0x80008000u);
            }
            const half8 bh = __builtin_bit_cast(half8, hi), bl = __builtin_bit_cast(half8, lo);
            Ph = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0[s], bh, Ph, 0, 0, 0);
            if constexpr (!PAIR) Pl = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1[s], bh, Pl, 0, 0, 0);
            Pc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0[s], bl, Pc, 0, 0, 0);
        }
        const f4 P = (Ph + Pl) + Pc;
        const float dd = h_lo(d.d);
        f4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = us[i] * (dd * P[i]);
        return r;
    }
};

// ---- 32-element block formats (Q8_0, Q4_0, Q5_0) and FP16 --------------------------
//
// An item is 8 consecutive 32-element blocks of a row (256 k, the same unit as a
// K-quant super-block, so the activation chunks and k splits are shared).  MFMA s
// of an item covers block s alone: lane group g supplies its elements
// [8 g, 8 g + 8), so each block's product (x_hi.q + x_lo.q, q an exact fp16
// integer) is finished in one output register set and scaled by that block's d
// -- the output lane's column is the weight row it loaded.  The staged
// activations hold k in groups of 8 with the (0,2),(1,3),(4,6),(5,7) pair order,
// which each format's unpack produces.  Blocks start at any 2-byte offset: the
// loads round down to a dword and funnel-shift, and read only dwords that lie
// inside the item (the parity of s, a compile-time constant, says which).

// One block: P = x_hi . w + x_lo . w on the matrix cores (one MFMA when the
// rows are paired), r += d * P.
template <bool PAIR>
__device__ __forceinline__ void blk_accumulate(const half8 a0, const half8 a1, const half8 bw, float d, f4& r) {
    f4 P = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bw, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    if constexpr (!PAIR) P = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bw, P, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = __builtin_fmaf(d, P[i], r[i]);
}

template <bool PAIR>
__device__ __forceinline__ void blk_load_x(const _Float16* x0, const _Float16* x1, half8 (&a0)[8], half8 (&a1)[8]) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        a0[s] = *reinterpret_cast<const half8*>(x0 + 32 * s);
        if constexpr (!PAIR) a1[s] = *reinterpret_cast<const half8*>(x1 + 32 * s);
    }
}

__device__ __forceinline__ float half_bits(uint32_t h) { return h_lo(h); }

// Q8_0 (ref:src/kernels/dequantize.cu:34-47): 34-byte blocks, int8 quants at
// byte 2.  Lane slice = 8 quants at 34 s + 2 + 8 g: dword offset 2 for even s
// (3 dwords, shifted), 0 for odd s (2 dwords).  q + 128 (sign bit flipped) is
// placed in the 1024 + b pattern and 1152 subtracted: q exactly.
struct Q8Item {
    uint32_t q[8][3];
    uint32_t d[8];
};
struct SkQ8_0 {
    static constexpr int kBlockBytes = 272;  // 8 blocks
    static constexpr int kSliceStride = 8;
    typedef Q8Item Item;
    static __device__ __forceinline__ void load(Item& d, const uint8_t* it, int g) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint8_t* p = it + 34 * s + 8 * g + (s & 1 ? 2 : 0);  // dword-aligned
            d.q[s][0] = ld_u32(p);
            d.q[s][1] = ld_u32(p + 4);
            d.q[s][2] = (s & 1) ? 0u : ld_u32(p + 8);
            d.d[s] = *reinterpret_cast<const uint16_t*>(it + 34 * s);
        }
    }
    template <bool PAIR>
    static __device__ __forceinline__ f4 block(const Item& d, const _Float16* x0, const _Float16* x1,
                                               const _Float16*, bool, int, const float (&us)[4]) {
        half8 a0[8], a1[8];
        blk_load_x<PAIR>(x0, x1, a0, a1);
        const uint32_t off = f16x2_splat(-1152.0f);
        f4 r = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint32_t w0 = ((s & 1) ? d.q[s][0] : __builtin_amdgcn_alignbyte(d.q[s][1], d.q[s][0], 2)) ^ 0x80808080u;
            const uint32_t w1 = ((s & 1) ? d.q[s][1] : __builtin_amdgcn_alignbyte(d.q[s][2], d.q[s][1], 2)) ^ 0x80808080u;
            typedef uint32_t u4 __attribute__((ext_vector_type(4)));
            const u4 b = u4{pk_fma_f16(and_or(w0, 0x00FF00FFu, 0x64006400u), 0x3C003C00u, off),
                            pk_fma_f16(and_or(w0 >> 8, 0x00FF00FFu, 0x64006400u), 0x3C003C00u, off),
                            pk_fma_f16(and_or(w1, 0x00FF00FFu, 0x64006400u), 0x3C003C00u, off),
                            pk_fma_f16(and_or(w1 >> 8, 0x00FF00FFu, 0x64006400u), 0x3C003C00u, off)};
            blk_accumulate<PAIR>(a0[s], a1[s], __builtin_bit_cast(half8, b), half_bits(d.d[s]), r);
        }
        f4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = us[i] * r[i];
        return o;
    }
};

// Q4_0 in the reference's element order (element e <- qs[e / 2], low nibble for
// even e; ref:src/kernels/dequantize.cu:84-100): 18-byte blocks, the lane's 8
// elements are the 4 bytes at 18 s + 2 + 4 g.  Bytes (b0 b1 b2 b3) are permuted
// to (b0 b2 b1 b3), so nibble fields at shifts 0, 4, 8, 12 give the element
// pairs (0,2), (1,3), (4,6), (5,7); 1032 is subtracted from 1024 + nib.
struct Q4Item {
    uint32_t q[8][2];
    uint32_t d[8];
};
struct SkQ4_0 {
    static constexpr int kBlockBytes = 144;
    static constexpr int kSliceStride = 8;
    typedef Q4Item Item;
    static __device__ __forceinline__ void load(Item& d, const uint8_t* it, int g) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint8_t* p = it + 18 * s + 4 * g + (s & 1 ? 2 : 0);  // dword-aligned
            d.q[s][0] = ld_u32(p);
            d.q[s][1] = (s & 1) ? 0u : ld_u32(p + 4);
            d.d[s] = *reinterpret_cast<const uint16_t*>(it + 18 * s);
        }
    }
    template <bool PAIR>
    static __device__ __forceinline__ f4 block(const Item& d, const _Float16* x0, const _Float16* x1,
                                               const _Float16*, bool, int, const float (&us)[4]) {
        half8 a0[8], a1[8];
        blk_load_x<PAIR>(x0, x1, a0, a1);
        const uint32_t off = f16x2_splat(-1032.0f);
        f4 r = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint32_t w = (s & 1) ? d.q[s][0] : __builtin_amdgcn_alignbyte(d.q[s][1], d.q[s][0], 2);
            const uint32_t wp = __builtin_amdgcn_perm(w, w, 0x03010200u);  // bytes (b0, b2, b1, b3)
            typedef uint32_t u4 __attribute__((ext_vector_type(4)));
            const u4 b = u4{pk_fma_f16(and_or(wp, 0x000F000Fu, 0x64006400u), 0x3C003C00u, off),
                            pk_fma_f16(and_or(wp >> 4, 0x000F000Fu, 0x64006400u), 0x3C003C00u, off),
                            pk_fma_f16(and_or(wp >> 8, 0x000F000Fu, 0x64006400u), 0x3C003C00u, off),
                            pk_fma_f16(and_or(wp >> 12, 0x000F000Fu, 0x64006400u), 0x3C003C00u, off)};
            blk_accumulate<PAIR>(a0[s], a1[s], __builtin_bit_cast(half8, b), half_bits(d.d[s]), r);
        }
        f4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = us[i] * r[i];
        return o;
    }
};

// Q5_0 (ref:src/kernels/dequantize.cu:137-164): 22-byte blocks, d, qh (u32 LE)
// at 2, qs at 6; element e: low nibble of qs[e % 16] for e < 16 else the high
// one, high bit = bit e of qh.  Lane group g takes qs bytes [8 (g & 1), +8)
// (nibble shift 4 (g >> 1)) and qh byte g; each bit pair moves to bits 4 and 20
// of its fp16 pair, OR-ed into the 1024 pattern; 1040 is subtracted.
struct Q5Item {
    uint32_t q[8][3];
    uint32_t h[8];
    uint32_t d[8];
};
struct SkQ5_0 {
    static constexpr int kBlockBytes = 176;
    static constexpr int kSliceStride = 8;
    typedef Q5Item Item;
    static __device__ __forceinline__ void load(Item& d, const uint8_t* it, int g) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint8_t* blk = it + 22 * s;
            const uint8_t* p = blk + 6 + 8 * (g & 1) - (s & 1 ? 0 : 2);  // dword-aligned
            d.q[s][0] = ld_u32(p);
            d.q[s][1] = ld_u32(p + 4);
            d.q[s][2] = (s & 1) ? 0u : ld_u32(p + 8);
            const uintptr_t hb = reinterpret_cast<uintptr_t>(blk + 2 + g);
            d.h[s] = (ld_u32(reinterpret_cast<const uint8_t*>(hb & ~static_cast<uintptr_t>(3))) >> (8 * (hb & 3))) & 0xFFu;
            d.d[s] = *reinterpret_cast<const uint16_t*>(blk);
        }
    }
    template <bool PAIR>
    static __device__ __forceinline__ f4 block(const Item& d, const _Float16* x0, const _Float16* x1,
                                               const _Float16*, bool, int g, const float (&us)[4]) {
        half8 a0[8], a1[8];
        blk_load_x<PAIR>(x0, x1, a0, a1);
        const uint32_t off = f16x2_splat(-1040.0f);
        const uint32_t sh = 4 * (g >> 1);
        f4 r = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint32_t w0 = ((s & 1) ? d.q[s][0] : __builtin_amdgcn_alignbyte(d.q[s][1], d.q[s][0], 2)) >> sh;
            const uint32_t w1 = ((s & 1) ? d.q[s][1] : __builtin_amdgcn_alignbyte(d.q[s][2], d.q[s][1], 2)) >> sh;
            const uint32_t t = d.h[s];  // qh byte g in the low 8 bits
            const uint32_t h02 = ((t << 4) | (t << 18)) & 0x00100010u;
            const uint32_t h13 = ((t << 3) | (t << 17)) & 0x00100010u;
            const uint32_t h46 = (t | (t << 14)) & 0x00100010u;
            const uint32_t h57 = ((t >> 1) | (t << 13)) & 0x00100010u;
            typedef uint32_t u4 __attribute__((ext_vector_type(4)));
            const u4 b = u4{pk_fma_f16(and_or(w0, 0x000F000Fu, 0x64006400u | h02), 0x3C003C00u, off),
                            pk_fma_f16(and_or(w0 >> 8, 0x000F000Fu, 0x64006400u | h13), 0x3C003C00u, off),
                            pk_fma_f16(and_or(w1, 0x000F000Fu, 0x64006400u | h46), 0x3C003C00u, off),
                            pk_fma_f16(and_or(w1 >> 8, 0x000F000Fu, 0x64006400u | h57), 0x3C003C00u, off)};
            blk_accumulate<PAIR>(a0[s], a1[s], __builtin_bit_cast(half8, b), half_bits(d.d[s]), r);
        }
        f4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = us[i] * r[i];
        return o;
    }
};

// FP16 weights (ref:src/kernels/matmul_quant.cu:510-558): the lane's 8 halves
// at 64 s + 16 g are the B operand after a half swap into the (0,2),(1,3),(4,6),
// (5,7) order; products fp16 x fp16 are exact in fp32, two MFMA chains.
struct F16Item {
    u32x4 v[8];
};
struct SkF16 {
    static constexpr int kBlockBytes = 512;
    static constexpr int kSliceStride = 8;
    typedef F16Item Item;
    static __device__ __forceinline__ void load(Item& d, const uint8_t* it, int g) {
#pragma unroll
        for (int s = 0; s < 8; ++s) d.v[s] = ld_u32x4(it + 64 * s + 16 * g);
    }
    template <bool PAIR>
    static __device__ __forceinline__ f4 block(const Item& d, const _Float16* x0, const _Float16* x1,
                                               const _Float16*, bool, int, const float (&us)[4]) {
        half8 a0[8], a1[8];
        blk_load_x<PAIR>(x0, x1, a0, a1);
        f4 Ph = f4{0.f, 0.f, 0.f, 0.f}, Pl = Ph;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const u32x4 v = d.v[s];
            typedef uint32_t u4 __attribute__((ext_vector_type(4)));
            const u4 b = u4{__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.y, v.x, 0x07060302u),
                            __builtin_amdgcn_perm(v.w, v.z, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u)};
            const half8 bw = __builtin_bit_cast(half8, b);
            if constexpr (PAIR) {  // two chains over alternate slices
                if (s & 1) Pl = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0[s], bw, Pl, 0, 0, 0);
                else Ph = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0[s], bw, Ph, 0, 0, 0);
            } else {
                Ph = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0[s], bw, Ph, 0, 0, 0);
                Pl = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1[s], bw, Pl, 0, 0, 0);
            }
        }
        const f4 P = Ph + Pl;
        f4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = us[i] * P[i];
        return o;
    }
};

// p[0] + p[256] + ... + p[256 (KS - 1)], in that order, all reads issued first.
template <int KS>
__device__ __forceinline__ float sum_splits(const float* p) {
    float v[KS];
#pragma unroll
    for (int i = 0; i < KS; ++i) v[i] = p[256 * i];
    float s = v[0];
#pragma unroll
    for (int i = 1; i < KS; ++i) s += v[i];
    return s;
}

// C = the S partial sums of a workspace K split added in split order, times the RMSNorm row
// factor of all S sums of squares (split.hpp's steps, which the consumers that read the
// partial sums directly repeat).  Four consecutive outputs per thread (N % 4 == 0, C 16-byte
// aligned: the launcher checks); all of a thread's loads are in flight together (exactly S of
// them for the common counts, sixteen clamped ones otherwise).
__global__ __launch_bounds__(256) void split_reduce_kernel(const SplitSums p, float* __restrict__ C, int M) {
    const long i4 = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (4 * i4 >= static_cast<long>(M) * p.N) return;
    const f32x4 t = split_sum4_any(p.part + 4 * i4, p.stride, p.S);
    const float fac = split_factor(p, static_cast<int>(4 * i4 / p.N));
    *reinterpret_cast<f32x4*>(C + 4 * i4) = t * fac;
}

// Workgroup = NW waves = (NW / KS) tiles x KS k-splits.  The grid strides
// over groups of NW / KS tiles; wave w works on tile w / KS of the group and
// on super-blocks j = w % KS, + KS, ... of the current activation chunk.
// Argument order: the 14 dwords of B, C, A and the eight integers are
// preloaded into SGPRs at wave launch (an aggregate argument and the hidden
// grid sizes are not), so the plain path issues its first loads without
// waiting on a scalar load of the argument block.  The activation pointer is
// passed on its own (A == P.a); the rest of the prologue comes last.
template <class F, int NW, int MODE, bool PAIR, int NPT, bool XPF>
__global__ __launch_bounds__(64 * NW) void skinny_kernel(const uint8_t* __restrict__ B, float* __restrict__ C,
                                                             const float* __restrict__ A, int M, int N, int K, int KC,
                                                             int ks_log2, int ngroups, int nchunks, int nblocks,
                                                             int cs_log2, float* __restrict__ part, const ActIn Pin) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    ActIn P = Pin;  // the activation pointer from its own (preloaded) argument
    P.a = A;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, nl = lane & 15;
    const int KS = 1 << ks_log2;              // k-splits per tile (power of two)
    const int TW = NW >> ks_log2;             // tiles per group
    const int my_tile = wave >> ks_log2, my_split = wave & (KS - 1);
    const long rbytes = static_cast<long>(K >> 8) * F::kBlockBytes;
    const int sb_chunk = KC / 256;
    const int nitems = (sb_chunk - my_split + KS - 1) >> ks_log2;  // super-blocks per wave per chunk
    // chunk split across workgroups (cs_log2 > 0): workgroup b takes chunks
    // [c_begin, c_begin + cps) of groups b >> cs_log2, + gstride, ..., and adds
    // its partial sums into C (zero-filled by the launcher), or, with a
    // workspace, stores them to part[split][m][n] for a fixed-order reduction
    const int cps = nchunks >> cs_log2;
    const int split = static_cast<int>(blockIdx.x) & ((1 << cs_log2) - 1);
    const int c_begin = split * cps;
    float* const mypart = part ? part + kSkPartOff + static_cast<long>(split) * M * N : nullptr;
    auto put = [&](int m, int n, float v) {
        float* dst = C + static_cast<long>(m) * N + n;
        if (!cs_log2)
            *dst = v;
        else if (mypart)
            mypart[static_cast<long>(m) * N + n] = v;
        else
            atomicAdd(dst, v);
    };
    const int grp0 = static_cast<int>(blockIdx.x) >> cs_log2, gstride = nblocks >> cs_log2;
    // RMSNorm: h + r goes to hidden_out from the workgroups of the first group (each stages its chunks)
    const bool write_h = grp0 == 0;
    // at most NPT activation items per thread (the launcher guarantees it for NPT > 1)
    const bool few = NPT > 1 || M * (KC / 8) <= 64 * NW;
    // weight row of this lane in group grp (clamped: the last tile may be partial)
    auto row_ptr = [&](int grp) {
        const int row = min((grp * TW + my_tile) * 16 + nl, N - 1);
        return B + static_cast<long>(row) * rbytes;
    };
    auto load_item = [&](typename F::Item& d, const uint8_t* cp, int it) {
        F::load(d, cp + static_cast<long>(it << ks_log2) * F::kBlockBytes, g);
    };
    // item it if it exists, else a placeholder read that every lane takes from the
    // same address (one cache line per instruction; the registers go unused)
    auto load_item_or_none = [&](typename F::Item& d, const uint8_t* cp, int it) {
        const bool real = it < nitems;
        F::load(d, real ? cp + static_cast<long>(it << ks_log2) * F::kBlockBytes : B, real ? g : 0);
    };
    // The first chunk of the first group is requested before anything else is
    // computed: the single-item activation loads, then the first two
    // super-blocks of this wave.  Everything after waits on them anyway.
    // Weight loads are never under a condition: the compiler then knows how many
    // are in flight and waits only for the ones a computation needs (a guarded
    // load makes it wait for all of them).  A wave with one item fills b1 with a
    // placeholder read instead.
    typename F::Item b0, b1;
    ActRaw<MODE> xa[NPT], xb[NPT];
    {
        const uint8_t* cp = row_ptr(grp0) + static_cast<long>(((c_begin * KC) >> 8) + my_split) * F::kBlockBytes;
        if (few) {
            sk_load_few<MODE, 64 * NW, NPT>(P, M, K, c_begin * KC, KC, xa, xb);
            // every wave's activation loads enter the vector-memory queue before any
            // weight load: the L1 returns data in request order, and the weights
            // miss to HBM while the activations are L2 hits (no wait here)
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
        }
        load_item(b0, cp, 0);
        load_item_or_none(b1, cp, 1);
    }
    __builtin_amdgcn_sched_barrier(0);

    const SkLds L = sk_layout(M, KC, NW, K, MODE == kActRMSNorm);
    // A operand of this lane (lane row m_a): activation row xrow, its hi and lo
    // parts (plain) or one of them (paired: lo on odd lane rows)
    const int m_a = lane & 15;
    const int xrow = min(PAIR ? m_a >> 1 : m_a, M - 1);
    const bool odd = PAIR && (m_a & 1);
    const int ntiles = (N + 15) >> 4;
    const _Float16* xh = reinterpret_cast<const _Float16*>(lds + L.xh);
    const _Float16* xl = reinterpret_cast<const _Float16*>(lds + L.xl);
    const _Float16* xs = reinterpret_cast<const _Float16*>(lds + L.xs);
    const _Float16* x0 = (odd ? xl : xh) + xrow * sk_xstride(KC) + F::kSliceStride * g;
    const _Float16* x1 = xl + xrow * sk_xstride(KC) + F::kSliceStride * g;
    const _Float16* xsr = xs + xrow * sk_sstride(KC) + 4 * g;
    const float* unscale = reinterpret_cast<const float*>(lds + L.scl);
    float* red = reinterpret_cast<float*>(lds + L.red);

    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
    auto run_item = [&](const typename F::Item& d, int it) {
        const int jj = my_split + (it << ks_log2);
        // unscale of this lane's four output rows: activation rows 4g .. 4g+3,
        // paired 2g, 2g, 2g+1, 2g+1
        float us[4];
        if constexpr (PAIR) {
            const f32x2 u2 = *reinterpret_cast<const f32x2*>(unscale + jj * 16 + 2 * g);
            us[0] = us[1] = u2.x;
            us[2] = us[3] = u2.y;
        } else {
            const f32x4 u4 = *reinterpret_cast<const f32x4*>(unscale + jj * 16 + 4 * g);
            us[0] = u4.x, us[1] = u4.y, us[2] = u4.z, us[3] = u4.w;
        }
        acc += F::template block<PAIR>(d, x0 + jj * 256, x1 + jj * 256, xsr + 16 * jj, odd, g, us);
    };
    // RMSNorm: the row factor of output row m (the sums of every chunk stay in LDS); with K split
    // over workgroups the factor is applied where the partial sums are added
    auto row_factor = [&](int m) {
        if constexpr (MODE == kActRMSNorm) {
            if (cs_log2) return 1.0f;
            const float* ssq = reinterpret_cast<const float*>(lds + L.ssq);
            float ss = 0.0f;
            for (int sb = 0; sb < (K >> 8); ++sb) ss += ssq[sb * 16 + min(m, M - 1)];
            return rms_factor(ss, K, P.eps);
        } else {
            (void)m;
            return 1.0f;
        }
    };
    // C of group grp: this lane's outputs are rows 4g + r (r < 4), paired rows
    // 2g + r (r < 2) as the sum of the hi and lo lane rows; the KS k-split
    // partials of each tile are reduced through LDS, red[w][r][lane]
    auto finish_group = [&](int grp) {
        const int tile = grp * TW + my_tile;
        constexpr int kRows = PAIR ? 2 : 4;
        f4 out = acc;
        if constexpr (PAIR) out = f4{acc[0] + acc[1], acc[2] + acc[3], 0.f, 0.f};
        if (KS == 1) {
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                const int m = kRows * g + r, n = tile * 16 + nl;
                if (m < M && n < N && tile < ntiles) put(m, n, out[r] * row_factor(m));
            }
        } else {
#pragma unroll
            for (int r = 0; r < kRows; ++r) red[(wave * 4 + r) * 64 + lane] = out[r];
            __syncthreads();
            // threads of wave w finish tile w / KS, register r = (w % KS) ... spread 4 regs x 64 lanes per tile
            for (int e = threadIdx.x; e < TW * 256; e += 64 * NW) {
                const int t = e >> 8, r = (e >> 6) & 3, ln = e & 63;
                if (r >= kRows) continue;
                const float* rp = red + ((t << ks_log2) * 4 + r) * 64 + ln;  // split sp at rp[256 sp]
                const float sum = ks_log2 == 1 ? sum_splits<2>(rp) : ks_log2 == 2 ? sum_splits<4>(rp) : sum_splits<8>(rp);
                const int tt = grp * TW + t;
                const int m = kRows * (ln >> 4) + r, n = tt * 16 + (ln & 15);
                if (m < M && n < N && tt < ntiles) put(m, n, sum * row_factor(m));
            }
            if (grp + gstride < ngroups) __syncthreads();  // the next group reuses red[]
        }
    };

    // chunks c = c_begin .. c_begin + cps - 1 of groups grp0, + gstride, ...;
    // the weights of each chunk were requested before the previous one finished
    int grp = grp0, c = c_begin;
    while (true) {
        const int k0 = c * KC;
        const uint8_t* cp = row_ptr(grp) + static_cast<long>((k0 >> 8) + my_split) * F::kBlockBytes;
        // activations are staged for every chunk of the first group, and for
        // every group when the workgroup has several chunks
        if (grp == grp0 || cps > 1) {
            if (few) sk_stage_few<MODE, 64 * NW, NPT>(xa, xb, P, M, K, k0, KC, lds, L, write_h);
            else sk_stage<MODE, 64 * NW>(P, M, K, k0, KC, lds, L, write_h);
        }
        // XPF (several chunks, register staging): the next chunk's activations are
        // requested now, so their latency hides behind this chunk's items; always
        // issued (a placeholder read when no chunk follows) to keep the compiler's
        // wait counts exact
        if constexpr (XPF) {
            const bool lastc = c + 1 == c_begin + cps;
            const bool none = lastc && grp + gstride >= ngroups;
            sk_load_few<MODE, 64 * NW, NPT>(P, M, K, lastc ? c_begin * KC : k0 + KC, KC, xa, xb, none);
        }
        // two super-blocks in flight: each item's registers are refilled with the
        // item two ahead right after it is used; the last two drain without loads
        int it = 0;
        for (; it + 2 < nitems; it += 2) {
            run_item(b0, it);
            load_item(b0, cp, it + 2);
            run_item(b1, it + 1);
            load_item_or_none(b1, cp, it + 3);
        }
        run_item(b0, it);
        if (it + 1 < nitems) run_item(b1, it + 1);

        const bool last_chunk = c + 1 == c_begin + cps;
        const int ngrp = last_chunk ? grp + gstride : grp, nc = last_chunk ? c_begin : c + 1;
        if (ngrp >= ngroups) {  // nothing left to request
            finish_group(grp);
            break;
        }
        // the next chunk is requested before the chunk barrier and this group's reduction
        {
            const uint8_t* np = row_ptr(ngrp) + static_cast<long>(((nc * KC) >> 8) + my_split) * F::kBlockBytes;
            if constexpr (!XPF)
                if (few && cps > 1) sk_load_few<MODE, 64 * NW, NPT>(P, M, K, nc * KC, KC, xa, xb);
            load_item(b0, np, 0);
            load_item_or_none(b1, np, 1);
        }
        if (cps > 1) __syncthreads();  // the next chunk overwrites the staged activations
        if (last_chunk) {
            finish_group(grp);
            acc = f4{0.f, 0.f, 0.f, 0.f};
        }
        grp = ngrp;
        c = nc;
    }
    // RMSNorm with a workspace split: the workgroups of the first group store their chunks'
    // sums of squares per row for the reduction (the other groups' are the same)
    if constexpr (MODE == kActRMSNorm) {
        if (mypart && grp0 == 0 && threadIdx.x < 16) {
            const float* ssq = reinterpret_cast<const float*>(lds + L.ssq) + ((c_begin * KC) >> 8) * 16;
            float ss = 0.0f;
            for (int sb = 0; sb < (cps * KC) >> 8; ++sb) ss += ssq[sb * 16 + threadIdx.x];
            part[split * 16 + threadIdx.x] = ss;
        }
    }
}

}  // namespace dev

namespace detail {

bool skinny_supported(int fmt, int M, int K, const void* B) {
    if (M < 1 || M > 16 || K % 256 != 0) return false;
    // Q4_K from 2 rows (16-byte loads of 144-byte blocks); the batch-1 GEMV measured faster at M = 1
    // (8192 x 2048 4.79 -> 4.55 us, 2048 x 2048 3.43 -> 2.87, 512 x 2048 3.33 -> 2.72)
    if (fmt == kFmtQ4_K) return M >= 2 && (reinterpret_cast<uintptr_t>(B) & 15u) == 0;
    // Q6_K: the batch-1 GEMV streams it at HBM rate; 2..16 rows share each decoded block here
    if (fmt == kFmtQ6_K) return M >= 2 && (reinterpret_cast<uintptr_t>(B) & 1u) == 0;
    // the 32-element formats and FP16 likewise from 2 rows; rows of 8-block items stay dword-aligned
    if (fmt == kFmtQ8_0 || fmt == kFmtQ4_0 || fmt == kFmtQ5_0 || fmt == kFmtF16)
        return M >= 2 && (reinterpret_cast<uintptr_t>(B) & 3u) == 0;
    return false;
}

// A workspace of a K split over workgroups holds the sums of squares and partial sums of this
// shape, and the reduction's 16-byte stores of C are aligned.
static bool split_ws_fits(const float* ws, long ws_floats, const float* C, int M, int N, int groups, int cs_log2) {
    (void)groups;
    return ws && (1 << cs_log2) <= dev::kSkMaxSplits && N % 4 == 0 &&
           (reinterpret_cast<uintptr_t>(C) & 15u) == 0 && (reinterpret_cast<uintptr_t>(ws) & 15u) == 0 &&
           ws_floats >= dev::kSkPartOff + (static_cast<long>(M) * N << cs_log2);
}

template <class F, int NW, int MODE, bool PAIR, int NPT, bool XPF = false>
static int launch_sk(const ActIn& A, const void* B, float* C, int M, int N, int K, int KC, int KS,
                     hipStream_t stream, int cs_force = -1, float* ws = nullptr, long ws_floats = 0,
                     SplitSums* defer = nullptr, int defer_S = 0) {
    if (defer) defer->S = 0;
    // large chunks need more than the default 64 KB of dynamic LDS: raise the limit once per kernel and device
    constexpr int kMaxDevices = 64;
    static std::atomic<bool> ready[kMaxDevices];
    int devid = 0;
    if (hipGetDevice(&devid) != hipSuccess || devid < 0 || devid >= kMaxDevices) return kFailed;
    if (!ready[devid].load(std::memory_order_acquire)) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&dev::skinny_kernel<F, NW, MODE, PAIR, NPT, XPF>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
            return kFailed;
        ready[devid].store(true, std::memory_order_release);
    }
    const int ntiles = (N + 15) / 16;
    const int TW = NW / KS;
    const int groups = (ntiles + TW - 1) / TW;
    int ks_log2 = 0;
    while ((1 << ks_log2) < KS) ++ks_log2;
    // enough workgroups for ~2048 waves; beyond that each workgroup strides over tile groups
    int blocks = groups < 2048 / NW ? groups : 2048 / NW;
    if (blocks < 1) blocks = 1;
    const dev::SkLds L = dev::sk_layout(M, KC, NW, K, MODE == kActRMSNorm);
    if (L.bytes > 160 * 1024) return -1;
    // Few tile groups and several activation chunks (the FFN down projection at
    // M = 5..16: 128 groups, 2 or 4 chunks): every workgroup would stage all of
    // K on half the CUs, so the chunks are split over 2 workgroups per group
    // that add into a zero-filled C (0 + a + b equals 0 + b + a exactly, so the
    // result does not depend on their order).  The RMSNorm prologue needs every
    // chunk's sum of squares in one workgroup and is not split.
    const int nchunks = K / KC;
    int cs_log2 = 0;
    if (cs_force >= 0)
        cs_log2 = cs_force;
    else if (MODE != kActRMSNorm && 2 * groups <= 2048 / NW && nchunks % 2 == 0)
        cs_log2 = 1;
    // With a workspace the partial sums are stored and a second launch adds them in split order
    // (deterministic; the RMSNorm row factor is applied there).  Without one, fp32 atomics into
    // a zero-filled C: exact in either order for two partials, otherwise the last bits can vary
    // between runs.  The RMSNorm prologue splits only with a workspace (its row factor needs
    // every split).  An in-kernel reduction by the last workgroup of each group to finish was
    // measured: its agent-scope release/acquire fences (L2 write-back and invalidate on every
    // XCD) made the decode step slower, 1.35 -> 1.91 ms at M = 16.
    const long mn = static_cast<long>(M) * N;
    float* part = nullptr;
    if (cs_log2 > 0 && split_ws_fits(ws, ws_floats, C, M, N, groups, cs_log2)) part = ws;
    if (MODE == kActRMSNorm && cs_log2 > 0 && !part) return -1;
    if (cs_log2 > 0) {
        blocks = groups << cs_log2;
        if (!part) launch_fill_zero(C, mn, stream);
    }
    hipLaunchKernelGGL((dev::skinny_kernel<F, NW, MODE, PAIR, NPT, XPF>), dim3(blocks), dim3(64 * NW), L.bytes, stream,
                       static_cast<const uint8_t*>(B), C, A.a, M, N, K, KC, ks_log2, groups, nchunks, blocks, cs_log2,
                       part, A);
    if (part) {
        SplitSums sums;
        sums.part = part + dev::kSkPartOff;
        sums.ssq = MODE == kActRMSNorm ? part : nullptr;
        sums.stride = mn;
        sums.S = 1 << cs_log2;
        sums.N = N;
        sums.K = K;
        sums.eps = A.eps;
        if (defer && (defer_S == 0 || defer_S == sums.S))
            *defer = sums;  // the consumer adds them up
        else
            hipLaunchKernelGGL(dev::split_reduce_kernel, dim3(static_cast<unsigned>((mn / 4 + 255) / 256)), dim3(256),
                               0, stream, sums, C, M);
    }
    return 0;
}

int launch_split_reduce(const SplitSums& p, float* C, int M, hipStream_t stream) {
    const long mn = static_cast<long>(M) * p.N;
    hipLaunchKernelGGL(dev::split_reduce_kernel, dim3(static_cast<unsigned>((mn / 4 + 255) / 256)), dim3(256), 0, stream,
                       p, C, M);
    return 0;
}

// up to 8 activation rows: hi and lo parts share each MFMA (paired lane rows)
template <class F, int MODE>
static int launch_sk_rows(const ActIn& A, const void* B, float* C, int M, int N, int K, int KC, int KS,
                          hipStream_t stream, int cs = -1, float* ws = nullptr, long wsf = 0,
                          SplitSums* df = nullptr, int dS = 0) {
    if (M <= 8) {
        // Q4_K with two activation items per thread (M = 1 at K = 8192, the FFN down
        // projection): their loads are issued at entry as well instead of after the
        // weights (measured 7.5 -> 6.7 us); the one-item kernel stays as it is
        if constexpr (std::is_same<F, dev::SkQ4K>::value)
            if (M * (KC / 8) > 512 && M * (KC / 8) <= 1024)
                return launch_sk<F, 8, MODE, true, 2>(A, B, C, M, N, K, KC, KS, stream, cs, ws, wsf, df, dS);
        return launch_sk<F, 8, MODE, true, 1>(A, B, C, M, N, K, KC, KS, stream, cs, ws, wsf, df, dS);
    }
    // Q4_K, more than 8 rows, plain activations, up to eight items per thread:
    // all of a chunk's activation loads are in registers ahead of time, and with
    // several chunks (M = 16 at the FFN down shape: 4 of 2048) the next chunk's
    // are requested while this one computes (29.5 -> 26.4 us there; a single
    // chunk is faster without that request: 2048 x 2048 8.3 against 9.1 us)
    if constexpr (std::is_same<F, dev::SkQ4K>::value && MODE == kActPlain)
        if (M * (KC / 8) > 512 && M * (KC / 8) <= 4096) {
            if (K > KC && cs != static_cast<int>(__builtin_ctz(static_cast<unsigned>(K / KC))))
                return launch_sk<F, 8, MODE, false, 8, true>(A, B, C, M, N, K, KC, KS, stream, cs, ws, wsf, df, dS);
            return launch_sk<F, 8, MODE, false, 8, false>(A, B, C, M, N, K, KC, KS, stream, cs, ws, wsf, df, dS);
        }
    return launch_sk<F, 8, MODE, false, 1>(A, B, C, M, N, K, KC, KS, stream, cs, ws, wsf, df, dS);
}

template <int MODE>
static int launch_skinny_m(int fmt, const ActIn& A, const void* B, float* C, int M, int N, int K,
                           hipStream_t stream, float* ws = nullptr, long wsf = 0, SplitSums* df = nullptr,
                           int dS = 0) {
    if (df) df->S = 0;
    // activation chunk: the largest multiple of 256 dividing K with M * KC <= kSkChunk
    // (few chunks: every chunk is staged once per workgroup)
    const int ntiles = (N + 15) / 16;
    int KC = (dev::kSkChunk / M) / 256 * 256;
    if (KC > K) KC = K;
    while (KC > 256 && K % KC != 0) KC -= 256;
    if (KC < 256 || K % KC != 0) return -1;
    const int sb = KC / 256;  // super-blocks per chunk
    // split K over the waves of a workgroup when there are too few tiles for ~2048 waves
    int KS = 1;
    while (KS < 8 && KS * 2 <= sb && static_cast<long>(ntiles) * KS < 2048) KS *= 2;
    // Split K over workgroups instead (from 2 rows with a workspace, from 9 without): every wave
    // takes its own 16-row tile (8 per workgroup) and each workgroup one chunk of K, the chunks
    // sized so that ~256 workgroups run.  A
    // staged activation then feeds 8 tiles instead of 8 / KS, and each workgroup stages only
    // its chunk.  With a workspace a second launch (or the consumer) adds the partial sums and
    // applies the RMSNorm row factor: every shape splits.  Without one, the partial sums
    // go into a zero-filled C with atomics, which pays only when the activations take several
    // chunks (K > KC, the FFN down projection; 2048 x 2048 at M = 16 measured 8.5 us unsplit,
    // 5.2 + 5.3 us split into 8 and reduced by a second launch), and not for the RMSNorm
    // prologue, whose row factor needs every chunk's sum of squares.
    // (The single-chunk o projection, 2048 x 2048 at M = 16, traces 5.2 + 4.7 us split and
    // reduced against 9.0 unsplit, yet the graph-replayed decode step is faster with the split:
    // 1.135 against 1.168 ms.)
    const bool ws_split = ws && N % 4 == 0 && (reinterpret_cast<uintptr_t>(C) & 15u) == 0 &&
                          wsf >= skinny_workspace_floats(M, N);
    int cs = -1;
    if ((M > 1 && ws_split) || (M > 8 && MODE != kActRMSNorm && K > KC)) {
        const long groups8 = (ntiles + 7) / 8;
        int split = 1;
        while (split < 16 && groups8 * split * 2 <= 256 && K % (256 * split * 2) == 0) split *= 2;
        if (split > 1) {
            KC = K / split;
            KS = 1;
            cs = __builtin_ctz(static_cast<unsigned>(split));
            if (M * KC > dev::kSkChunk) return -1;  // cannot happen: split > 1 only shrinks KC
        }
    }
    // eight waves per workgroup (8 / KS tiles each): measured faster than four for
    // every decode shape, from 512 x 2048 to the 128256 x 2048 lm_head
    switch (fmt) {
        case kFmtQ6_K: return launch_sk_rows<dev::SkQ6K, MODE>(A, B, C, M, N, K, KC, KS, stream, cs, ws, wsf, df, dS);
        case kFmtQ4_K: return launch_sk_rows<dev::SkQ4K, MODE>(A, B, C, M, N, K, KC, KS, stream, cs, ws, wsf, df, dS);
        case kFmtQ8_0: return launch_sk_rows<dev::SkQ8_0, MODE>(A, B, C, M, N, K, KC, KS, stream, cs, ws, wsf, df, dS);
        case kFmtQ4_0: return launch_sk_rows<dev::SkQ4_0, MODE>(A, B, C, M, N, K, KC, KS, stream, cs, ws, wsf, df, dS);
        case kFmtQ5_0: return launch_sk_rows<dev::SkQ5_0, MODE>(A, B, C, M, N, K, KC, KS, stream, cs, ws, wsf, df, dS);
        case kFmtF16: return launch_sk_rows<dev::SkF16, MODE>(A, B, C, M, N, K, KC, KS, stream, cs, ws, wsf, df, dS);
    }
    return -1;
}

int launch_skinny(int fmt, const float* A, const void* B, float* C, int M, int N, int K, hipStream_t stream) {
    const ActIn act{A, nullptr, nullptr, nullptr, K, 0.0f};
    return launch_skinny_m<kActPlain>(fmt, act, B, C, M, N, K, stream);
}

int launch_skinny_act(int mode, int fmt, const ActIn& act, const void* B, float* C, int M, int N, int K,
                      hipStream_t stream, float* ws, long ws_floats, SplitSums* defer, int defer_S) {
    if (defer) defer->S = 0;
    switch (mode) {
        case kActPlain:
            return launch_skinny_m<kActPlain>(fmt, act, B, C, M, N, K, stream, ws, ws_floats, defer, defer_S);
        case kActSwiGLU:
            return launch_skinny_m<kActSwiGLU>(fmt, act, B, C, M, N, K, stream, ws, ws_floats, defer, defer_S);
        case kActRMSNorm:
            return launch_skinny_m<kActRMSNorm>(fmt, act, B, C, M, N, K, stream, ws, ws_floats, defer, defer_S);
        case kActSwiGLU2:
            return launch_skinny_m<kActSwiGLU2>(fmt, act, B, C, M, N, K, stream, ws, ws_floats, defer, defer_S);
    }
    return -1;
}

// groups x splits <= 256 and 128 columns per group: N x splits <= 32768 (see kSkPartOff)
bool skinny_atomic_split(int M, int K) {
    // launch_skinny_m without a workspace: plain activations split K over workgroups (fp32 atomics
    // into C) from 9 rows when the activations take several chunks
    if (M <= 8 || M > 16 || K % 256 != 0) return false;
    int KC = (dev::kSkChunk / M) / 256 * 256;
    if (KC > K) KC = K;
    while (KC > 256 && K % KC != 0) KC -= 256;
    return KC >= 256 && K > KC;
}

long skinny_workspace_floats(int M, int N) {
    (void)N;
    return dev::kSkPartOff + 32768L * M;
}

}  // namespace detail
}  // namespace cri

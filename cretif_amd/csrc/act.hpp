// act.hpp -- activation prologues of the fused decode matmuls (see ActIn in
// internal.hpp): four consecutive activations of row m at column k are loaded
// raw (all of a batch's loads first) and then turned into the operand values.
//
// SwiGLU follows ref:src/kernels/elementwise.cu:93-99 (silu(x) = x / (1 + exp(-x)))
// and :300-305 (the product with up); RMSNorm with a residual follows
// ref:src/kernels/elementwise.cu:463-504 (v = input + residual, sum of v^2 over
// the row, normed = v * weight * rsqrt(mean + eps)); here the weight multiplies
// the staged value and the row factor multiplies the finished output row,
// which is the same product in another order.
#pragma once

#include "common.hpp"
#include "internal.hpp"

namespace cri {
namespace dev {

template <int MODE>
struct ActRaw;
template <>
struct ActRaw<kActPlain> {
    f32x4 a;
};
template <>
struct ActRaw<kActSwiGLU> {
    f32x4 g, u;
};
template <>
struct ActRaw<kActRMSNorm> {
    f32x4 h, r, w;
};
template <>
struct ActRaw<kActRMSNormS> {
    f32x4 h, r[kResMaxSplits], w;
};
template <>
struct ActRaw<kActSwiGLU2> {
    f32x4 g0, g1, u0, u1;
    float s[kResMaxSplits];  // the sums of squares of row m (nss of them used)
};

// Loads of x[m][k .. k+4) (k % 4 == 0, all four in range); rows lda floats apart
// (the kernels pass K in plain mode, so P.lda is not read there).
template <int MODE>
__device__ __forceinline__ void act_load(ActRaw<MODE>& raw, const ActIn& P, int m, int k, long lda) {
    const long off = static_cast<long>(m) * lda + k;
    if constexpr (MODE == kActPlain) {
        raw.a = ld_f32x4(P.a + off);
    } else if constexpr (MODE == kActSwiGLU) {
        raw.g = ld_f32x4(P.a + off);
        raw.u = ld_f32x4(P.b + off);
    } else if constexpr (MODE == kActRMSNormS) {
        raw.h = ld_f32x4(P.a + off);
#pragma unroll
        for (int s = 0; s < kResMaxSplits; ++s) raw.r[s] = ld_f32x4(P.b + min(s, P.kn - 1) * P.split + off);
        raw.w = ld_f32x4(P.w + k);
    } else if constexpr (MODE == kActSwiGLU2) {
        raw.g0 = ld_f32x4(P.a + off);
        raw.g1 = ld_f32x4(P.a + P.split + off);
        raw.u0 = ld_f32x4(P.b + off);
        raw.u1 = ld_f32x4(P.b + P.split + off);
        const float* sq = P.w ? P.w : P.a;  // without sums of squares: an unused in-bounds read
#pragma unroll
        for (int i = 0; i < kResMaxSplits; ++i) raw.s[i] = sq[16 * min(i, P.nss - 1) + m];
    } else {
        raw.h = ld_f32x4(P.a + off);
        raw.r = P.b ? ld_f32x4(P.b + off) : f32x4{0.f, 0.f, 0.f, 0.f};
        raw.w = ld_f32x4(P.w + k);
    }
}

// silu(x) = x / (1 + e^-x) with the hardware exp2 and reciprocal (v_exp_f32,
// v_rcp_f32; ~1 ulp each, a few ulp in all against the reference's expf and
// IEEE divide): the prologue evaluates it for every staged activation of
// every workgroup.  Past |x| = 88 the exponent saturates to 0 or inf and the
// result to x or -0, as the reference's.
__device__ __forceinline__ float silu_f(float x) {
    const float e = __builtin_amdgcn_exp2f(x * -1.44269504088896341f);
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// Operand values from the raw loads.  RMSNorm adds v^2 (in k order) to ss and,
// when write_h, stores v to h_out[m*K + k].
template <int MODE>
__device__ __forceinline__ f32x4 act_finish(const ActRaw<MODE>& raw, const ActIn& P, int m, int k, int K, float& ss,
                                            bool write_h) {
    if constexpr (MODE == kActPlain) {
        (void)P; (void)m; (void)k; (void)K; (void)ss; (void)write_h;
        return raw.a;
    } else if constexpr (MODE == kActSwiGLU) {
        (void)m; (void)k; (void)K; (void)ss; (void)write_h;
        return f32x4{silu_f(raw.g.x) * raw.u.x, silu_f(raw.g.y) * raw.u.y, silu_f(raw.g.z) * raw.u.z,
                     silu_f(raw.g.w) * raw.u.w};
    } else if constexpr (MODE == kActSwiGLU2) {
        (void)m; (void)k; (void)K; (void)ss; (void)write_h;
        // the reduction kernel's steps: (split 0 + split 1) * row factor (1 without RMSNorm)
        float ss = raw.s[0];
#pragma unroll
        for (int i = 1; i < kResMaxSplits; ++i)
            if (i < P.nss) ss += raw.s[i];
        const float f = P.w ? 1.0f / sqrtf(ss / static_cast<float>(P.kn) + P.eps) : 1.0f;
        // (split 0: one partial sum, the second load read it again)
        const f32x4 g = (P.split ? raw.g0 + raw.g1 : raw.g0) * f, u = (P.split ? raw.u0 + raw.u1 : raw.u0) * f;
        return f32x4{silu_f(g.x) * u.x, silu_f(g.y) * u.y, silu_f(g.z) * u.z, silu_f(g.w) * u.w};
    } else {
        f32x4 r;
        if constexpr (MODE == kActRMSNormS) {  // the residual's partial sums, in split order
            r = raw.r[0];
#pragma unroll
            for (int s = 1; s < kResMaxSplits; ++s)
                if (s < P.kn) r += raw.r[s];
        } else {
            r = raw.r;
        }
        const f32x4 v = raw.h + r;
        ss = __builtin_fmaf(v.x, v.x, ss);
        ss = __builtin_fmaf(v.y, v.y, ss);
        ss = __builtin_fmaf(v.z, v.z, ss);
        ss = __builtin_fmaf(v.w, v.w, ss);
        if (write_h && P.h_out) {
            float* dst = P.h_out + static_cast<long>(m) * K + k;
            dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
        }
        return v * raw.w;
    }
}

// The RMSNorm row factor from the row's sum of squares.
__device__ __forceinline__ float rms_factor(float ss, int K, float eps) {
    return 1.0f / sqrtf(ss / static_cast<float>(K) + eps);
}

}  // namespace dev
}  // namespace cri

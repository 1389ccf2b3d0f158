// split.hpp -- reading a decode-batch matmul whose K was split over workgroups
// and left unreduced (SplitSums): the partial sums added in split order, times
// the RMSNorm row factor of all splits' sums of squares.  The reduction kernel
// and the consumers that take the partial sums directly use these same steps,
// so C comes out bit-identical whichever of them adds it up.
#pragma once

#include "common.hpp"
#include "internal.hpp"

namespace cri {
namespace dev {

constexpr int kSplitMaxS = 16;

// 1/sqrt(sum_s ssq[s*16 + m] / K + eps) over the nss (else S) sums in order, or 1 without RMSNorm;
// every load unconditional (splits past S read split S - 1, unused)
__device__ __forceinline__ float split_factor(const SplitSums& p, int m) {
    if (!p.ssq) return 1.0f;
    const int ns = p.nss ? p.nss : p.S;
    float sq[kSplitMaxS];
#pragma unroll
    for (int s = 0; s < kSplitMaxS; ++s) sq[s] = p.ssq[min(s, ns - 1) * 16 + m];
    float ss = sq[0];
#pragma unroll
    for (int s = 1; s < kSplitMaxS; ++s)
        if (s < ns) ss += sq[s];
    return 1.0f / sqrtf(ss / static_cast<float>(p.K) + p.eps);
}

// sum over splits of part[s][off] in split order (off = m N + n)
__device__ __forceinline__ float split_sum(const SplitSums& p, long off) {
    float v[kSplitMaxS];
#pragma unroll
    for (int s = 0; s < kSplitMaxS; ++s) v[s] = p.part[min(s, p.S - 1) * p.stride + off];
    float t = v[0];
#pragma unroll
    for (int s = 1; s < kSplitMaxS; ++s)
        if (s < p.S) t += v[s];
    return t;
}

// split_sum with the split count known at compile time (S <= kSplitMaxS): the same additions in
// the same order, S loads instead of kSplitMaxS
template <int S>
__device__ __forceinline__ float split_sum_n(const SplitSums& p, long off) {
    float v[S];
#pragma unroll
    for (int s = 0; s < S; ++s) v[s] = p.part[s * p.stride + off];
    float t = v[0];
#pragma unroll
    for (int s = 1; s < S; ++s) t += v[s];
    return t;
}

// the same for four consecutive elements (16-byte loads: part, stride and off multiples of 4)
template <int S>
__device__ __forceinline__ f32x4 split_sum4_n(const float* part, long stride) {
    f32x4 v[S];
#pragma unroll
    for (int s = 0; s < S; ++s) v[s] = *reinterpret_cast<const f32x4*>(part + s * stride);
    f32x4 t = v[0];
#pragma unroll
    for (int s = 1; s < S; ++s) t += v[s];
    return t;
}
__device__ __forceinline__ f32x4 split_sum4_any(const float* part, long stride, int S) {
    switch (S) {
        case 1: return split_sum4_n<1>(part, stride);
        case 2: return split_sum4_n<2>(part, stride);
        case 4: return split_sum4_n<4>(part, stride);
        case 8: return split_sum4_n<8>(part, stride);
        default: {
            f32x4 v[kSplitMaxS];
#pragma unroll
            for (int s = 0; s < kSplitMaxS; ++s) v[s] = *reinterpret_cast<const f32x4*>(part + min(s, S - 1) * stride);
            f32x4 t = v[0];
#pragma unroll
            for (int s = 1; s < kSplitMaxS; ++s)
                if (s < S) t += v[s];
            return t;
        }
    }
}

// split_sum dispatched on the common split counts
__device__ __forceinline__ float split_sum_any(const SplitSums& p, long off) {
    switch (p.S) {
        case 1: return split_sum_n<1>(p, off);
        case 2: return split_sum_n<2>(p, off);
        case 4: return split_sum_n<4>(p, off);
        case 8: return split_sum_n<8>(p, off);
        default: return split_sum(p, off);
    }
}

}  // namespace dev
}  // namespace cri

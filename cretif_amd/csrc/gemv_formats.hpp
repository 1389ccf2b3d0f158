// gemv_formats.hpp -- per-format decode for the batch-1 GEMV (y = W x).
//
// A "unit" is 64 consecutive-in-storage weights of one row.  A lane owns the
// same unit index in every row it visits, so the 64 activations of that unit
// are loaded once into VGPRs and reused for every row (they are never
// re-read from memory inside the row loop).  Each format provides
//
//   Data            raw bytes of one unit, loaded with dword-aligned vector loads
//   Xr              the unit's activations (+ per-block activation sums)
//   load_x(xr, x, unit)       activations, in the order dot() consumes them
//   load(d, row, unit)        the unit's bytes of one row
//   dot(d, xr)                fp32 partial dot product of the unit
//
// Decode follows the reference formulas (ref:src/kernels/dequantize.cu):
// block scales are applied per block to partial sums instead of per element,
// and constant offsets (-8, -16, -32, -dmin*mn) are applied through
// per-block activation sums, which is the same sum reassociated.
#pragma once

#include "common.hpp"

namespace cri {
namespace dev {

// ---------------------------------------------------------------------------
// shared helpers
// ---------------------------------------------------------------------------
// x points at the workgroup's LDS copy of the activations, stored padded: element
// k at k + 4 (k / 64).  A lane reads the 64 activations of its unit, and the lanes
// of a row hold consecutive units, 64 floats apart; padded, their 16-byte reads
// start 68 floats apart and fall in different banks (unpadded, a read instruction
// sent all of its lanes to the same banks).
__host__ __device__ __forceinline__ int xpad(int k) { return k + ((k >> 6) << 2); }

__device__ __forceinline__ void load_x64(float (&v)[64], const float* x, int k0) {  // k0 % 64 == 0
    const float* xu = x + xpad(k0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        f32x4 t = *reinterpret_cast<const f32x4*>(xu + 4 * i);
        v[4 * i + 0] = t.x;
        v[4 * i + 1] = t.y;
        v[4 * i + 2] = t.z;
        v[4 * i + 3] = t.w;
    }
}

__device__ __forceinline__ float sum_range(const float (&v)[64], int b, int n) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < n; ++i) s += v[b + i];
    return s;
}

// ---------------------------------------------------------------------------
// Q4_K: unit = (super-block j, 64-element chunk c) = 32 bytes of qs.
// Low nibbles of qs[32c + l] are elements 64c + l (sub-block 2c), high
// nibbles are elements 64c + 32 + l (sub-block 2c+1)
// (ref:src/kernels/dequantize.cu:307-319).
// ---------------------------------------------------------------------------
struct GemvQ4K {
    static constexpr int kPref1 = 1;  // row-groups in flight per wave at UPL = 1 (8192 x 2048: 4.84 us at 4, 4.55 at 1)
    static constexpr bool kSpread = false;  // one wave per kPref1 row groups above 2048 groups
    static constexpr bool kPairUnits = true;  // two units per lane at K = 2048 for N >= 8192 (8192 x 2048: Q4_K 4.53 -> 4.37 us, Q4_0 4.43 -> 4.23; 16384 x 2048 Q4_K 6.94 -> 6.09)
    static constexpr int kBlockBytes = 144;
    struct Data {
        u32x4 h;       // d, dmin, scales[0..11]
        u32x4 q0, q1;  // qs[32c .. 32c+32)
    };
    struct Xr {
        float v[64];
        float xs_lo, xs_hi;
    };
    static __device__ __forceinline__ void load_x(Xr& r, const float* x, int unit) {
        load_x64(r.v, x, unit * 64);
        r.xs_lo = sum_range(r.v, 0, 32);
        r.xs_hi = sum_range(r.v, 32, 32);
    }
    static __device__ __forceinline__ void load(Data& d, const uint8_t* __restrict__ row, int unit) {
        const uint8_t* p = row + (unit >> 2) * kBlockBytes;
        const int c = unit & 3;
        d.h = ld_u32x4(p);
        d.q0 = ld_u32x4(p + 16 + 32 * c);
        d.q1 = ld_u32x4(p + 32 + 32 * c);
    }
    static __device__ __forceinline__ float dot(const Data& d, const Xr& r, int unit) {
        const int c = unit & 3;
        // 6-bit scale/min of sub-blocks 2c and 2c+1 (ref:src/kernels/dequantize.cu:298-305).
        // c < 2:  sc = s[sb] & 63, mn = s[sb+4] & 63
        // c >= 2: sc = (s[sb+4] & 15) | (s[sb-4] >> 6) << 4, mn = (s[sb+4] >> 4) | (s[sb] >> 6) << 4
        const bool low = c < 2;
        const uint32_t o = (c & 1) * 16;
        const uint32_t h1 = d.h.y, h2 = d.h.z, h3 = d.h.w;
        const uint32_t a_sc = low ? h1 : h3;
        const uint32_t a_mn = low ? h2 : h3;
        const uint32_t wa = low ? 6 : 4;
        const uint32_t wb = low ? 0 : 2;
        const uint32_t om = low ? 0 : 4;
        const uint32_t sc_lo = ubfe(a_sc, o, wa) | (ubfe(h1, o + 6, wb) << 4);
        const uint32_t mn_lo = ubfe(a_mn, o + om, wa) | (ubfe(h2, o + 6, wb) << 4);
        const uint32_t sc_hi = ubfe(a_sc, o + 8, wa) | (ubfe(h1, o + 14, wb) << 4);
        const uint32_t mn_hi = ubfe(a_mn, o + 8 + om, wa) | (ubfe(h2, o + 14, wb) << 4);

        float s_lo0 = 0.f, s_lo1 = 0.f, s_hi0 = 0.f, s_hi1 = 0.f;
        const uint32_t q[8] = {d.q0.x, d.q0.y, d.q0.z, d.q0.w, d.q1.x, d.q1.y, d.q1.z, d.q1.w};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t w = q[t], u = w >> 8;
            const uint32_t a = w & 0x000F000Fu;  // lo nibbles of bytes 4t, 4t+2
            const uint32_t b = w & 0x00F000F0u;  // 16 * hi nibbles of bytes 4t, 4t+2
            const uint32_t e = u & 0x000F000Fu;  // lo nibbles of bytes 4t+1, 4t+3
            const uint32_t f = u & 0x00F000F0u;  // 16 * hi nibbles of bytes 4t+1, 4t+3
            s_lo0 = __builtin_fmaf(h_lo(a), r.v[4 * t + 0], s_lo0);
            s_lo1 = __builtin_fmaf(h_lo(e), r.v[4 * t + 1], s_lo1);
            s_lo0 = __builtin_fmaf(h_hi(a), r.v[4 * t + 2], s_lo0);
            s_lo1 = __builtin_fmaf(h_hi(e), r.v[4 * t + 3], s_lo1);
            s_hi0 = __builtin_fmaf(h_lo(b), r.v[32 + 4 * t + 0], s_hi0);
            s_hi1 = __builtin_fmaf(h_lo(f), r.v[32 + 4 * t + 1], s_hi1);
            s_hi0 = __builtin_fmaf(h_hi(b), r.v[32 + 4 * t + 2], s_hi0);
            s_hi1 = __builtin_fmaf(h_hi(f), r.v[32 + 4 * t + 3], s_hi1);
        }
        const float dd = h_lo(d.h.x), dmin = h_hi(d.h.x);
        // s_lo holds nib * 2^-24 * x; s_hi holds 16 * nib * 2^-24 * x.
        const float t = (s_lo0 + s_lo1) * static_cast<float>(sc_lo) +
                        (s_hi0 + s_hi1) * (static_cast<float>(sc_hi) * 0.0625f);
        const float m = static_cast<float>(mn_lo) * r.xs_lo + static_cast<float>(mn_hi) * r.xs_hi;
        return (dd * kTwo24) * t - dmin * m;
    }
};

// ---------------------------------------------------------------------------
// Q8_0: unit = two consecutive blocks (68 bytes, dword aligned when the row
// holds an even number of blocks).  Block A: d @0, qs @2..33; block B: d @34,
// qs @36..67 (ref:src/kernels/dequantize.cu:34-48).
// ---------------------------------------------------------------------------
struct GemvQ8_0 {
    static constexpr int kPref1 = 1;  // row-groups in flight per wave at UPL = 1 (8192 x 2048: 5.67 us at 2, 5.29 at 1)
    static constexpr bool kSpread = false;  // one wave per kPref1 row groups above 2048 groups
    static constexpr bool kPairUnits = false;
    static constexpr int kPairBytes = 68;
    struct Data {
        u32x4 w0, w1, w2, w3;
        uint32_t w4;
    };
    struct Xr {
        float v[64];
    };
    static __device__ __forceinline__ void load_x(Xr& r, const float* x, int unit) {
        load_x64(r.v, x, unit * 64);
    }
    static __device__ __forceinline__ void load(Data& d, const uint8_t* __restrict__ row, int unit) {
        const uint8_t* p = row + unit * kPairBytes;
        d.w0 = ld_u32x4(p);
        d.w1 = ld_u32x4(p + 16);
        d.w2 = ld_u32x4(p + 32);
        d.w3 = ld_u32x4(p + 48);
        d.w4 = ld_u32(p + 64);
    }
    static __device__ __forceinline__ float dot(const Data& d, const Xr& r, int) {
        const uint32_t w[17] = {d.w0.x, d.w0.y, d.w0.z, d.w0.w, d.w1.x, d.w1.y, d.w1.z, d.w1.w,
                                d.w2.x, d.w2.y, d.w2.z, d.w2.w, d.w3.x, d.w3.y, d.w3.z, d.w3.w, d.w4};
        float sa0 = 0.f, sa1 = 0.f, sb0 = 0.f, sb1 = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i += 2) {
            sa0 = __builtin_fmaf(sbyte(w[(2 + i) >> 2], (2 + i) & 3), r.v[i], sa0);
            sa1 = __builtin_fmaf(sbyte(w[(3 + i) >> 2], (3 + i) & 3), r.v[i + 1], sa1);
            sb0 = __builtin_fmaf(sbyte(w[(36 + i) >> 2], (36 + i) & 3), r.v[32 + i], sb0);
            sb1 = __builtin_fmaf(sbyte(w[(37 + i) >> 2], (37 + i) & 3), r.v[33 + i], sb1);
        }
        const float da = h_lo(w[0]), db = h_hi(w[8]);
        return da * (sa0 + sa1) + db * (sb0 + sb1);
    }
};

// ---------------------------------------------------------------------------
// Q4_0: unit = two blocks (36 bytes).  Reference element order: element i of a
// block is qs[i/2], low nibble for even i (ref:src/kernels/dequantize.cu:87-97).
// Block A: d @0, qs @2..17; block B: d @18, qs @20..35.
// ---------------------------------------------------------------------------
struct GemvQ4_0 {
    static constexpr int kPref1 = 1;  // row-groups in flight per wave at UPL = 1 (8192 x 2048: 4.63 us at 4, 4.41 at 1)
    static constexpr bool kSpread = false;  // one wave per kPref1 row groups above 2048 groups
    static constexpr bool kPairUnits = true;  // two units per lane at K = 2048 for N >= 8192 (8192 x 2048: Q4_K 4.53 -> 4.37 us, Q4_0 4.43 -> 4.23; 16384 x 2048 Q4_K 6.94 -> 6.09)
    static constexpr int kPairBytes = 36;
    struct Data {
        u32x4 w0, w1;
        uint32_t w2;
    };
    struct Xr {
        float v[64];
        float xs_a, xs_b;
    };
    static __device__ __forceinline__ void load_x(Xr& r, const float* x, int unit) {
        load_x64(r.v, x, unit * 64);
        r.xs_a = sum_range(r.v, 0, 32);
        r.xs_b = sum_range(r.v, 32, 32);
    }
    static __device__ __forceinline__ void load(Data& d, const uint8_t* __restrict__ row, int unit) {
        const uint8_t* p = row + unit * kPairBytes;
        d.w0 = ld_u32x4(p);
        d.w1 = ld_u32x4(p + 16);
        d.w2 = ld_u32(p + 32);
    }
    static __device__ __forceinline__ float dot(const Data& d, const Xr& r, int) {
        const uint32_t w[9] = {d.w0.x, d.w0.y, d.w0.z, d.w0.w, d.w1.x, d.w1.y, d.w1.z, d.w1.w, d.w2};
        float la = 0.f, ha = 0.f, lb = 0.f, hb = 0.f;
        // qs byte at pair offset `byte` belongs to block A (2..17) or B (20..35)
#pragma unroll
        for (int D = 0; D < 9; ++D) {
#pragma unroll
            for (int par = 0; par < 2; ++par) {
                const uint32_t s = w[D] >> (8 * par);
                const uint32_t lo = s & 0x000F000Fu;
                const uint32_t hi = s & 0x00F000F0u;
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const int byte = 4 * D + par + 2 * half;
                    const bool in_a = byte >= 2 && byte < 18;
                    const bool in_b = byte >= 20 && byte < 36;
                    if (!in_a && !in_b) continue;
                    const int j = in_a ? byte - 2 : byte - 20;
                    const int e = (in_a ? 0 : 32) + 2 * j;
                    const float nl = half ? h_hi(lo) : h_lo(lo);
                    const float nh = half ? h_hi(hi) : h_lo(hi);
                    if (in_a) {
                        la = __builtin_fmaf(nl, r.v[e], la);
                        ha = __builtin_fmaf(nh, r.v[e + 1], ha);
                    } else {
                        lb = __builtin_fmaf(nl, r.v[e], lb);
                        hb = __builtin_fmaf(nh, r.v[e + 1], hb);
                    }
                }
            }
        }
        const float da = h_lo(w[0]), db = h_lo(w[4] >> 16);
        const float ta = la * kTwo24 + ha * (kTwo24 * 0.0625f) - 8.0f * r.xs_a;
        const float tb = lb * kTwo24 + hb * (kTwo24 * 0.0625f) - 8.0f * r.xs_b;
        return da * ta + db * tb;
    }
};

// ---------------------------------------------------------------------------
// Q5_0: unit = two blocks (44 bytes).  Block A: d @0, qh @2..5, qs @6..21;
// block B: d @22, qh @24..27, qs @28..43.  Element i: low4 = qs[i%16] (low
// nibble for i < 16), high bit = bit i of qh (ref:src/kernels/dequantize.cu:140-164).
// ---------------------------------------------------------------------------
struct GemvQ5_0 {
    static constexpr int kPref1 = 1;  // row-groups in flight per wave at UPL = 1 (8192 x 2048: 5.52 us at 4, 5.14 at 1)
    static constexpr bool kSpread = false;  // one wave per kPref1 row groups above 2048 groups
    static constexpr bool kPairUnits = true;  // 8192 x 2048 5.05 -> 4.99 us, 16384 x 2048 8.14 -> 7.52
    static constexpr int kPairBytes = 44;
    struct Data {
        u32x4 w0, w1;
        uint32_t w8, w9, w10;
    };
    struct Xr {
        float v[64];
        float xs_a, xs_b;
    };
    static __device__ __forceinline__ void load_x(Xr& r, const float* x, int unit) {
        load_x64(r.v, x, unit * 64);
        r.xs_a = sum_range(r.v, 0, 32);
        r.xs_b = sum_range(r.v, 32, 32);
    }
    static __device__ __forceinline__ void load(Data& d, const uint8_t* __restrict__ row, int unit) {
        const uint8_t* p = row + unit * kPairBytes;
        d.w0 = ld_u32x4(p);
        d.w1 = ld_u32x4(p + 16);
        d.w8 = ld_u32(p + 32);
        d.w9 = ld_u32(p + 36);
        d.w10 = ld_u32(p + 40);
    }
    static __device__ __forceinline__ float block(const uint32_t qh, const uint32_t (&qs)[4], const float* v,
                                                  float xs, float dd) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t w = qs[t];
            const uint32_t nlo = ubfe(qh, 4 * t, 4), nhi = ubfe(qh, 16 + 4 * t, 4);
            // spread 4 bits to bit 4 of each byte (no carries between the copies)
            const uint32_t lo = (w & 0x0F0F0F0Fu) | ((nlo * 0x02040810u) & 0x10101010u);
            const uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) | ((nhi * 0x02040810u) & 0x10101010u);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                s0 = __builtin_fmaf(ubyte(lo, b), v[4 * t + b], s0);
                s1 = __builtin_fmaf(ubyte(hi, b), v[16 + 4 * t + b], s1);
            }
        }
        return dd * ((s0 + s1) - 16.0f * xs);
    }
    static __device__ __forceinline__ float dot(const Data& d, const Xr& r, int) {
        const uint32_t w0 = d.w0.x, w1 = d.w0.y, w2 = d.w0.z, w3 = d.w0.w, w4 = d.w1.x, w5 = d.w1.y,
                       w6 = d.w1.z, w7 = d.w1.w;
        const uint32_t qha = align_bytes(w1, w0, 2);
        const uint32_t qsa[4] = {align_bytes(w2, w1, 2), align_bytes(w3, w2, 2), align_bytes(w4, w3, 2),
                                 align_bytes(w5, w4, 2)};
        const uint32_t qsb[4] = {w7, d.w8, d.w9, d.w10};
        const float da = h_lo(w0), db = h_hi(w5);
        return block(qha, qsa, r.v, r.xs_a, da) + block(w6, qsb, r.v + 32, r.xs_b, db);
    }
};

// ---------------------------------------------------------------------------
// Q6_K: unit = (super-block j, 128-chunk c, half h): the 16-element runs
// l in [16h, 16h+16) of the four quarters of chunk c.  Bytes used:
// ql[64c+16h ..+16) (quarters 0/2), ql[64c+32+16h ..+16) (quarters 1/3),
// qh[32c+16h ..+16), scales[8c+2q+h], d (ref:src/kernels/dequantize.cu:218-243).
// Super-blocks are 210 bytes, so odd ones start at 2 mod 4: every field is
// read through dword-aligned windows and funnel-shifted into place.
// ---------------------------------------------------------------------------
struct GemvQ6K {
    static constexpr int kPref1 = 2;  // row-groups in flight per wave at UPL = 1 (lm_head: 46.0 us at 3, 45.3 at 2, 49.8 at 1)
    // one row group per wave up to the wave budget at UPL = 1, whatever N: the
    // decode is long enough that more, shorter waves win (8192 x 2048: 8.20 -> 6.94 us)
    static constexpr bool kSpread = true;
    static constexpr bool kPairUnits = false;
    static constexpr int kBlockBytes = 210;
    struct Data {
        uint32_t a[5], b[5], h[5];  // aligned windows of ql lo-run, ql hi-run, qh
        uint32_t s0, s1, s2;        // window over scales[8c .. 8c+8)
        uint32_t dh;                // d (as 16 bits)
        uint32_t shift;             // byte misalignment of the super-block (0 or 2)
    };
    struct Xr {
        float v[64];  // v[16q + i] = x[256j + 128c + 32q + 16h + i]
        float xs[4];
    };
    static __device__ __forceinline__ void load_x(Xr& r, const float* x, int unit) {
        const int j = unit >> 2, c = (unit >> 1) & 1, h = unit & 1;
        const int k0 = 256 * j + 128 * c + 16 * h;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f32x4 t = *reinterpret_cast<const f32x4*>(x + xpad(k0 + 32 * q + 4 * i));
                r.v[16 * q + 4 * i + 0] = t.x;
                r.v[16 * q + 4 * i + 1] = t.y;
                r.v[16 * q + 4 * i + 2] = t.z;
                r.v[16 * q + 4 * i + 3] = t.w;
            }
#pragma unroll
        for (int q = 0; q < 4; ++q) r.xs[q] = sum_range(r.v, 16 * q, 16);
    }
    static __device__ __forceinline__ void load(Data& d, const uint8_t* __restrict__ row, int unit) {
        const int j = unit >> 2, c = (unit >> 1) & 1, h = unit & 1;
        const uint8_t* p = row + j * kBlockBytes;
        const uint32_t s = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3u);
        d.shift = s;
        const uint8_t* pa = p + 64 * c + 16 * h - s;
        const uint8_t* pb = pa + 32;
        const uint8_t* ph = p + 128 + 32 * c + 16 * h - s;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            d.a[i] = ld_u32(pa + 4 * i);
            d.b[i] = ld_u32(pb + 4 * i);
            d.h[i] = ld_u32(ph + 4 * i);
        }
        const uint8_t* ps = p + 192 + 8 * c - s;
        d.s0 = ld_u32(ps);
        d.s1 = ld_u32(ps + 4);
        d.s2 = s ? ld_u32(ps + 8) : 0u;  // only a misaligned block needs the third dword
        d.dh = *reinterpret_cast<const uint16_t*>(p + 208);
    }
    static __device__ __forceinline__ float dot(const Data& d, const Xr& r, int unit) {
        const uint32_t s = d.shift;
        const int h = unit & 1;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t qa = align_bytes(d.a[t + 1], d.a[t], s);
            const uint32_t qb = align_bytes(d.b[t + 1], d.b[t], s);
            const uint32_t qh = align_bytes(d.h[t + 1], d.h[t], s);
            const uint32_t q0 = (qa & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u);
            const uint32_t q1 = (qb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u);
            const uint32_t q2 = ((qa >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u);
            const uint32_t q3 = ((qb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                acc[0] = __builtin_fmaf(ubyte(q0, b), r.v[0 + 4 * t + b], acc[0]);
                acc[1] = __builtin_fmaf(ubyte(q1, b), r.v[16 + 4 * t + b], acc[1]);
                acc[2] = __builtin_fmaf(ubyte(q2, b), r.v[32 + 4 * t + b], acc[2]);
                acc[3] = __builtin_fmaf(ubyte(q3, b), r.v[48 + 4 * t + b], acc[3]);
            }
        }
        // scales[8c + 2q + h], q = 0..3: bytes h, 2+h, 4+h, 6+h of the 8-byte run
        const uint32_t sc_lo = align_bytes(d.s1, d.s0, s);  // run bytes 0..3
        const uint32_t sc_hi = align_bytes(d.s2, d.s1, s);  // run bytes 4..7
        const float sc0 = sbyte(sc_lo, h), sc1 = sbyte(sc_lo, 2 + h);
        const float sc2 = sbyte(sc_hi, h), sc3 = sbyte(sc_hi, 2 + h);
        const float t = sc0 * (acc[0] - 32.0f * r.xs[0]) + sc1 * (acc[1] - 32.0f * r.xs[1]) +
                        sc2 * (acc[2] - 32.0f * r.xs[2]) + sc3 * (acc[3] - 32.0f * r.xs[3]);
        return h_lo(d.dh) * t;
    }
};

// ---------------------------------------------------------------------------
// FP16 weights: unit = 64 halves (128 bytes); fma(fpext(half), x, acc).
// ---------------------------------------------------------------------------
struct GemvF16 {
    static constexpr int kPref1 = 1;  // row-groups in flight per wave at UPL = 1 (8192 x 2048: 9.08 us at 2, 8.38 at 1)
    static constexpr bool kSpread = false;  // one wave per kPref1 row groups above 2048 groups
    static constexpr bool kPairUnits = false;
    struct Data {
        u32x4 w[8];
    };
    struct Xr {
        float v[64];
    };
    static __device__ __forceinline__ void load_x(Xr& r, const float* x, int unit) {
        load_x64(r.v, x, unit * 64);
    }
    static __device__ __forceinline__ void load(Data& d, const uint8_t* __restrict__ row, int unit) {
        const uint8_t* p = row + unit * 128;
#pragma unroll
        for (int i = 0; i < 8; ++i) d.w[i] = ld_u32x4(p + 16 * i);
    }
    static __device__ __forceinline__ float dot(const Data& d, const Xr& r, int) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t w[4] = {d.w[i].x, d.w[i].y, d.w[i].z, d.w[i].w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                s0 = __builtin_fmaf(h_lo(w[t]), r.v[8 * i + 2 * t], s0);
                s1 = __builtin_fmaf(h_hi(w[t]), r.v[8 * i + 2 * t + 1], s1);
            }
        }
        return s0 + s1;
    }
};

// ---------------------------------------------------------------------------
// FP32 weights (transposed-B GEMV): unit = 64 floats (256 bytes).
// ---------------------------------------------------------------------------
struct GemvF32 {
    static constexpr int kPref1 = 2;  // row-groups in flight per wave at UPL = 1
    static constexpr bool kSpread = false;  // one wave per kPref1 row groups above 2048 groups
    static constexpr bool kPairUnits = false;
    struct Data {
        f32x4 w[16];
    };
    struct Xr {
        float v[64];
    };
    static __device__ __forceinline__ void load_x(Xr& r, const float* x, int unit) {
        load_x64(r.v, x, unit * 64);
    }
    static __device__ __forceinline__ void load(Data& d, const uint8_t* __restrict__ row, int unit) {
        const float* p = reinterpret_cast<const float*>(row) + unit * 64;
#pragma unroll
        for (int i = 0; i < 16; ++i) d.w[i] = ld_f32x4(p + 4 * i);
    }
    static __device__ __forceinline__ float dot(const Data& d, const Xr& r, int) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            s0 = __builtin_fmaf(d.w[i].x, r.v[4 * i + 0], s0);
            s1 = __builtin_fmaf(d.w[i].y, r.v[4 * i + 1], s1);
            s0 = __builtin_fmaf(d.w[i].z, r.v[4 * i + 2], s0);
            s1 = __builtin_fmaf(d.w[i].w, r.v[4 * i + 3], s1);
        }
        return s0 + s1;
    }
};

}  // namespace dev
}  // namespace cri

// mfma_gemm.hip -- fused dequant GEMM on the matrix cores for multi-token
// (prefill) batches: C[M,N] = A[M,K] * dequant(B[N,K])^T, every weight format.
// The C ABI sends it the prefill shapes that the register-decode kernel of
// prefill.hip does not take: K % 64 == 0 but K % 256 != 0 (e.g. K = 576), or
// activations that are not 16-byte aligned.
//
// The reference computes the same product with one fp32 FMA chain per output
// (ref:src/kernels/matmul_quant.cu:64-130 Q8_0, :142-204 Q4_0, :216-297 Q5_0,
// :309-386 Q4_K, :398-498 Q6_K, :510-558 FP16).  Here:
//   * a workgroup owns a 128(n) x 128(m) output tile, its four waves 64 x 64
//     each (4 x 4 v_mfma_f32_16x16x32_f16 tiles, 64 fp32 accumulators);
//   * the k loop advances 64 columns per step.  Every thread decodes one
//     32-element run of one weight row (a Q8_0/Q4_0/Q5_0 block, a Q4_K
//     sub-block, a Q6_K quarter chunk or 32 fp16 values) and converts eight
//     4-element pieces of activation rows (16 lanes cover one row's 256
//     bytes, so each load instruction touches 4 rows), both to fp16, into
//     LDS.  LDS is
//     double-buffered and the next step's global loads are in flight during
//     the current step's 32 MFMAs, so each step has one barrier;
//   * LDS rows hold 64 halves (128 B) with the 16-byte chunks swizzled by
//     row, so the staging writes and the ds_read_b128 operand fetches are
//     free of bank conflicts;
//   * weights are the MFMA A operand (rows of the product are n), activations
//     the B operand, so each lane ends with 4 consecutive n of one row m and
//     stores them as one 16-byte write;
//   * workgroup ids are remapped so that the 32 workgroups an XCD runs at a
//     time are consecutive tiles sharing activation rows (each XCD has its own
//     L2).  When the tiles cannot fill 256 CUs the k range is split over
//     workgroups and partial tiles are added into a zeroed C with fp32 atomics.
// Numerics: each weight is the reference's dequantized value rounded once to
// fp16 (Q8_0/Q4_0/Q5_0/FP16 exactly that; Q4_K/Q6_K evaluate d*sc*q - dmin*mn
// in fp16 arithmetic with one or two roundings), each activation is rounded
// to fp16 (relative 2^-11), products are exact and sums are fp32, so outputs
// agree with the fp32 reference to about 2e-4 normwise; the stated tolerance
// is 1e-3.  Operands must stay within the fp16 range (|x| < 65504).
#include <atomic>

#include "common.hpp"
#include "decode.hpp"
#include "internal.hpp"

namespace cri {
namespace dev {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kTileM = 128, kTileN = 128, kStepK = 64;
constexpr int kThreads = 512;
constexpr int kOperandBytes = 128 * kStepK * 2;       // one operand tile, one stage
constexpr int kStageBytes = 2 * kOperandBytes;        // activations + weights
constexpr int kLdsBytes = 3 * kStageBytes;            // three-stage ring

constexpr uint32_t kMagic = 0x64646464u;              // bytes 0x64: fp16 1024 + byte when paired

__device__ __forceinline__ uint32_t hsplat_bits(_Float16 v) {
    const uint32_t b = __builtin_bit_cast(uint16_t, v);
    return b | (b << 16);
}
__device__ __forceinline__ uint32_t pk_add(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a) + __builtin_bit_cast(h2, b));
}
__device__ __forceinline__ uint32_t pk_mul(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a) * __builtin_bit_cast(h2, b));
}
__device__ __forceinline__ uint32_t pk_fma(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b),
                                                                  __builtin_bit_cast(h2, c)));
}
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}
__device__ __forceinline__ uint32_t alignb(uint32_t hi, uint32_t lo, uint32_t shift) {
    return __builtin_amdgcn_alignbyte(hi, lo, shift);
}
// bytes b0 and b1 (or b2 and b3) of w as the fp16 pair (1024 + b0, 1024 + b1)
__device__ __forceinline__ uint32_t magic_lo(uint32_t w) { return perm(kMagic, w, 0x04010400u); }
__device__ __forceinline__ uint32_t magic_hi(uint32_t w) { return perm(kMagic, w, 0x04030402u); }

// LDS rows are 128 bytes (64 halves) of eight 16-byte chunks; chunk c of row
// r is stored in slot c ^ (r & 7) ^ ((r >> 3) & 1).  It depends on r mod 16
// only; measured on gfx950 (SQ_LDS_BANK_CONFLICT = 0) it is conflict-free for
// the 32 x 16 operand fetches of v_mfma_f32_32x32x16_f16 (32 consecutive
// rows, one chunk per half-wave), for the weight staging writes (64
// consecutive rows, one chunk) and the activation staging writes (16 lanes
// per row), and the operand fetches run about 25% faster than with c ^ (r & 7).
__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int lds_off(int r, int c) { return (r << 7) + ((c ^ swz(r)) << 4); }

// ---------------------------------------------------------------------------
// Weight stagers.  load(): the global loads of one thread's 32-element run of
// row `row` at k step `step` (h = which half of the 64 columns; wave-uniform).
// convert(): the 32 fp16 values in k order, packed two per dword.

// ref:src/kernels/dequantize.cu:45-47 -- x = d * q, q int8.  Two 34-byte blocks
// per step; the pair starts 4-byte aligned, the second block 2 bytes off.
struct WQ8_0 {
    static constexpr int kFmt = kFmtQ8_0;
    static constexpr int kRegs = 9;
    static __device__ __forceinline__ void load(uint32_t (&w)[kRegs], const uint8_t* row, int step, int h) {
        const uint8_t* p = row + step * 68 + 32 * h;
        const u32x4 a = ld_u32x4(p), b = ld_u32x4(p + 16);
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
        w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
        w[8] = ld_u32(p + 32);
    }
    template <int H>
    static __device__ __forceinline__ void convert(const uint32_t (&w)[kRegs], int, uint32_t (&o)[16]) {
        uint32_t d, q[8];
        if constexpr (H == 0) {
            d = w[0] & 0xFFFFu;
#pragma unroll
            for (int i = 0; i < 8; ++i) q[i] = alignb(w[i + 1], w[i], 2);
        } else {
            d = w[0] >> 16;
#pragma unroll
            for (int i = 0; i < 8; ++i) q[i] = w[i + 1];
        }
        const uint32_t d2 = d | (d << 16);
        const uint32_t bias = hsplat_bits(static_cast<_Float16>(-1152.0f));  // 1024 + 128
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t x = q[i] ^ 0x80808080u;  // int8 -> q + 128
            o[2 * i] = pk_mul(pk_add(magic_lo(x), bias), d2);
            o[2 * i + 1] = pk_mul(pk_add(magic_hi(x), bias), d2);
        }
    }
};

// ref:src/kernels/dequantize.cu:84-100 -- element e <- qs[e/2], low nibble for
// even e; x = d * (nib - 8).  18-byte blocks, pair of 36 bytes per step.
struct WQ4_0 {
    static constexpr int kFmt = kFmtQ4_0;
    static constexpr int kRegs = 5;
    static __device__ __forceinline__ void load(uint32_t (&w)[kRegs], const uint8_t* row, int step, int h) {
        const uint8_t* p = row + step * 36 + 16 * h;
        const u32x4 a = ld_u32x4(p);
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
        w[4] = ld_u32(p + 16);
    }
    template <int H>
    static __device__ __forceinline__ void convert(const uint32_t (&w)[kRegs], int, uint32_t (&o)[16]) {
        uint32_t d, q[4];
        if constexpr (H == 0) {
            d = w[0] & 0xFFFFu;
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = alignb(w[i + 1], w[i], 2);
        } else {
            d = w[0] >> 16;
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = w[i + 1];
        }
        const uint32_t d2 = d | (d << 16);
        const uint32_t bias = hsplat_bits(static_cast<_Float16>(-1032.0f));  // 1024 + 8
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t u = q[i] & 0x0F0F0F0Fu, v = (q[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                // (low nibble, high nibble) of byte b = elements 8i + 2b, 8i + 2b + 1
                const uint32_t sel = static_cast<uint32_t>(b) | (0x0Cu << 8) | ((4u + b) << 16) | (0x0Cu << 24);
                const uint32_t pair = perm(v, u, sel) | 0x64006400u;
                o[4 * i + b] = pk_mul(pk_add(pair, bias), d2);
            }
        }
    }
};

// ref:src/kernels/dequantize.cu:137-164 -- low nibble of qs[e] for e < 16, high
// nibble of qs[e-16] otherwise, bit e of the little-endian qh as bit 4;
// x = d * (q5 - 16).  22-byte blocks, pair of 44 bytes per step.
struct WQ5_0 {
    static constexpr int kFmt = kFmtQ5_0;
    static constexpr int kRegs = 6;
    static __device__ __forceinline__ void load(uint32_t (&w)[kRegs], const uint8_t* row, int step, int h) {
        const uint8_t* p = row + step * 44 + 20 * h;
        const u32x4 a = ld_u32x4(p);
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
        const u32x2_a4 b = *reinterpret_cast<const u32x2_a4*>(p + 16);
        w[4] = b.x; w[5] = b.y;
    }
    // four bits t (< 16) to bit 4 of four bytes
    static __device__ __forceinline__ uint32_t spread4(uint32_t t) { return ((t * 0x00204081u) & 0x01010101u) << 4; }
    template <int H>
    static __device__ __forceinline__ void convert(const uint32_t (&w)[kRegs], int, uint32_t (&o)[16]) {
        uint32_t d, qh, q[4];
        if constexpr (H == 0) {
            d = w[0] & 0xFFFFu;
            qh = alignb(w[1], w[0], 2);
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = alignb(w[i + 2], w[i + 1], 2);
        } else {
            d = w[0] >> 16;
            qh = w[1];
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = w[i + 2];
        }
        const uint32_t d2 = d | (d << 16);
        const uint32_t bias = hsplat_bits(static_cast<_Float16>(-1040.0f));  // 1024 + 16
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t u = (q[i] & 0x0F0F0F0Fu) | spread4((qh >> (4 * i)) & 0xFu);
            const uint32_t v = ((q[i] >> 4) & 0x0F0F0F0Fu) | spread4((qh >> (16 + 4 * i)) & 0xFu);
            o[2 * i] = pk_mul(pk_add(magic_lo(u), bias), d2);
            o[2 * i + 1] = pk_mul(pk_add(magic_hi(u), bias), d2);
            o[8 + 2 * i] = pk_mul(pk_add(magic_lo(v), bias), d2);
            o[9 + 2 * i] = pk_mul(pk_add(magic_hi(v), bias), d2);
        }
    }
};

// ref:src/kernels/dequantize.cu:289-324 -- super-block of 256: d, dmin, 12
// bytes of 6-bit (sc, mn) pairs, 128 bytes of nibbles; element 64j + l
// (l < 32) is the low nibble of qs[32j + l] in sub-block 2j, element
// 64j + 32 + l its high nibble in sub-block 2j + 1; x = d*sc*q - dmin*mn.
// One k step = one 64-element chunk j; h picks the sub-block.
struct WQ4_K {
    static constexpr int kFmt = kFmtQ4_K;
    static constexpr int kRegs = 12;
    static __device__ __forceinline__ void load(uint32_t (&w)[kRegs], const uint8_t* row, int step, int h) {
        const uint8_t* sb = row + (step >> 2) * 144;
        const u32x4 hd = ld_u32x4(sb);
        const uint8_t* qs = sb + 16 + (step & 3) * 32;
        const u32x4 a = ld_u32x4(qs), b = ld_u32x4(qs + 16);
        w[0] = hd.x; w[1] = hd.y; w[2] = hd.z; w[3] = hd.w;
        w[4] = a.x; w[5] = a.y; w[6] = a.z; w[7] = a.w;
        w[8] = b.x; w[9] = b.y; w[10] = b.z; w[11] = b.w;
    }
    template <int H>
    static __device__ __forceinline__ void convert(const uint32_t (&w)[kRegs], int step, uint32_t (&o)[16]) {
        const int s = 2 * (step & 3) + H;  // sub-block, wave-uniform
        // scales[i] by shifts of register values (no indexed access to w), and
        // both encodings evaluated then selected, so the loop body has no branch
        const uint64_t s07 = (static_cast<uint64_t>(w[2]) << 32) | w[1];
        const int s4 = s & 3;
        const uint32_t b_s = static_cast<uint32_t>(s07 >> (8 * s)) & 0xFFu;              // scales[s]
        const uint32_t b_s4 = static_cast<uint32_t>(s07 >> (8 * s4 + 32)) & 0xFFu;        // scales[s + 4], s < 4
        const uint32_t b_hi = (w[3] >> (8 * s4)) & 0xFFu;                                 // scales[s + 4], s >= 4
        const uint32_t b_lo = static_cast<uint32_t>(s07 >> (8 * s4)) & 0xFFu;             // scales[s - 4], s >= 4
        const bool low = s < 4;
        const uint32_t sc = low ? (b_s & 63u) : ((b_hi & 15u) | ((b_lo >> 6) << 4));
        const uint32_t mn = low ? (b_s4 & 63u) : ((b_hi >> 4) | ((b_s >> 6) << 4));
        const uint32_t dd = w[0] & 0xFFFFu;
        const float dmin = h_hi(w[0]);
        const uint32_t d2 = dd | (dd << 16);
        const uint32_t sc2 = hsplat_bits(static_cast<_Float16>(static_cast<float>(sc)));
        const uint32_t scb = hsplat_bits(static_cast<_Float16>(-1024.0f * static_cast<float>(sc)));
        const uint32_t mn2 = hsplat_bits(static_cast<_Float16>(-dmin * static_cast<float>(mn)));
        constexpr int sh = 4 * H;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t u = (w[4 + i] >> sh) & 0x0F0F0F0Fu;
            // (1024 + q) * sc - 1024 * sc = sc * q exactly (<= 945), then d*(sc*q) - dmin*mn
            o[2 * i] = pk_fma(pk_fma(magic_lo(u), sc2, scb), d2, mn2);
            o[2 * i + 1] = pk_fma(pk_fma(magic_hi(u), sc2, scb), d2, mn2);
        }
    }
};

// ref:src/kernels/dequantize.cu:215-243 -- super-block of 256 (210 bytes, d
// last): element 128c + 32q + l takes the low (q < 2) or high nibble of
// ql[64c + 32(q&1) + l] and bits 2q..2q+1 of qh[32c + l]; scale int8
// scales[8c + 2q + l/16]; x = d * sc * (q6 - 32).  One k step = one half
// (c, q in {0,1} or {2,3}) of a 128-element chunk; h picks q within it.  The
// super-blocks are only 2-byte aligned, so the loads funnel-shift.
struct WQ6_K {
    static constexpr int kFmt = kFmtQ6_K;
    static constexpr int kRegs = 20;
    static __device__ __forceinline__ void load(uint32_t (&w)[kRegs], const uint8_t* row, int step, int h) {
        const uint8_t* sb = row + (step >> 2) * 210;
        const int j = step & 3, c = j >> 1, q = 2 * (j & 1) + h;
        const uint8_t* pl = sb + 32 * (q & 1) + 64 * c;
        const uint8_t* ph = sb + 128 + 32 * c;
        const uint8_t* al = reinterpret_cast<const uint8_t*>(reinterpret_cast<uintptr_t>(pl) & ~uintptr_t(3));
        const uint8_t* ah = reinterpret_cast<const uint8_t*>(reinterpret_cast<uintptr_t>(ph) & ~uintptr_t(3));
        const u32x4 l0 = ld_u32x4(al), l1 = ld_u32x4(al + 16);
        const u32x4 q0 = ld_u32x4(ah), q1 = ld_u32x4(ah + 16);
        w[0] = l0.x; w[1] = l0.y; w[2] = l0.z; w[3] = l0.w; w[4] = l1.x; w[5] = l1.y; w[6] = l1.z; w[7] = l1.w;
        w[8] = ld_u32(al + 32);  // stays inside the super-block: pl + 32 <= sb + 128
        w[9] = q0.x; w[10] = q0.y; w[11] = q0.z; w[12] = q0.w; w[13] = q1.x; w[14] = q1.y; w[15] = q1.z; w[16] = q1.w;
        w[17] = ld_u32(ah + 32);  // ph + 32 <= sb + 192
        // the two 32-byte runs have the same byte shift: sb is even and the offsets are multiples of 32
        // two int8 scales and d, 16-bit loads (even addresses)
        const uint32_t scales = *reinterpret_cast<const uint16_t*>(sb + 192 + 8 * c + 2 * q);
        w[18] = scales | (static_cast<uint32_t>(reinterpret_cast<uintptr_t>(pl) & 3) << 16);  // + byte shift
        w[19] = *reinterpret_cast<const uint16_t*>(sb + 208);
    }
    template <int H>
    static __device__ __forceinline__ void convert(const uint32_t (&w)[kRegs], int step, uint32_t (&o)[16]) {
        const int q = 2 * (step & 1) + H;
        const uint32_t shift = w[18] >> 16;
        const int sc0 = static_cast<int8_t>(w[18] & 0xFFu), sc1 = static_cast<int8_t>((w[18] >> 8) & 0xFFu);
        const uint32_t dd = w[19] & 0xFFFFu;
        const uint32_t d2 = dd | (dd << 16);
        const uint32_t s0 = hsplat_bits(static_cast<_Float16>(static_cast<float>(sc0)));
        const uint32_t s1 = hsplat_bits(static_cast<_Float16>(static_cast<float>(sc1)));
        const uint32_t bias = hsplat_bits(static_cast<_Float16>(-1056.0f));  // 1024 + 32
        const int lsh = 4 * (q >> 1), hsh = 2 * q;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t ql = alignb(w[i + 1], w[i], shift);
            const uint32_t qh = alignb(w[10 + i], w[9 + i], shift);
            const uint32_t u = ((ql >> lsh) & 0x0F0F0F0Fu) | (((qh >> hsh) & 0x03030303u) << 4);
            const uint32_t sc = i < 4 ? s0 : s1;
            // (q6 - 32) exact; times sc (exact while |sc*(q6-32)| <= 2048); times d
            o[2 * i] = pk_mul(pk_mul(pk_add(magic_lo(u), bias), sc), d2);
            o[2 * i + 1] = pk_mul(pk_mul(pk_add(magic_hi(u), bias), sc), d2);
        }
    }
};

// ref:src/kernels/matmul_quant.cu:510-558 -- fp16 weights, used as they are.
struct WF16 {
    static constexpr int kFmt = kFmtF16;
    static constexpr int kRegs = 16;
    static __device__ __forceinline__ void load(uint32_t (&w)[kRegs], const uint8_t* row, int step, int h) {
        const uint8_t* p = row + step * 128 + 64 * h;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 a = ld_u32x4(p + 16 * i);
            w[4 * i] = a.x; w[4 * i + 1] = a.y; w[4 * i + 2] = a.z; w[4 * i + 3] = a.w;
        }
    }
    template <int H>
    static __device__ __forceinline__ void convert(const uint32_t (&w)[kRegs], int, uint32_t (&o)[16]) {
#pragma unroll
        for (int i = 0; i < 16; ++i) o[i] = w[i];
    }
};

// Staging registers of one thread for one k step: four 4-float pieces of
// activations (every thread) and, for the weight stagers, one weight run.
template <class W, bool WST>
struct Stage;
template <class W>
struct Stage<W, true> {
    f32x4 a[4];
    uint32_t w[W::kRegs];
};
template <class W>
struct Stage<W, false> {
    f32x4 a[4];
};

// One workgroup's share: output tile (mt, nt) over k steps [s_begin, s_end).
struct TileJob {
    const float* A;
    const uint8_t* B;
    float* C;
    int M, N, K;
    long row_bytes;
    int mt, nt, s_begin, s_end;
    int atomic, vec_store;
};

// Eight waves, wave = 4 a + 2 b + c.  Both roles are compile-time per wave so
// the loop body has no branches and every register index is static:
//   staging: every thread converts four 16-byte pieces of activation rows
//            (16 lanes per 256-byte row piece); waves with a = 0 also stage
//            weight rows [64 b, 64 b + 64), columns [32 c, 32 c + 32) of
//            each step;
//   compute: (wm, wn, wk) = (b, a, c): m rows [64 wm, +64) x n rows [64 wn,
//            +64) over k sub-steps 2 wk, 2 wk + 1 (16 columns each) of every
//            step, as 2 x 2 tiles of v_mfma_f32_32x32x16_f16.  The two k
//            halves (waves w and w ^ 1) are added through LDS at the end.
// The two waves on a SIMD (w and w + 4) are one weight stager and one other,
// so conversion work is even across SIMDs.
template <class W, bool AST, int WK>
__device__ __forceinline__ void run_tile(const TileJob& J, char* lds) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wb = __builtin_amdgcn_readfirstlane((tid >> 7) & 1);
    constexpr int H = WK;

    // staging roles
    const uint8_t* wrow = nullptr;
    int wst = 0;
    if constexpr (!AST) {
        const int srow = (wb << 6) + lane;
        wrow = J.B + static_cast<long>(min(J.nt * kTileN + srow, J.N - 1)) * J.row_bytes;
        wst = lds_off(srow, 4 * H);  // chunk 4H + c is at wst ^ (c << 4)
    }
    const int acol = tid & 15;
    const int arow0 = tid >> 4;  // 0..31; rows arow0 + 32 i
    const float* abase = J.A + static_cast<long>(acol) * 4;
    int aoff[4];  // element offsets of the staged activation rows (M * K < 2^31)
#pragma unroll
    for (int i = 0; i < 4; ++i) aoff[i] = min(J.mt * kTileM + arow0 + 32 * i, J.M - 1) * J.K;
    const int ast = lds_off(arow0, acol >> 1) + 8 * (acol & 1);  // + 32 i rows = + 4096 i bytes

    // compute role.  A 32 x 16 operand: lane reads row base + (lane & 31),
    // 16-byte chunk 2 ks + (lane >> 5); base is a multiple of 32, so the
    // swizzled slot is (2 ks + (lane >> 5)) ^ swz(lane & 31).
    const int wm = wb;
    constexpr int wn = AST ? 1 : 0;
    const int fr = lane & 31, fc = lane >> 5;
    int fb[2];
#pragma unroll
    for (int kq = 0; kq < 2; ++kq) fb[kq] = (fr << 7) + (((2 * (2 * WK + kq) + fc) ^ swz(fr)) << 4);

    f16v acc[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[t][u][r] = 0.0f;

    auto load = [&](Stage<W, !AST>& st, int step) {
        const float* ap = abase + step * kStepK;
#pragma unroll
        for (int i = 0; i < 4; ++i) st.a[i] = ld_f32x4(ap + aoff[i]);
        if constexpr (!AST) W::load(st.w, wrow, step, H);
    };
    // valid = false (the padding step of an odd step count) stores zero
    // activations, so that step's MFMAs add nothing.
    float amax[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // largest |activation| of the staged rows
    auto stage_store = [&](const Stage<W, !AST>& st, int step, char* buf, bool valid) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f4 v = st.a[i];
            const float mx = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
            amax[i] = valid ? fmaxf(amax[i], mx) : amax[i];
            const uint32_t lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{st.a[i].x, st.a[i].y}, h2));
            const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{st.a[i].z, st.a[i].w}, h2));
            *reinterpret_cast<u32x2*>(buf + ast + 4096 * i) = u32x2{valid ? lo : 0u, valid ? hi : 0u};
        }
        if constexpr (!AST) {
            char* wbuf = buf + kOperandBytes;
            uint32_t o[16];
            W::template convert<H>(st.w, step, o);
#pragma unroll
            for (int c = 0; c < 4; ++c)
                *reinterpret_cast<u32x4*>(wbuf + (wst ^ (c << 4))) =
                    u32x4{o[4 * c], o[4 * c + 1], o[4 * c + 2], o[4 * c + 3]};
        }
    };

    struct Opnd {
        half8 w[2][2], a[2][2];
    };
    auto read_opnd = [&](Opnd& R, const char* buf) {
        const char* abuf = buf;
        const char* wbuf = buf + kOperandBytes;
#pragma unroll
        for (int kq = 0; kq < 2; ++kq) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
                R.w[kq][t] = *reinterpret_cast<const half8*>(wbuf + fb[kq] + ((wn * 64 + 32 * t) << 7));
#pragma unroll
            for (int u = 0; u < 2; ++u)
                R.a[kq][u] = *reinterpret_cast<const half8*>(abuf + fb[kq] + ((wm * 64 + 32 * u) << 7));
        }
    };
    auto mma = [&](const Opnd& R) {
#pragma unroll
        for (int kq = 0; kq < 2; ++kq)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int u = 0; u < 2; ++u)
                    acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(R.w[kq][t], R.a[kq][u], acc[t][u], 0, 0, 0);
    };

    // Pipeline over relative steps t = s - s_begin, three LDS buffers (step t
    // lives in buffer t % 3), two operand and two staging register sets.  At
    // the top of iteration t the operands of step t are in registers, step
    // t + 1 is in LDS and the global loads of step t + 2 are in flight.
    // Iteration t runs step t's MFMAs and, between them, issues the loads of
    // step t + 3, reads step t + 1's operands and converts step t + 2 into
    // LDS; it syncs once, and the MFMAs after each barrier never wait on LDS.  The loop runs an even number of iterations (one loop exit
    // keeps the accumulators in one register set); an odd step count gets a
    // padding step of zero activations.  Loads past the end repeat the last
    // step (in bounds).
    const int nst = J.s_end - J.s_begin;
    const int nst2 = (nst + 1) & ~1;
    auto step_of = [&](int t) { return J.s_begin + min(t, nst - 1); };
    auto buf_of = [&](int t) { return lds + (t % 3) * kStageBytes; };
    Stage<W, !AST> S0, S1;
    Opnd R0, R1;
    load(S0, step_of(0));
    load(S1, step_of(1));
    stage_store(S0, J.s_begin, buf_of(0), true);
    stage_store(S1, J.s_begin + 1, buf_of(1), nst > 1);
    load(S0, step_of(2));
    __syncthreads();
    read_opnd(R0, buf_of(0));

    auto iter = [&](Opnd& Rc, Opnd& Rn, Stage<W, !AST>& Sc, Stage<W, !AST>& Sn, int t) {
        mma(Rc);
        load(Sn, step_of(t + 3));
        read_opnd(Rn, buf_of(t + 1));
        stage_store(Sc, J.s_begin + t + 2, buf_of(t + 2), t + 2 < nst);
        // Spread the loads, operand reads, conversion and staging writes
        // between the MFMAs, so the wave keeps issuing while each MFMA runs.
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);  // VMEM read
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
            __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);  // VALU
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
        }
        __syncthreads();
    };
    for (int t = 0; t < nst2; t += 2) {
        iter(R0, R1, S0, S1, t);
        iter(R1, R0, S1, S0, t + 1);
    }

    // Rows whose activations left fp16's comfortable range (>= 65504 is inf; a
    // nonzero row below 2^-10 keeps only subnormal precision) are flagged in an
    // LDS area above the staged C tile; their fp16 results are not stored and
    // they are recomputed in fp32 at the end.
    int* const rowflag = reinterpret_cast<int*>(lds + kLdsBytes) - kTileM;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float v = amax[i];
        v = fmaxf(v, __shfl_xor(v, 1));
        v = fmaxf(v, __shfl_xor(v, 2));
        v = fmaxf(v, __shfl_xor(v, 4));
        v = fmaxf(v, __shfl_xor(v, 8));
        if (acol == 0) rowflag[arow0 + 32 * i] = (v >= 65504.0f || (v > 0.0f && v < 0x1p-10f)) ? 1 : 0;
    }

    // Add the two k halves: wave (wm, wn, wk) keeps n tile t = wk and hands
    // t = 1 - wk to its partner (wave ^ 1) through LDS (8 KB per wave).
    constexpr int keep = WK, give = 1 - WK;
    const int pair = (tid >> 7);  // = 2 a + b, one LDS slot pair per (wm, wn)
    float* mine = reinterpret_cast<float*>(lds) + (pair * 2 + WK) * 2048;        // written by the partner
    float* theirs = reinterpret_cast<float*>(lds) + (pair * 2 + (1 - WK)) * 2048;  // read by the partner
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) theirs[(u * 16 + r) * 64 + lane] = acc[give][u][r];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[keep][u][r] += mine[(u * 16 + r) * 64 + lane];

    // The finished 128 x 128 tile goes through LDS so that the global accesses
    // run along rows: a lane's own values (C[m][n .. n+3], n = 32 keep + 8 g +
    // 4 fc, m = 32 u + fr in the wave's 64 x 64 block) sit 32 rows apart, and
    // an fp32 atomic add per lane in that layout touches 32 cache lines per
    // instruction (measured: the split-K adds of a 512 x 2048 x 8192 GEMM took
    // 86 us this way).  Read back along rows, an instruction covers 64
    // consecutive floats (atomics) or two full 512-byte rows (stores).
    constexpr int kCS = kTileN + 4;  // row stride (floats) of the staged tile
    static_assert(kTileM * kCS * 4 + kTileM * 4 <= kLdsBytes, "the staged C tile and the row flags must fit in the LDS ring");
    float* ct = reinterpret_cast<float*>(lds);
    __syncthreads();  // every partner read of the k-half exchange is done
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int ml = wm * 64 + 32 * u + fr, nl = wn * 64 + 32 * keep + 8 * g + 4 * fc;
            *reinterpret_cast<f4*>(ct + ml * kCS + nl) =
                f4{acc[keep][u][4 * g], acc[keep][u][4 * g + 1], acc[keep][u][4 * g + 2], acc[keep][u][4 * g + 3]};
        }
    __syncthreads();
    const int m0 = J.mt * kTileM, n0 = J.nt * kTileN;
    if (J.atomic) {
        const int c = tid & 127, n = n0 + c;
#pragma unroll 8
        for (int i = 0; i < kTileM / 4; ++i) {
            const int r = (tid >> 7) + 4 * i, m = m0 + r;
            if (m < J.M && n < J.N && !rowflag[r]) atomicAdd(J.C + static_cast<long>(m) * J.N + n, ct[r * kCS + c]);
        }
    } else if (J.vec_store) {  // N % 4 == 0, C 16-byte aligned
        const int c = (tid & 31) * 4, n = n0 + c;
#pragma unroll
        for (int i = 0; i < kTileM / 16; ++i) {
            const int r = (tid >> 5) + 16 * i, m = m0 + r;
            if (m < J.M && n < J.N && !rowflag[r])
                *reinterpret_cast<f4*>(J.C + static_cast<long>(m) * J.N + n) = *reinterpret_cast<const f4*>(ct + r * kCS + c);
        }
    } else {
        const int c = tid & 127, n = n0 + c;
#pragma unroll 8
        for (int i = 0; i < kTileM / 4; ++i) {
            const int r = (tid >> 7) + 4 * i, m = m0 + r;
            if (m < J.M && n < J.N && !rowflag[r]) J.C[static_cast<long>(m) * J.N + n] = ct[r * kCS + c];
        }
    }

    // fp32 path for flagged rows: thread -> column n0 + (tid & 127) of the flagged rows
    // r = tid >> 7 (mod 4), the reference's per-element decode and a sequential fp32 sum over
    // this workgroup's k range
    for (int r = tid >> 7; r < kTileM; r += 4) {
        if (!rowflag[r]) continue;  // uniform over each wave
        const int m = m0 + r, n = n0 + (tid & 127);
        if (m >= J.M || n >= J.N) continue;
        const float* x = J.A + static_cast<long>(m) * J.K;
        const uint8_t* wp = J.B + static_cast<long>(n) * J.row_bytes;
        float sum = 0.0f;
        for (int k = J.s_begin * kStepK; k < J.s_end * kStepK; ++k)
            sum = __builtin_fmaf(x[k], decode_row_elem(W::kFmt, wp, k), sum);
        float* cp = J.C + static_cast<long>(m) * J.N + n;
        if (J.atomic)
            atomicAdd(cp, sum);
        else
            *cp = sum;
    }
}

template <class W>
__global__ __launch_bounds__(kThreads) void mfma_gemm_kernel(const float* __restrict__ A, const uint8_t* __restrict__ B,
                                                             float* __restrict__ C, int M, int N, int K, long row_bytes,
                                                             int MT, int NT, int steps_per_split, int remap,
                                                             int atomic, int vec_store) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    int bid = blockIdx.x;
    if (remap) {  // XCD x (= bid % 8) runs a contiguous run of tiles
        const int per_xcd = gridDim.x >> 3;
        bid = (bid & 7) * per_xcd + (bid >> 3);
    }
    TileJob J;
    J.nt = bid % NT;
    const int rest = bid / NT;
    J.mt = rest % MT;
    const int ks = rest / MT;
    J.s_begin = ks * steps_per_split;
    J.s_end = min(K / kStepK, J.s_begin + steps_per_split);
    if (J.s_begin >= J.s_end) return;
    J.A = A; J.B = B; J.C = C;
    J.M = M; J.N = N; J.K = K;
    J.row_bytes = row_bytes;
    J.atomic = atomic; J.vec_store = vec_store;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    switch ((wave >> 2) * 2 + (wave & 1)) {
        case 0: run_tile<W, false, 0>(J, lds); break;
        case 1: run_tile<W, false, 1>(J, lds); break;
        case 2: run_tile<W, true, 0>(J, lds); break;
        default: run_tile<W, true, 1>(J, lds); break;
    }
}

}  // namespace
}  // namespace dev

namespace detail {

bool mfma_gemm_supported(int fmt, int M, int N, int K, const void* A, const void* B) {
    (void)N;
    if (fmt < kFmtQ8_0 || fmt > kFmtF16) return false;
    if (M < 1 || K < dev::kStepK || K % dev::kStepK != 0) return false;
    if (static_cast<long>(M) * K >= (1L << 31)) return false;  // 32-bit activation offsets
    return (reinterpret_cast<uintptr_t>(B) & 3) == 0 && (reinterpret_cast<uintptr_t>(A) & 3) == 0;
}

namespace {

// The kernels use more than the default 64 KB of dynamic LDS; the limit is
// raised once per kernel and device.
template <class W>
int launch_w(dim3 grid, hipStream_t stream, const float* A, const uint8_t* B, float* C, int M, int N, int K, long rb,
             int MT, int NT, int sps, int remap, int atomic, int vec) {
    constexpr int kMaxDevices = 64;
    static std::atomic<bool> ready[kMaxDevices];
    int devid = 0;
    if (hipGetDevice(&devid) != hipSuccess || devid < 0 || devid >= kMaxDevices) return kFailed;
    if (!ready[devid].load(std::memory_order_acquire)) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&dev::mfma_gemm_kernel<W>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, dev::kLdsBytes) != hipSuccess)
            return kFailed;
        ready[devid].store(true, std::memory_order_release);
    }
    hipLaunchKernelGGL(dev::mfma_gemm_kernel<W>, grid, dim3(dev::kThreads), dev::kLdsBytes, stream, A, B, C, M, N, K,
                       rb, MT, NT, sps, remap, atomic, vec);
    return 0;  // the launch's own status is read by the caller (hipGetLastError)
}

}  // namespace

int launch_mfma_gemm(int fmt, const float* A, const void* B, float* C, int M, int N, int K, hipStream_t stream) {
    const int MT = (M + dev::kTileM - 1) / dev::kTileM;
    const int NT = (N + dev::kTileN - 1) / dev::kTileN;
    const long tiles = static_cast<long>(MT) * NT;
    const int nsteps = K / dev::kStepK;
    int ks = 1;
    // split k while the tiles alone leave CUs idle, keeping >= 8 steps per split
    while (tiles * ks < 256 && nsteps >= 16 * ks) ks *= 2;
    const int sps = (nsteps + ks - 1) / ks;
    ks = (nsteps + sps - 1) / sps;
    const long grid = tiles * ks;
    if (grid > 0x7FFFFFFFL) return -1;
    const int remap = (grid % 8 == 0) ? 1 : 0;
    const int atomic = ks > 1 ? 1 : 0;
    const int vec = (N % 4 == 0 && (reinterpret_cast<uintptr_t>(C) & 15) == 0) ? 1 : 0;
    if (atomic) launch_fill_zero(C, static_cast<long>(M) * N, stream);
    const uint8_t* Bb = static_cast<const uint8_t*>(B);
    const long rb = row_bytes(fmt, K);
    const dim3 g(static_cast<unsigned>(grid));
    switch (fmt) {
        case kFmtQ8_0: return launch_w<dev::WQ8_0>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, atomic, vec);
        case kFmtQ4_0: return launch_w<dev::WQ4_0>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, atomic, vec);
        case kFmtQ5_0: return launch_w<dev::WQ5_0>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, atomic, vec);
        case kFmtQ4_K: return launch_w<dev::WQ4_K>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, atomic, vec);
        case kFmtQ6_K: return launch_w<dev::WQ6_K>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, atomic, vec);
        case kFmtF16: return launch_w<dev::WF16>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, atomic, vec);
    }
    return -1;
}

}  // namespace detail
}  // namespace cri

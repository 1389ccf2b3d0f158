// prefill.hip -- fused dequant GEMM for multi-token (prefill) batches on the
// matrix cores, C[M,N] = A[M,K] * dequant(B[N,K])^T, for Q4_K, Q8_0, Q6_K,
// Q4_0, Q5_0 and FP16 weights with K % 256 == 0 (other K keep the LDS-staged
// kernel of mfma_gemm.hip).
//
// The reference computes the product with one fp32 FMA chain per output
// (ref:src/kernels/matmul_quant.cu:64-130 Q8_0, :142-205 Q4_0, :215-290 Q5_0,
// :309-386 Q4_K, :398-498 Q6_K, :510-557 FP16).
// Here:
//   * a workgroup of eight waves (two per SIMD, so one wave's dependency
//     stalls are filled by the other's work) owns a 64(m) x 256(n) output
//     tile; wave w owns the 32 weight rows [32 w, 32 w + 32) and all 64 m, as
//     two v_mfma_f32_32x32x16_f16 tiles (32 fp32 accumulators per lane);
//   * activations are the MFMA A operand: each k step (64 columns) every
//     thread converts 8 fp32 values of two rows to fp16 and writes them to a
//     double-buffered LDS tile of 64 rows x 64 halves, which all eight waves
//     read (8 ds_read_b128 per wave and step);
//   * weights are the B operand: each wave copies its 32 rows' bytes of a
//     group of four steps into its own LDS area with coalesced loads (Q4_K,
//     Q4_0, Q5_0: global_load_lds into the other of two areas, a group ahead,
//     kDmaGroup; Q8_0, Q6_K: through registers; FP16, 512 bytes per row and
//     group, per step into a ring of three step buffers, kDirect), and each
//     lane decodes the bytes of its own weight row (its output column) from
//     there in registers, to the reference's dequantized value rounded once to
//     fp16 (Q8_0: d * q; Q4_0, Q5_0: d * (q - 8), d * (q - 16); Q4_K:
//     d * (sc * q) - dmin * mn, sc * q exact; Q6_K: twice, (q - 32) fp16(d sc)),
//     two weights per packed op;
//   * a lane's bytes of one step are contiguous runs (Q4_K: 16 quant bytes of
//     the super-block chunk; Q8_0, Q4_0, Q5_0: one whole block; Q6_K: 16 bytes of
//     each of two ql runs and of qh), so the 8 k of
//     each MFMA sub-step are not consecutive k; the activation fragment of
//     every sub-step is fetched from the LDS columns of the same k, so the
//     products and sums are the same as in k order;
//   * a lane's outputs are C[m][n] for its column n and 16 rows m, so the 32
//     lanes of a half-wave store 128 contiguous bytes of one row;
//   * the eight m blocks that share a weight block are consecutive workgroups
//     on one XCD (each XCD has its own L2), so the weights come from HBM once;
//     when the tiles cannot fill 256 CUs the k range is split over workgroups
//     that add into a zeroed C with fp32 atomics, or, given a workspace, store
//     their partial sums there for a fixed-order reduction;
//   * a stacked gate/up matrix can take a SiLU(gate) * up epilogue: a tile's
//     128 output columns are 128 gate rows and the matching 128 up rows.
// Activations outside fp16's comfortable range would lose the 1e-3 bound (a
// value >= 65504 becomes inf; a row whose largest magnitude is below 2^-10
// keeps only subnormal precision), so each thread tracks the largest
// magnitude of its rows; the rows flagged that way are recomputed in fp32 from
// the reference's per-element decode at the end of the tile (the fp16 MFMA
// results of those rows are not stored).  Dequantized weights must fit fp16
// (|x| < 65504), as every GGUF model's do.
#include <atomic>
#include <type_traits>

#include "common.hpp"
#include "decode.hpp"
#include "internal.hpp"
#include "split.hpp"
#include "act.hpp"

namespace cri {
namespace dev {
namespace {

typedef _Float16 ph8 __attribute__((ext_vector_type(8)));
typedef _Float16 ph2 __attribute__((ext_vector_type(2)));
typedef float pf16v __attribute__((ext_vector_type(16)));
typedef float pf2 __attribute__((ext_vector_type(2)));
typedef uint32_t pu2 __attribute__((ext_vector_type(2)));
typedef uint32_t pu4a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int kPTM = 64, kPTN = 256, kPKS = 64, kPThreads = 512;
constexpr int kPStage = kPTM * kPKS * 2;  // one fp16 activation tile, bytes
constexpr int kPDirectStep = 32 * kPKS * 2;  // one FP16 weight step buffer: a wave's 32 rows x 64 halves
constexpr uint32_t kPMagic = 0x64646464u;
constexpr float kPRowMax = 65504.0f;      // at or above: fp16 infinity
constexpr float kPRowMin = 0x1p-10f;      // below (and nonzero): subnormal precision only

__device__ __forceinline__ uint32_t p_perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}
// bytes b0, b1 (lo) or b2, b3 (hi) of w as the fp16 pair (1024 + b, 1024 + b')
__device__ __forceinline__ uint32_t p_mlo(uint32_t w) { return p_perm(kPMagic, w, 0x04010400u); }
__device__ __forceinline__ uint32_t p_mhi(uint32_t w) { return p_perm(kPMagic, w, 0x04030402u); }
// byte P of w as the fp16 pair (1024 + b, 1024 + b)
template <int P>
__device__ __forceinline__ uint32_t p_msplat(uint32_t w) {
    return p_perm(kPMagic, w, 0x04000400u | (P << 16) | P);
}
__device__ __forceinline__ constexpr uint32_t p_const(float lo, float hi) {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(lo))) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(hi))) << 16);
}
__device__ __forceinline__ uint32_t p_fma(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(ph2, a), __builtin_bit_cast(ph2, b),
                                                                  __builtin_bit_cast(ph2, c)));
}
__device__ __forceinline__ uint32_t p_add(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(ph2, a) + __builtin_bit_cast(ph2, b));
}
__device__ __forceinline__ uint32_t p_mul(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(ph2, a) * __builtin_bit_cast(ph2, b));
}

// 16 bytes at a dword-aligned address (Q8_0 rows are only dword-aligned)
__device__ __forceinline__ u32x4 p_load16(const uint8_t* p) {
    const pu4a4 v = *reinterpret_cast<const pu4a4*>(p);
    return u32x4{v.x, v.y, v.z, v.w};
}

// 16 bytes per lane from global memory straight into LDS (lane l: bytes 16 l from lds, which is
// wave-uniform).  A helper of its own: with the builtin written inside the kernel's lambdas, the
// host compilation pass emitted no launch stub for some instantiations.
__device__ __forceinline__ void p_dma16(const uint8_t* g, char* lds) { __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0); }

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt bits 3:0 and 15:14; expcnt and lgkmcnt left at their
// no-wait maxima).  The compiler does not order a global_load_lds into LDS before later ds_reads
// of the same bytes, so the FP16 path waits for its copies itself.
template <int N>
__device__ __forceinline__ void p_wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// LDS tile of 64 fp16 columns per row (activations; FP16 weight steps): row r
// (128 bytes) holds 8 chunks of 8 halves; chunk c is stored in slot c ^ (r & 7)
// ^ ((r >> 3) & 1) (conflict-free for 32-row operand fetches, one chunk per
// half-wave).
__device__ __forceinline__ int p_off(int r, int c) { return (r << 7) + ((c ^ (r & 7) ^ ((r >> 3) & 1)) << 4); }

// ---------------------------------------------------------------------------
// B-operand formats.  A wave's weight bytes of one group (four k steps) are
// kCopyPieces 16-byte pieces of each of its 32 rows (load_piece from the row's
// group start, piece_bytes what is stored); they are copied into a per-wave
// LDS area, kRowBytes per row, with coalesced loads (kCopyPieces lanes per
// row), so each cache line is requested once; kTail formats add one dword per
// row (load_tail, stored after the rows).  read<J>(): one lane's bytes of step
// J of the group from that area.  prep<J>(): the step's scale constants.
// sub<J, S>(): the 8 fp16 weights (4 dwords) of MFMA sub-step S of a step at
// position J.  chunk(S, h): which 8-column chunk of the 64-column step those 8
// weights are, so the activation fragment is fetched from the same k.  Splits
// start on a multiple of four steps, so J = step mod 4 is a compile-time
// position.

// ref:src/kernels/dequantize.cu:289-324.  Step j of a super-block is its
// 64-element chunk j: elements 64j + e (e < 32) are the low nibbles of
// qs[32j + e] in sub-block 2j, elements 64j + 32 + e the high nibbles in
// sub-block 2j + 1; x = d * sc * q - dmin * mn.  Lane half h takes qs[32j +
// 16h .. + 16): sub-steps 0, 1 are the low nibbles of its bytes 0..7, 8..15
// (k = 64j + 16h + 0..15), sub-steps 2, 3 their high nibbles (k + 32).  A
// group is one super-block (144 bytes per row).
struct PQ4K {
    static constexpr int kFmt = kFmtQ4_K;
    static constexpr int kBlockK = 256;
    static constexpr int kRowBytes = 144;
    static constexpr int kCopyPieces = kRowBytes / 16;
    static constexpr bool kTail = false;
    using Piece = u32x4;
    static constexpr int kAreaBytes = 32 * kRowBytes;
    static constexpr int kReadPhase = 0;  // the next step's bytes are read in phase 0
    static constexpr int kMfmaPrio = 0;   // wave priority while issuing a phase's MFMAs (none)
    static constexpr bool kActSwap = false;  // activation chunks in k order
    static constexpr bool kDirect = false;  // bytes copied through the wave's LDS area
    static constexpr bool kOneGroupPerTrip = false;
    static constexpr bool kDmaGroup = true;
    static __device__ __forceinline__ Piece load_piece(const uint8_t* p) { return p_load16(p); }
    static __device__ __forceinline__ u32x4 piece_bytes(const Piece& p) { return p; }
    static __device__ __forceinline__ long group_offset(int first_step) { return (first_step >> 2) * 144L; }
    struct Frag {
        u32x4 hdr;  // d, dmin (fp16), scales[12]
        u32x4 qs;   // qs[32j + 16h .. + 16)
    };
    template <int J>
    static __device__ __forceinline__ void read(Frag& f, const char* row, int h) {
        f.hdr = *reinterpret_cast<const u32x4*>(row);
        f.qs = *reinterpret_cast<const u32x4*>(row + 16 + 32 * J + 16 * h);
    }
    static __device__ __forceinline__ constexpr int chunk(int s, int h) { return 4 * (s >> 1) + 2 * h + (s & 1); }
    struct Consts {
        uint32_t a[2], c[2], m[2], d2;  // fp16 pairs; [0]: low nibbles, [1]: high nibbles
    };
    // 6-bit (sc, mn) of sub-blocks 2J and 2J + 1 (ref:src/kernels/dequantize.cu:298-305),
    // as bytes of a dword: J < 2 takes scales[0..3] / [4..7] & 63, J >= 2 the
    // split encoding (scales[8..11] nibbles + top bits of scales[0..3] / [4..7])
    template <int J>
    static __device__ __forceinline__ void prep(const Frag& f, Consts& k) {
        uint32_t scd, mnd;
        if constexpr (J < 2) {
            scd = f.hdr.y & 0x3F3F3F3Fu;
            mnd = f.hdr.z & 0x3F3F3F3Fu;
        } else {
            scd = (f.hdr.w & 0x0F0F0F0Fu) | ((f.hdr.y >> 2) & 0x30303030u);
            mnd = ((f.hdr.w >> 4) & 0x0F0F0F0Fu) | ((f.hdr.z >> 2) & 0x30303030u);
        }
        constexpr int b0 = 2 * (J & 1);
        const uint32_t m1024 = p_const(-1024.0f, -1024.0f);
        const uint32_t sc0 = p_add(p_msplat<b0>(scd), m1024), sc1 = p_add(p_msplat<b0 + 1>(scd), m1024);
        const uint32_t mn0 = p_add(p_msplat<b0>(mnd), m1024), mn1 = p_add(p_msplat<b0 + 1>(mnd), m1024);
        const uint32_t nd = p_perm(f.hdr.x, f.hdr.x, 0x03020302u) ^ 0x80008000u;  // (-dmin, -dmin)
        k.d2 = p_perm(f.hdr.x, f.hdr.x, 0x01000100u);
        // low nibbles: (1024 + q) sc - 1024 sc = sc q exactly (<= 945);
        // high nibbles masked in place are 16 q: (1024 + 16 q) sc/16 - 64 sc
        k.a[0] = sc0;
        k.c[0] = p_mul(sc0, p_const(-1024.0f, -1024.0f));
        k.a[1] = p_mul(sc1, p_const(0.0625f, 0.0625f));
        k.c[1] = p_mul(sc1, p_const(-64.0f, -64.0f));
        k.m[0] = p_mul(mn0, nd);
        k.m[1] = p_mul(mn1, nd);
    }
    // B fragment of sub-step S: d (sc q) - dmin mn, one rounding to fp16
    template <int J, int S>
    static __device__ __forceinline__ void sub(const Frag& f, const Consts& k, uint32_t (&b)[4]) {
        constexpr int hi = S >= 2 ? 1 : 0;
        constexpr uint32_t mask = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
        const uint32_t src[2] = {(S & 1) ? f.qs.z : f.qs.x, (S & 1) ? f.qs.w : f.qs.y};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t u = src[i] & mask;
            b[2 * i] = p_fma(p_fma(p_mlo(u), k.a[hi], k.c[hi]), k.d2, k.m[hi]);
            b[2 * i + 1] = p_fma(p_fma(p_mhi(u), k.a[hi], k.c[hi]), k.d2, k.m[hi]);
        }
    }
};

// ref:src/kernels/dequantize.cu:45-47, x = d * q.  Step j covers the 34-byte
// blocks 2j and 2j + 1; lane half h decodes block 2j + h whole (sub-step S:
// its elements 8S .. 8S + 7, k = 64j + 32h + 8S ..).  K % 64 == 0 makes a
// row an even number of blocks, so a group (four steps, 272 bytes per row)
// starts dword-aligned; block 2j + h starts at byte 68j + 34h of it, its
// quants at 68j + 34h + 2.  A lane reads the 9 dwords from byte 68j + 32h
// and funnel-shifts its quants by 2 (h = 0) or 4 (h = 1) bytes.
struct PQ8_0 {
    static constexpr int kFmt = kFmtQ8_0;
    static constexpr int kBlockK = 32;
    static constexpr int kRowBytes = 272;
    static constexpr int kCopyPieces = kRowBytes / 16;
    static constexpr bool kTail = false;
    using Piece = u32x4;
    static constexpr int kAreaBytes = 32 * kRowBytes;
    static constexpr int kReadPhase = 0;  // the next step's bytes are read in phase 0
    static constexpr int kMfmaPrio = 0;   // wave priority while issuing a phase's MFMAs (none)
    static constexpr bool kActSwap = false;
    static constexpr bool kDirect = false;  // bytes copied through the wave's LDS area
    static constexpr bool kOneGroupPerTrip = false;
    static constexpr bool kDmaGroup = false;
    static __device__ __forceinline__ Piece load_piece(const uint8_t* p) { return p_load16(p); }
    static __device__ __forceinline__ u32x4 piece_bytes(const Piece& p) { return p; }
    static __device__ __forceinline__ long group_offset(int first_step) { return first_step * 68L; }
    struct Frag {
        uint32_t dw[9];
    };
    template <int J>
    static __device__ __forceinline__ void read(Frag& f, const char* row, int h) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(row + 68 * J + 32 * h);
#pragma unroll
        for (int i = 0; i < 9; ++i) f.dw[i] = p[i];
    }
    static __device__ __forceinline__ constexpr int chunk(int s, int h) { return 4 * h + s; }
    struct Consts {
        uint32_t d2, sel;
    };
    template <int J>
    static __device__ __forceinline__ void prep(const Frag& f, Consts& k) {
        const bool h1 = (__lane_id() >> 5) != 0;
        k.d2 = p_perm(f.dw[0], f.dw[0], h1 ? 0x03020302u : 0x01000100u);
        k.sel = h1 ? 0x07060504u : 0x05040302u;  // dword pair -> quants shifted by 4 or 2 bytes
    }
    // B fragment of sub-step S: d * q, one rounding to fp16
    template <int J, int S>
    static __device__ __forceinline__ void sub(const Frag& f, const Consts& k, uint32_t (&b)[4]) {
        const uint32_t bias = p_const(-1152.0f, -1152.0f);  // 1024 + 128
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t q = p_perm(f.dw[2 * S + i + 1], f.dw[2 * S + i], k.sel);
            const uint32_t x = q ^ 0x80808080u;  // int8 -> q + 128
            b[2 * i] = p_mul(p_add(p_mlo(x), bias), k.d2);
            b[2 * i + 1] = p_mul(p_add(p_mhi(x), bias), k.d2);
        }
    }
};

// Shared by the two 32-element formats with 4-bit quants below: lane half h decodes block 2j + h of
// step j, whose fp16 d sits in the low (h = 0) or high (h = 1) half of the first dword the lane reads;
// sel realigns the bytes after d (two bytes past a dword for h = 0, four for h = 1).
struct P32Consts {
    uint32_t d2, sel, qh;
};
__device__ __forceinline__ void p32_prep(uint32_t dw0, P32Consts& k) {
    const bool h1 = (__lane_id() >> 5) != 0;
    k.d2 = p_perm(dw0, dw0, h1 ? 0x03020302u : 0x01000100u);
    k.sel = h1 ? 0x07060504u : 0x05040302u;
}

// ref:src/kernels/dequantize.cu:73-101, x = d * (q - 8), element i the low
// (even i) or high (odd i) nibble of quant byte i / 2.  Step j covers the
// 18-byte blocks 2j and 2j + 1 (a group of four steps is 144 bytes per row
// and starts dword-aligned, K % 256 == 0); lane half h decodes block 2j + h
// whole from the five dwords at byte 36j + 16h of the group.  Sub-step S is
// quant bytes 4S .. 4S + 3, elements 8S .. 8S + 7, in the order (0, 2, 1, 3,
// 4, 6, 5, 7): the low nibbles of two bytes form one fp16 pair, their high
// nibbles (masked in place, 16 q) the next; the activations are staged in the
// same order (kActSwap), so the products and sums are those of k order.
struct PQ4_0 {
    static constexpr int kFmt = kFmtQ4_0;
    static constexpr int kBlockK = 32;
    static constexpr int kRowBytes = 144;
    static constexpr int kCopyPieces = kRowBytes / 16;
    static constexpr bool kTail = false;
    using Piece = u32x4;
    static constexpr int kAreaBytes = 32 * kRowBytes;
    static constexpr int kReadPhase = 0;
    static constexpr int kMfmaPrio = 0;
    static constexpr bool kActSwap = true;  // chunk halves (x0, x2, x1, x3, x4, x6, x5, x7)
    static constexpr bool kDirect = false;  // bytes copied through the wave's LDS area
    static constexpr bool kOneGroupPerTrip = false;
    static constexpr bool kDmaGroup = true;
    static __device__ __forceinline__ Piece load_piece(const uint8_t* p) { return p_load16(p); }
    static __device__ __forceinline__ u32x4 piece_bytes(const Piece& p) { return p; }
    static __device__ __forceinline__ long group_offset(int first_step) { return first_step * 36L; }
    struct Frag {
        uint32_t dw[5];
    };
    template <int J>
    static __device__ __forceinline__ void read(Frag& f, const char* row, int h) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(row + 36 * J + 16 * h);
#pragma unroll
        for (int i = 0; i < 5; ++i) f.dw[i] = p[i];
    }
    static __device__ __forceinline__ constexpr int chunk(int s, int h) { return 4 * h + s; }
    using Consts = P32Consts;
    template <int J>
    static __device__ __forceinline__ void prep(const Frag& f, Consts& k) {
        p32_prep(f.dw[0], k);
    }
    // B fragment of sub-step S: d (q - 8), one rounding to fp16; (1024 + q) - 1032 and
    // (1024 + 16 q) / 16 - 72 are exact
    template <int J, int S>
    static __device__ __forceinline__ void sub(const Frag& f, const Consts& k, uint32_t (&b)[4]) {
        const uint32_t w = p_perm(f.dw[S + 1], f.dw[S], k.sel);
        const uint32_t lo = w & 0x0F0F0F0Fu, hi = w & 0xF0F0F0F0u;
        const uint32_t bl = p_const(-1032.0f, -1032.0f);
        const uint32_t c16 = p_const(0.0625f, 0.0625f), bh = p_const(-72.0f, -72.0f);
        b[0] = p_mul(p_add(p_mlo(lo), bl), k.d2);        // elements 8S, 8S + 2
        b[1] = p_mul(p_fma(p_mlo(hi), c16, bh), k.d2);   // 8S + 1, 8S + 3
        b[2] = p_mul(p_add(p_mhi(lo), bl), k.d2);        // 8S + 4, 8S + 6
        b[3] = p_mul(p_fma(p_mhi(hi), c16, bh), k.d2);   // 8S + 5, 8S + 7
    }
};

// ref:src/kernels/dequantize.cu:126-165, x = d * (q - 16) with q = the low
// (element i < 16) or high (i >= 16) nibble of qs[i % 16] and bit i of qh as
// bit 4.  Step j covers the 22-byte blocks 2j and 2j + 1 (176 bytes per row
// and group); lane half h decodes block 2j + h from the six dwords at byte
// 44j + 20h.  Sub-step S is elements 8S .. 8S + 7 in k order: the low (S < 2)
// or high nibbles of qs dwords 2 (S & 1), + 1.  Each element becomes the fp16
// 1024 + 16 q: its nibble times 16 in the low byte and its qh bit as bit 0 of
// the 0x64 high byte (256 = 16 * 16).
struct PQ5_0 {
    static constexpr int kFmt = kFmtQ5_0;
    static constexpr int kBlockK = 32;
    static constexpr int kRowBytes = 176;
    static constexpr int kCopyPieces = kRowBytes / 16;
    static constexpr bool kTail = false;
    using Piece = u32x4;
    static constexpr int kAreaBytes = 32 * kRowBytes;
    static constexpr int kReadPhase = 0;
    static constexpr int kMfmaPrio = 0;
    static constexpr bool kActSwap = false;
    static constexpr bool kDirect = false;  // bytes copied through the wave's LDS area
    static constexpr bool kOneGroupPerTrip = false;
    static constexpr bool kDmaGroup = true;
    static __device__ __forceinline__ Piece load_piece(const uint8_t* p) { return p_load16(p); }
    static __device__ __forceinline__ u32x4 piece_bytes(const Piece& p) { return p; }
    static __device__ __forceinline__ long group_offset(int first_step) { return first_step * 44L; }
    struct Frag {
        uint32_t dw[6];
    };
    template <int J>
    static __device__ __forceinline__ void read(Frag& f, const char* row, int h) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(row + 44 * J + 20 * h);
#pragma unroll
        for (int i = 0; i < 6; ++i) f.dw[i] = p[i];
    }
    static __device__ __forceinline__ constexpr int chunk(int s, int h) { return 4 * h + s; }
    using Consts = P32Consts;
    template <int J>
    static __device__ __forceinline__ void prep(const Frag& f, Consts& k) {
        p32_prep(f.dw[0], k);
        k.qh = p_perm(f.dw[1], f.dw[0], k.sel);
    }
    // B fragment of sub-step S: d (q - 16), one rounding to fp16; (1024 + 16 q) / 16 - 80 is exact
    template <int J, int S>
    static __device__ __forceinline__ void sub(const Frag& f, const Consts& k, uint32_t (&b)[4]) {
        const uint32_t c16 = p_const(0.0625f, 0.0625f), bias = p_const(-80.0f, -80.0f);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int t = 2 * (S & 1) + i;  // qs dword: elements 8S + 4i .. + 3 in its bytes
            const uint32_t w = p_perm(f.dw[t + 2], f.dw[t + 1], k.sel);
            const uint32_t u = (S >= 2 ? w : (w << 4)) & 0xF0F0F0F0u;
            // their four qh bits to bit 0 of the bytes of 0x64646464 (the products do not overlap)
            const uint32_t n = (k.qh >> (8 * S + 4 * i)) & 0xFu;
            const uint32_t mw = (__umul24(n, 0x204081u) & 0x01010101u) | 0x64646464u;
            b[2 * i] = p_mul(p_fma(p_perm(mw, u, 0x05010400u), c16, bias), k.d2);
            b[2 * i + 1] = p_mul(p_fma(p_perm(mw, u, 0x07030602u), c16, bias), k.d2);
        }
    }
};

// ref:src/kernels/matmul_quant.cu:510-557, FP16 weights: nothing to decode, but
// 512 bytes per row and group (16 KB of LDS per wave, more than the area
// allows), so the copy is per step instead (kDirect): each wave's 32 rows x 128
// bytes of a step go to LDS in four global_load_lds_dwordx4 (one row per 8
// lanes, so each cache line is requested once, and no registers), into a ring of
// three step buffers in the activation tile's swizzled layout; the copy of step
// t + 3 is issued while step t is multiplied, and lanes read their B fragments
// (lane half h: columns 32h .. 32h + 31, sub-step S: 32h + 8S .. + 8, k order)
// one step ahead, as the other formats do.  Loading each lane's 64 bytes of its
// own row straight into registers instead touches 32 cache lines per load
// instruction: 44.6 us at 512 x 8192 x 2048, against 32.3 us for the same loads
// made coalesced.
struct PF16 {
    static constexpr int kFmt = kFmtF16;
    static constexpr int kRowBytes = 0;
    static constexpr int kCopyPieces = 0;
    static constexpr bool kTail = false;
    static constexpr bool kDirect = true;
    static constexpr bool kOneGroupPerTrip = true;
    static constexpr bool kDmaGroup = false;
    using Piece = u32x4;
    static constexpr int kAreaBytes = 3 * kPDirectStep;  // the ring of three step buffers
    static constexpr int kReadPhase = 0;
    static constexpr int kMfmaPrio = 0;
    static constexpr bool kActSwap = false;
    struct Frag {
        u32x4 q[4];
    };
    // buf: the step's buffer; fr: the lane's row
    static __device__ __forceinline__ void read_buf(Frag& f, const char* buf, int fr, int h) {
#pragma unroll
        for (int s = 0; s < 4; ++s) f.q[s] = *reinterpret_cast<const u32x4*>(buf + p_off(fr, 4 * h + s));
    }
    static __device__ __forceinline__ constexpr int chunk(int s, int h) { return 4 * h + s; }
    struct Consts {};
    template <int J>
    static __device__ __forceinline__ void prep(const Frag&, Consts&) {}
    template <int J, int S>
    static __device__ __forceinline__ void sub(const Frag& f, const Consts&, uint32_t (&b)[4]) {
        b[0] = f.q[S].x;
        b[1] = f.q[S].y;
        b[2] = f.q[S].z;
        b[3] = f.q[S].w;
    }
};

// ref:src/kernels/dequantize.cu:179-244, x = d * sc * (q - 32) with q the 6-bit
// value of a low/high nibble of ql and two bits of qh.  Step j of a super-block
// is its 64 elements 64j ..: half c = j / 2 (128 elements), quarters 2 (j & 1) +
// qq, qq = 0, 1; element l (< 32) of a quarter takes ql[64c + 32qq + l] (low
// nibble for j even, high for j odd), bits 2 (2 (j & 1) + qq) of qh[32c + l] and
// scale sc[8c + 4 (j & 1) + 2qq + l / 16].  Lane half h takes l in [16h, 16h +
// 16): sub-step S is quarter qq = S & 1, l = 16h + 8 (S >> 1) + 0..7 (each sub-step
// has one scale; a lane's low qh and ql dwords are done after sub-step 1).  A group is one super-block
// (210 bytes per row: ql[128], qh[64], scales[16], d at 208), which starts 2
// bytes after a dword boundary for odd super-blocks (and for alternate rows when
// K / 256 is odd).  The copy reads 13 dword-aligned 16-byte pieces from the
// dword boundary at or below the super-block plus the dword after each piece,
// and stores the pieces shifted into place (v_alignbyte), so LDS holds super-block
// bytes 0 .. 207 (sc[12..15] at 204 .. 207) at offsets 0 .. 207 for either shift; d
// (bytes 208, 209) lies past the copied area, so a tail dword {sc[14], sc[15], d}
// read with two 16-bit loads sits after the wave's 32 rows.  Every byte read lies inside
// the super-block or the 2 bytes before it, which are the previous super-block's
// (a super-block at the buffer's dword-aligned start has no shift).  Weights are
// rounded twice: fp16(d * sc), then (q - 32) times it.
struct PQ6K {
    static constexpr int kFmt = kFmtQ6_K;
    static constexpr int kBlockK = 256;
    static constexpr int kRowBytes = 208;  // 13 pieces
    static constexpr int kCopyPieces = 13;
    static constexpr bool kTail = true;
    static constexpr int kAreaBytes = 32 * kRowBytes + 32 * 4;  // the rows, then one tail dword per row
    // the next step's bytes are read in phase 2, after half of this step's are decoded (registers)
    static constexpr int kReadPhase = 2;
    // the wave issuing a phase's MFMAs takes issue priority over the SIMD's other wave (s_setprio 3):
    // measured 46.5 -> 44.8-45.2 us at 512 x 8192 x 2048, the down shape unchanged (Q4_K and Q8_0
    // ran 1-3% slower with it)
    static constexpr int kMfmaPrio = 3;
    static constexpr bool kActSwap = false;
    static constexpr bool kDirect = false;  // bytes copied through the wave's LDS area
    // one group per loop trip: 45.9 -> 44.5 us at 512 x 8192 x 2048, same box (no gain for Q4_K, Q8_0, Q4_0)
    static constexpr bool kOneGroupPerTrip = true;
    static constexpr bool kDmaGroup = false;
    static __device__ __forceinline__ long group_offset(int first_step) { return (first_step >> 2) * 210L; }
    struct Piece {
        u32x4 v;     // the 16 bytes from the dword boundary
        uint32_t e;  // bytes 0, 1: the two bytes after them; bits 16..17: the shift (0 or 2)
    };
    // ptr: the super-block start of the row plus 16 * piece
    static __device__ __forceinline__ Piece load_piece(const uint8_t* ptr) {
        const uint32_t sh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ptr) & 3);
        const uint8_t* a = ptr - sh;
        Piece p;
        p.v = p_load16(a);
        // shift 2: the dword after the piece (for the last piece, bytes 206 .. 209 of the
        // super-block); shift 0 needs none and reads the piece's own last dword, so no read
        // passes the super-block's end
        p.e = (*reinterpret_cast<const uint32_t*>(a + 12 + 2 * sh) & 0xFFFFu) | (sh << 16);
        return p;
    }
    static __device__ __forceinline__ u32x4 piece_bytes(const Piece& p) {
        const uint32_t sh = p.e >> 16;
        return u32x4{__builtin_amdgcn_alignbyte(p.v.y, p.v.x, sh), __builtin_amdgcn_alignbyte(p.v.z, p.v.y, sh),
                     __builtin_amdgcn_alignbyte(p.v.w, p.v.z, sh), __builtin_amdgcn_alignbyte(p.e, p.v.w, sh)};
    }
    // {sc[14], sc[15], d}: two 16-bit loads at even addresses inside the super-block
    static __device__ __forceinline__ uint32_t load_tail(const uint8_t* grow) {
        return static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(grow + 206)) |
               (static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(grow + 208)) << 16);
    }
    struct Frag {
        u32x4 l0, l1;  // ql[64c + 16h .. + 16), ql[64c + 32 + 16h .. + 16)
        u32x4 qh;      // qh[32c + 16h .. + 16)
        uint32_t scw;  // sc[8c + 4 (j & 1) .. + 4)
        uint32_t tail; // sc[14], sc[15], d
    };
    template <int J>
    static __device__ __forceinline__ void read(Frag& f, const char* row, int h) {
        constexpr int c = J >> 1, odd = J & 1;
        f.l0 = *reinterpret_cast<const u32x4*>(row + 64 * c + 16 * h);
        f.l1 = *reinterpret_cast<const u32x4*>(row + 64 * c + 32 + 16 * h);
        f.qh = *reinterpret_cast<const u32x4*>(row + 128 + 32 * c + 16 * h);
        f.scw = *reinterpret_cast<const uint32_t*>(row + 192 + 8 * c + 4 * odd);
        const int fr = __lane_id() & 31;  // row is the area's row fr; the tails follow the 32 rows
        f.tail = *reinterpret_cast<const uint32_t*>(row + (32 - fr) * kRowBytes + 4 * fr);
    }
    static __device__ __forceinline__ constexpr int chunk(int s, int h) { return 4 * (s & 1) + 2 * h + (s >> 1); }
    struct Consts {
        uint32_t dsc[2];  // fp16(d * sc) pairs of quarters qq = 0, 1
    };
    // sc byte b of w (int8) as the fp16 pair (sc, sc): (1024 + (sc + 128)) - 1152, exact
    static __device__ __forceinline__ uint32_t sc_pair(uint32_t w, uint32_t b) {
        return p_add(p_perm(kPMagic, w ^ 0x80808080u, 0x04000400u | (b << 16) | b), p_const(-1152.0f, -1152.0f));
    }
    template <int J>
    static __device__ __forceinline__ void prep(const Frag& f, Consts& k) {
        const uint32_t h = __lane_id() >> 5;
        const uint32_t d2 = p_perm(f.tail, f.tail, 0x03020302u);  // (d, d)
        k.dsc[0] = p_mul(sc_pair(f.scw, h), d2);
        k.dsc[1] = p_mul(J == 3 ? sc_pair(f.tail, h) : sc_pair(f.scw, h + 2), d2);
    }
    // B fragment of sub-step S: (q - 32) fp16(d sc)
    template <int J, int S>
    static __device__ __forceinline__ void sub(const Frag& f, const Consts& k, uint32_t (&b)[4]) {
        constexpr int odd = J & 1, qq = S & 1, half = S >> 1;
        constexpr int hs = 4 - (4 * odd + 2 * qq);  // qh bits 4 odd + 2 qq -> bits 4..5 of each byte
        const u32x4& l = qq ? f.l1 : f.l0;
        const uint32_t lw[2] = {half ? l.z : l.x, half ? l.w : l.y};
        const uint32_t hw[2] = {half ? f.qh.z : f.qh.x, half ? f.qh.w : f.qh.y};
        const uint32_t bias = p_const(-1056.0f, -1056.0f);  // 1024 + 32
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t lo = odd ? (lw[i] >> 4) : lw[i];
            const uint32_t hb = (hs >= 0 ? (hw[i] << (hs >= 0 ? hs : 0)) : (hw[i] >> (hs < 0 ? -hs : 0))) & 0x30303030u;
            const uint32_t u = (lo & 0x0F0F0F0Fu) | hb;
            b[2 * i] = p_mul(p_add(p_mlo(u), bias), k.dsc[qq]);
            b[2 * i + 1] = p_mul(p_add(p_mhi(u), bias), k.dsc[qq]);
        }
    }
};


template <int J>
using pos_t = std::integral_constant<int, J>;

// dynamic LDS: two activation buffers of four step tiles, then one weight area per wave
template <class W>
constexpr int prefill_lds_bytes() {
    return 8 * kPStage + (kPThreads / 64) * W::kAreaBytes * (W::kDmaGroup ? 2 : 1);
}

template <class W>
__global__ __launch_bounds__(kPThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_gemm_kernel(
    const float* __restrict__ A, const uint8_t* __restrict__ B, float* __restrict__ C, int M, int N, int K,
    long row_bytes, int MT, int NT, int steps_per_split, int remap, int atomic, float* __restrict__ part, int swiglu) {
    static_assert(prefill_lds_bytes<W>() >= 256 + kPTM * kPTN * 4, "the swiglu epilogue's C tile fits in LDS");
    extern __shared__ __attribute__((aligned(16))) char lds[];
    int* const rowflag = reinterpret_cast<int*>(lds);  // after the k loop
    int bid = blockIdx.x;
    if (remap) {  // XCD x (= bid % 8) runs a contiguous run of logical tiles
        const int per_xcd = gridDim.x >> 3;
        bid = (bid & 7) * per_xcd + (bid >> 3);
    }
    const int mt = bid % MT;  // the m blocks of one weight block are consecutive
    const int rest = bid / MT;
    const int nt = rest % NT;
    const int ksplit = rest / NT;
    const int s_begin = ksplit * steps_per_split;
    const int s_end = min(K / kPKS, s_begin + steps_per_split);
    if (s_begin >= s_end) return;
    const int nst = s_end - s_begin;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, fr = lane & 31;
    // swiglu: B holds N = 2F rows, gate [0, F) then up [F, 2F), and C = SiLU(A gate^T) * (A up^T)
    // is [M, F]; the tile's kPTN / 2 output columns are gate rows (waves 0-3) and the same up rows
    // (waves 4-7), met in LDS after the k loop
    const int F = N >> 1;
    const int m0 = mt * kPTM;
    const int n0 = swiglu ? (wave >> 2) * F + nt * (kPTN / 2) + 32 * (wave & 3) : nt * kPTN + 32 * wave;

    // activation staging: 16 lanes cover one row's 64 columns (256 contiguous bytes per load
    // instruction and row); thread -> columns 4 ap .. 4 ap + 3 of rows ar0 and ar0 + 32
    const int ap = tid & 15, ar0 = tid >> 4;
    const float* abase = A + 4 * ap;
    int arow_off[2], aw[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        arow_off[i] = min(m0 + ar0 + 32 * i, M - 1) * K;  // M * K < 2^31
        aw[i] = p_off(ar0 + 32 * i, ap >> 1) + 8 * (ap & 1);
    }
    float amax[2] = {0.0f, 0.0f};

    // weight copy: the wave's rows n0c + r (clamped to N - 1), chunk c = 64 i + lane of the
    // group's 32 * kCopyPieces pieces -> row c / kCopyPieces, piece c % kCopyPieces, stored at
    // byte 16 c of the wave's area (rows kRowBytes = 16 kCopyPieces apart), tails after the rows
    constexpr int kPieces = W::kCopyPieces, kChunks = 32 * kPieces, kLoads = (kChunks + 63) / 64;
    constexpr int kLoadsA = kLoads > 0 ? kLoads : 1;  // array extent (kDirect formats copy nothing)
    const int n0c = min(n0, N - 1);
    const uint8_t* const wbase = B + static_cast<long>(n0c) * row_bytes;
    int woff[kLoadsA];  // < 32 rows: 32 * row_bytes < 2^31 is a launch condition
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        constexpr int kP = kPieces > 0 ? kPieces : 1;
        const int c = min(64 * i + lane, kChunks - 1);
        const int r = c / kP;
        woff[i] = (min(n0 + r, N - 1) - n0c) * static_cast<int>(row_bytes) + 16 * (c % kP);
    }
    // kTail formats: lane l (and l + 32, a duplicate) reads row l's tail dword
    const int wtoff = (min(n0 + (lane & 31), N - 1) - n0c) * static_cast<int>(row_bytes);
    char* const warea = lds + 8 * kPStage + wave * W::kAreaBytes * (W::kDmaGroup ? 2 : 1);
    const char* const wrow = warea + fr * W::kRowBytes;  // this lane's row in the area
    // kDmaGroup formats: group q's bytes in area buffer q & 1
    auto wrow_b = [&](int b) { return wrow + b * W::kAreaBytes; };
    // kDirect formats: copy instruction i of a step takes row r = 8 i + lane / 8 of the wave's
    // rows; its lane writes LDS bytes 16 lane of the instruction's kilobyte, which p_off puts at
    // chunk c = (lane & 7) ^ (r & 7) ^ ((r >> 3) & 1) of row r
    int doff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 8 * i + (lane >> 3);
        const int c = (lane & 7) ^ (r & 7) ^ ((r >> 3) & 1);
        doff[i] = (min(n0 + r, N - 1) - n0c) * static_cast<int>(row_bytes) + 16 * c;
    }

    // A-operand fetch offsets: m tile u, sub-step s -> row 32 u + fr, the chunk of the
    // k that this half-wave's B fragment holds
    int aoff[2][4];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int s = 0; s < 4; ++s) aoff[u][s] = p_off(32 * u + fr, W::chunk(s, h));

    pf16v acc[2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[u][i] = 0.0f;

    // The k loop runs in groups of four steps.  At the start of group q the
    // bytes of group q + 1 are requested in one batch -- the wave's weight
    // bytes and this thread's activation values of the four steps -- and
    // consumed within the same group: the weight bytes are written to the
    // wave's LDS area after group q's last read of it (third iteration), its
    // first step decoded in the fourth, which also stages the activations
    // into the other LDS buffer.  So every load is waited for in the code
    // block that issued it, two to three iterations later.  kDmaGroup formats
    // copy the weight bytes straight into the other of two areas instead (no
    // registers, no LDS write), waited for where the third iteration first
    // reads them; kDirect (FP16) copies one step at a time into a ring of
    // three step buffers, each copy issued two iterations before the
    // iteration that reads it (see iter).  A split is whole
    // groups (K % 256 == 0 and splits start on a group), so nst is a
    // multiple of four; the loads issued after the last group repeat the
    // split's last step (in bounds) and what they stage is never read (their
    // values are that step's again, so the range guard's maxima stay the same).
    const int ngrp = nst >> 2;
    auto step_of = [&](int t) { return s_begin + min(t, nst - 1); };
    // relative step t of the split -> its buffer in the ring (kDirect)
    auto step_buf = [&](int t) { return warea + (t % 3) * kPDirectStep; };
    auto dma = [&](int t) {  // four copy instructions of 8 rows x 128 bytes
        char* const buf = step_buf(t);
        const uint8_t* const g = wbase + static_cast<long>(step_of(t)) * (2 * kPKS);
#pragma unroll
        for (int i = 0; i < 4; ++i) p_dma16(g + doff[i], buf + (kPDirectStep / 4) * i);
    };
    f32x4 av[4][2];  // activations of the next group: [step][row]
    typename W::Piece wr[kLoadsA];  // weight bytes of the next group
    uint32_t wt = 0;               // kTail formats: this lane's row's tail dword of the next group
    // kDmaGroup: group q's weight bytes straight into LDS buffer q & 1 (piece c = 64 i + lane at
    // byte 16 c, the layout write_w stores)
    auto dma_group = [&](int q) {
        if constexpr (W::kDmaGroup) {
            const uint8_t* g = wbase + W::group_offset(step_of(4 * q));
            char* const buf = warea + (q & 1) * W::kAreaBytes;
#pragma unroll
            for (int i = 0; i < kLoads; ++i)
                if (64 * i + lane < kChunks) p_dma16(g + woff[i], buf + 1024 * i);
        }
    };
    auto load_next = [&](int q) {
        if constexpr (!W::kDirect && !W::kDmaGroup) {
            const uint8_t* g = wbase + W::group_offset(step_of(4 * q));
#pragma unroll
            for (int i = 0; i < kLoads; ++i) wr[i] = W::load_piece(g + woff[i]);
            if constexpr (W::kTail) wt = W::load_tail(g + wtoff);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 2; ++i) av[j][i] = ld_f32x4(abase + step_of(4 * q + j) * kPKS + arow_off[i]);
    };
    auto write_w = [&]() {
        if constexpr (!W::kDirect && !W::kDmaGroup) {
#pragma unroll
            for (int i = 0; i < kLoads; ++i)
                if (64 * i + lane < kChunks)
                    *reinterpret_cast<u32x4*>(warea + 16 * (64 * i + lane)) = W::piece_bytes(wr[i]);
            if constexpr (W::kTail)
                if (lane < 32) *reinterpret_cast<uint32_t*>(warea + 32 * W::kRowBytes + 4 * lane) = wt;
        }
    };
    // step j, row i of the next group into buffer buf (tile j)
    auto stage = [&](char* buf, int j, int i) {
        const f32x4 v = av[j][i];
        // two v_max3_f32 (abs source modifiers) per four values
        amax[i] = fmaxf(fmaxf(fmaxf(fmaxf(amax[i], fabsf(v.x)), fabsf(v.y)), fabsf(v.z)), fabsf(v.w));
        // kActSwap: halves (x0, x2, x1, x3) of the thread's four columns, the B order of PQ4_0
        const pf2 p0 = W::kActSwap ? pf2{v.x, v.z} : pf2{v.x, v.y};
        const pf2 p1 = W::kActSwap ? pf2{v.y, v.w} : pf2{v.z, v.w};
        const uint32_t lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(p0, ph2));
        const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(p1, ph2));
        *reinterpret_cast<pu2*>(buf + j * kPStage + aw[i]) = pu2{lo, hi};
    };
    auto afrag = [&](const char* tile, int u, int s) { return *reinterpret_cast<const ph8*>(tile + aoff[u][s]); };
    auto mma2 = [&](const ph8 (&a)[2], const uint32_t (&bf)[4][4], int s) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
            acc[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                a[u], __builtin_bit_cast(ph8, u32x4{bf[s][0], bf[s][1], bf[s][2], bf[s][3]}), acc[u], 0, 0, 0);
    };

    // One iteration: step 4q + j's B fragments are in bc and its activation
    // fragments in ac; fc holds the bytes of the next step (position J of its
    // group).  Four phases, one per 16-column sub-step, each: that sub-step's
    // two MFMAs, then -- while the matrix cores run them -- the B fragments of
    // the same sub-step of the next step (bn) and the same sub-step's
    // activation fragments of the next tile (an, when there is one in this
    // buffer); in the group's last iteration each phase instead stages two of
    // the next group's eight activation pieces into nxt.  Phase 0 also reads
    // the bytes of the step after next (fn, position J + 1), after writing the
    // next group's weight bytes when J == 3.  The phases are fenced so the
    // compiler keeps this order.
    auto iter = [&](auto pos, int q, const ph8 (&ac)[2][4], ph8 (&an)[2][4], const char* next_tile,
                    const uint32_t (&bc)[4][4], uint32_t (&bn)[4][4], const typename W::Frag& fc,
                    typename W::Frag& fn, char* nxt) {
        constexpr int J = decltype(pos)::value;
        constexpr bool kLast = J == 0;  // the group's last iteration decodes the next group's first step
        const int tr = 4 * q + (J == 0 ? 5 : J + 1);  // the step whose bytes this iteration reads
        typename W::Consts k;
        W::template prep<J>(fc, k);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const ph8 a[2] = {ac[0][s], ac[1][s]};
            if constexpr (W::kMfmaPrio > 0) __builtin_amdgcn_s_setprio(W::kMfmaPrio);
            mma2(a, bc, s);
            if constexpr (W::kMfmaPrio > 0) __builtin_amdgcn_s_setprio(0);
            if (s == 0) {
                W::template sub<J, 0>(fc, k, bn[0]);
                if constexpr (J == 3) write_w();
            }
            if (s == 1) W::template sub<J, 1>(fc, k, bn[1]);
            if (s == 2) W::template sub<J, 2>(fc, k, bn[2]);
            if (s == 3) W::template sub<J, 3>(fc, k, bn[3]);
            if (s == W::kReadPhase) {
                if constexpr (W::kDirect) {
                    // step t = 4q + J + 1 (4q + 5 in the group's last iteration), copied one
                    // iteration earlier: the group's first iteration has this group's eight
                    // activation loads behind that copy, the others nothing older to spare.
                    // Then the copy of step t + 1, into the buffer of the step this iteration
                    // multiplies (its fragments were read two iterations ago); the last
                    // iteration's copy is issued at the next group's start instead, since the
                    // barrier waits for every copy in flight
                    if constexpr (J == 1)
                        p_wait_vm<8>();
                    else
                        p_wait_vm<0>();
                    W::read_buf(fn, step_buf(tr), fr, h);
                    if constexpr (!kLast) dma(tr + 1);
                } else if constexpr (W::kDmaGroup) {
                    // positions 2, 3 of this group, then 0, 1 of the next (its copy, issued at this
                    // group's start, has this group's eight activation loads behind it)
                    if constexpr (J == 3) p_wait_vm<8>();
                    W::template read<(J + 1) & 3>(fn, wrow_b(J == 3 || J == 0 ? (q + 1) & 1 : q & 1), h);
                } else {
                    W::template read<(J + 1) & 3>(fn, wrow, h);
                }
            }
            if constexpr (kLast) {
                stage(nxt, s, 0);
                stage(nxt, s, 1);
            } else {
                an[0][s] = afrag(next_tile, 0, s);
                an[1][s] = afrag(next_tile, 1, s);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    ph8 fa[2][4], fb[2][4];
    typename W::Frag f0, f1;
    // group q, reading LDS activation buffer rd and staging the next group into wr
    auto group = [&](int q, const char* rd, char* wr_buf, uint32_t (&x)[4][4], uint32_t (&y)[4][4]) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) fa[u][s4] = afrag(rd, u, s4);
        if constexpr (W::kDirect) {
            dma(4 * q + 2);  // before the eight activation loads: the first iteration's wait counts them
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (W::kDmaGroup) {
            dma_group(q + 1);  // before the eight activation loads: the third iteration's wait counts them
            __builtin_amdgcn_sched_barrier(0);
        }
        load_next(q + 1);
        iter(pos_t<1>{}, q, fa, fb, rd + kPStage, x, y, f1, f0, wr_buf);
        iter(pos_t<2>{}, q, fb, fa, rd + 2 * kPStage, y, x, f0, f1, wr_buf);
        iter(pos_t<3>{}, q, fa, fb, rd + 3 * kPStage, x, y, f1, f0, wr_buf);
        iter(pos_t<0>{}, q, fb, fa, rd, y, x, f0, f1, wr_buf);
        __syncthreads();
    };

    uint32_t b0[4][4], b1[4][4];
    if constexpr (W::kDirect) {
        dma(0);
        dma(1);
    }
    if constexpr (W::kDmaGroup) dma_group(0);
    load_next(0);
    write_w();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        stage(lds, j, 0);
        stage(lds, j, 1);
    }
    if constexpr (W::kDirect) {
        p_wait_vm<0>();  // the copies of steps 0 and 1
        W::read_buf(f0, step_buf(0), fr, h);
    } else if constexpr (W::kDmaGroup) {
        p_wait_vm<0>();  // group 0's copy
        W::template read<0>(f0, wrow_b(0), h);
    } else
        W::template read<0>(f0, wrow, h);
    {
        typename W::Consts k;
        W::template prep<0>(f0, k);
        W::template sub<0, 0>(f0, k, b0[0]);
        W::template sub<0, 1>(f0, k, b0[1]);
        W::template sub<0, 2>(f0, k, b0[2]);
        W::template sub<0, 3>(f0, k, b0[3]);
    }
    if constexpr (W::kDirect)
        W::read_buf(f1, step_buf(1), fr, h);
    else
        W::template read<1>(f1, wrow_b(0), h);
    __syncthreads();
    char* const buf0 = lds;
    char* const buf1 = lds + 4 * kPStage;
    if constexpr (W::kOneGroupPerTrip) {
        // one group per trip, the buffers swapped: the reads of the next group's first steps
        // (issued in this group's last two iterations; global loads for kDirect formats) stay
        // ahead of their use; after an unrolled pair with a break between them the compiler
        // sinks them past the break
        char* rd = buf0;
        char* wb = buf1;
        for (int q = 0; q < ngrp; ++q) {
            group(q, rd, wb, b0, b1);
            char* const t = rd;
            rd = wb;
            wb = t;
        }
    } else {
        for (int q = 0; q < ngrp; q += 2) {
            group(q, buf0, buf1, b0, b1);
            if (q + 1 >= ngrp) break;
            group(q + 1, buf1, buf0, b0, b1);
        }
    }

    // kDirect: the copies issued for steps past the split's end land before the workgroup's LDS
    // is released
    if constexpr (W::kDirect || W::kDmaGroup) p_wait_vm<0>();

    // rows whose activations left fp16's range take the fp32 path below
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        float v = amax[i];
        v = fmaxf(v, __shfl_xor(v, 1));
        v = fmaxf(v, __shfl_xor(v, 2));
        v = fmaxf(v, __shfl_xor(v, 4));
        v = fmaxf(v, __shfl_xor(v, 8));
        if (ap == 0) rowflag[ar0 + 32 * i] = (v >= kPRowMax || (v > 0.0f && v < kPRowMin)) ? 1 : 0;
    }
    __syncthreads();
    // the 64 flags as one wave-uniform mask (bit ml: row m0 + ml takes the fp32 path)
    const unsigned long long flagged = __ballot(rowflag[lane] != 0);

    // lane: column n0 + fr, rows m0 + 32 u + 8 g + 4 h + r (accumulator 4 g + r); the stores
    // stream past the caches (the output is not read again by this kernel)
    // (part: a K split's partial sums, split s at part + s M N, plain stores in place of atomics)
    float* const out = part ? part + static_cast<long>(ksplit) * M * N : C;
    const bool add = atomic && !part;
    const int n = n0 + fr;
    const int mrows = M - m0;  // rows of this tile inside C
    if (swiglu) {
        // the 64 x 256 tile through LDS (above the flags; every operand read is done), then
        // thread -> output column nt * 128 + (tid & 127) of rows tid >> 7, + 4, ...:
        // SiLU(gate) * up with the bits of the separate elementwise kernel
        float* const ct = reinterpret_cast<float*>(lds + 256);
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int i = 0; i < 16; ++i) ct[(32 * u + 8 * (i >> 2) + 4 * h + (i & 3)) * kPTN + 32 * wave + fr] = acc[u][i];
        __syncthreads();
        const int j = tid & (kPTN / 2 - 1), col = nt * (kPTN / 2) + j;
        for (int ml = tid / (kPTN / 2); ml < kPTM; ml += kPThreads / (kPTN / 2))
            if (ml < mrows && col < F && !((flagged >> ml) & 1ull))
                __builtin_nontemporal_store(silu_f(ct[ml * kPTN + j]) * ct[ml * kPTN + kPTN / 2 + j],
                                            C + static_cast<long>(m0 + ml) * F + col);
    } else {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int ml = 32 * u + 8 * (i >> 2) + 4 * h + (i & 3);
                if (ml < mrows && n < N && !((flagged >> ml) & 1ull)) {
                    float* cp = out + static_cast<long>(m0 + ml) * N + n;
                    if (add)
                        atomicAdd(cp, acc[u][i]);
                    else
                        __builtin_nontemporal_store(acc[u][i], cp);
                }
            }
    }

    // fp32 path for flagged rows: thread -> column nt * 256 + (tid & 255) of the flagged rows
    // of parity tid >> 8, the reference's per-element decode and a sequential fp32 sum over
    // this workgroup's k range
    const int fmt = W::kFmt;
    if (swiglu) {
        // thread -> output column nt * 128 + (tid & 127) of the flagged rows of class tid >> 7 (mod
        // 4): the gate and up sums over the whole k range (no split), then SiLU(gate) * up
        for (unsigned long long rest = flagged & (0x1111111111111111ull << (tid >> 7)); rest != 0; rest &= rest - 1) {
            const int ml = __builtin_ctzll(rest);
            const int m = m0 + ml, col = nt * (kPTN / 2) + (tid & (kPTN / 2 - 1));
            if (m >= M || col >= F) continue;
            const float* x = A + static_cast<long>(m) * K;
            const uint8_t* gp = B + static_cast<long>(col) * row_bytes;
            const uint8_t* up = B + static_cast<long>(F + col) * row_bytes;
            float g = 0.0f, v = 0.0f;
            for (int k = 0; k < K; ++k) {
                g = __builtin_fmaf(x[k], decode_row_elem(fmt, gp, k), g);
                v = __builtin_fmaf(x[k], decode_row_elem(fmt, up, k), v);
            }
            C[static_cast<long>(m) * F + col] = silu_f(g) * v;
        }
        return;
    }
    for (unsigned long long rest = flagged & (0x5555555555555555ull << (tid >> 8)); rest != 0; rest &= rest - 1) {
        const int ml = __builtin_ctzll(rest);
        const int m = m0 + ml, nn = nt * kPTN + (tid & 255);
        if (m >= M || nn >= N) continue;
        const float* x = A + static_cast<long>(m) * K;
        const uint8_t* wp = B + static_cast<long>(nn) * row_bytes;
        float sum = 0.0f;
        for (int k = s_begin * kPKS; k < s_end * kPKS; ++k) sum = __builtin_fmaf(x[k], decode_row_elem(fmt, wp, k), sum);
        float* cp = out + static_cast<long>(m) * N + nn;
        if (add)
            atomicAdd(cp, sum);
        else
            *cp = sum;
    }
}

}  // namespace
}  // namespace dev

namespace detail {

bool prefill_supported(int fmt, int M, int N, int K, const void* A, const void* B) {
    if (fmt != kFmtQ4_K && fmt != kFmtQ8_0 && fmt != kFmtQ6_K && fmt != kFmtQ4_0 && fmt != kFmtQ5_0 && fmt != kFmtF16)
        return false;
    // whole groups of four 64-column steps (one Q4_K / Q6_K super-block, eight 32-element blocks)
    if (M < 1 || N < 1 || K < 4 * dev::kPKS || K % (4 * dev::kPKS) != 0) return false;
    if (static_cast<long>(M) * K >= (1L << 31) || 32 * row_bytes(fmt, K) >= (1L << 31)) return false;
    const uintptr_t a = reinterpret_cast<uintptr_t>(A), b = reinterpret_cast<uintptr_t>(B);
    // activations are read as 16-byte vectors, weights as 16-byte pieces of dword-aligned rows
    return (a & 15) == 0 && (b & 3) == 0;
}

namespace {

// The kernels use more than the default 64 KB of LDS; the limit is raised once per kernel and device.
template <class W>
int launch_w(dim3 grid, hipStream_t stream, const float* A, const uint8_t* B, float* C, int M, int N, int K, long rb,
             int MT, int NT, int sps, int remap, int atomic, float* part, int swiglu = 0) {
    constexpr int kMaxDevices = 64;
    constexpr int kLds = dev::prefill_lds_bytes<W>();
    static std::atomic<bool> ready[kMaxDevices];
    int devid = 0;
    if (hipGetDevice(&devid) != hipSuccess || devid < 0 || devid >= kMaxDevices) return kFailed;
    if (!ready[devid].load(std::memory_order_acquire)) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&dev::prefill_gemm_kernel<W>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, kLds) != hipSuccess)
            return kFailed;
        ready[devid].store(true, std::memory_order_release);
    }
    hipLaunchKernelGGL(dev::prefill_gemm_kernel<W>, grid, dim3(dev::kPThreads), kLds, stream, A, B, C, M, N, K, rb,
                       MT, NT, sps, remap, atomic, part, swiglu);
    return 0;  // the launch's own status is read by the caller
}

}  // namespace

// k steps per split and the number of splits: the k range is split over workgroups (whole
// groups of four steps each) while the tiles alone fill fewer than 256 CUs
static int prefill_steps_per_split(int M, int N, int K, int* splits) {
    const long tiles = static_cast<long>((M + dev::kPTM - 1) / dev::kPTM) * ((N + dev::kPTN - 1) / dev::kPTN);
    const int nsteps = K / dev::kPKS;
    int kmax = 1;
    while (tiles * kmax < 256 && nsteps >= 16 * kmax) kmax *= 2;
    // one workgroup per CU: of the splits up to kmax, the one with the fewest groups of four steps
    // in sequence on a CU (rounds of 256 workgroups x groups per split), the fewer splits on a tie
    // (512 x 3072 x 2048: two splits in one round rather than four in two)
    const long groups = (nsteps + 3) / 4;
    int ks = 1;
    long best = groups;
    for (int k = 2; k <= kmax; k *= 2) {
        const long cost = (tiles * k + 255) / 256 * ((groups + k - 1) / k);
        if (cost < best) best = cost, ks = k;
    }
    int sps = (nsteps + ks - 1) / ks;
    sps = (sps + 3) / 4 * 4;  // groups of four steps: splits start on one
    *splits = (nsteps + sps - 1) / sps;
    return sps;
}

long prefill_workspace_floats(int M, int N, int K) {
    if (M < 1 || N < 1 || K < 4 * dev::kPKS || K % (4 * dev::kPKS) != 0) return 0;
    int ks = 1;
    prefill_steps_per_split(M, N, K, &ks);
    return ks > 1 && ks <= dev::kSplitMaxS ? static_cast<long>(ks) * M * N : 0;
}

int launch_prefill_swiglu(int fmt, const float* A, const void* B, float* C, int M, int F, int K, hipStream_t stream) {
    if (F < 1 || !prefill_supported(fmt, M, 2 * F, K, A, B)) return kDeclined;
    const int MT = (M + dev::kPTM - 1) / dev::kPTM;
    const int NT = (F + dev::kPTN / 2 - 1) / (dev::kPTN / 2);
    const long tiles = static_cast<long>(MT) * NT;
    // whole k range per workgroup: the epilogue needs finished sums
    int ks = 1;
    prefill_steps_per_split(M, 2 * F, K, &ks);
    if (ks > 1 || tiles > 0x7FFFFFFFL) return kDeclined;
    const int sps = K / dev::kPKS;
    const int remap = tiles % 8 == 0 ? 1 : 0;
    const long rb = row_bytes(fmt, K);
    const dim3 g(static_cast<unsigned>(tiles));
    const uint8_t* Bb = static_cast<const uint8_t*>(B);
    const int N = 2 * F;
    if (fmt == kFmtQ4_K) return launch_w<dev::PQ4K>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, 0, nullptr, 1);
    if (fmt == kFmtQ6_K) return launch_w<dev::PQ6K>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, 0, nullptr, 1);
    if (fmt == kFmtQ4_0) return launch_w<dev::PQ4_0>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, 0, nullptr, 1);
    if (fmt == kFmtQ5_0) return launch_w<dev::PQ5_0>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, 0, nullptr, 1);
    if (fmt == kFmtF16) return launch_w<dev::PF16>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, 0, nullptr, 1);
    return launch_w<dev::PQ8_0>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, 0, nullptr, 1);
}

int launch_prefill(int fmt, const float* A, const void* B, float* C, int M, int N, int K, hipStream_t stream, float* ws,
                   long ws_floats, SplitSums* defer, int defer_S) {
    if (defer) defer->S = 0;
    const int MT = (M + dev::kPTM - 1) / dev::kPTM;
    const int NT = (N + dev::kPTN - 1) / dev::kPTN;
    const long tiles = static_cast<long>(MT) * NT;
    int ks = 1;
    const int sps = prefill_steps_per_split(M, N, K, &ks);
    const long grid = tiles * ks;
    if (grid > 0x7FFFFFFFL) return kDeclined;
    const int remap = grid % 8 == 0 ? 1 : 0;
    const int atomic = ks > 1 ? 1 : 0;
    // A K split goes, when a workspace holds its partial sums, to plain stores there (split s at
    // ws + s M N), added up in split order by the consumer (defer) or by the reduction kernel:
    // deterministic, and no zero fill; without one, fp32 atomics into a zero-filled C, whose
    // order (and so the last bits) varies.  The atomics are dear: at 512 x 2048 x 8192 Q4_K the
    // kernel storing in their place took 35.3 against 43.0 us (same box), and with the workspace
    // and the reduction launch the product takes 37.3 against 41.1 us.
    const long mn = static_cast<long>(M) * N;
    float* part = nullptr;
    if (atomic && ws && ks <= dev::kSplitMaxS && ks * mn <= ws_floats && N % 4 == 0 &&
        (reinterpret_cast<uintptr_t>(ws) & 15u) == 0 && (defer ? defer_S == 0 || defer_S == ks
                                                              : (reinterpret_cast<uintptr_t>(C) & 15u) == 0))
        part = ws;
    if (atomic && !part) launch_fill_zero(C, mn, stream);
    const long rb = row_bytes(fmt, K);
    const dim3 g(static_cast<unsigned>(grid));
    const uint8_t* Bb = static_cast<const uint8_t*>(B);
    int rc;
    if (fmt == kFmtQ4_K)
        rc = launch_w<dev::PQ4K>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, atomic, part);
    else if (fmt == kFmtQ6_K)
        rc = launch_w<dev::PQ6K>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, atomic, part);
    else if (fmt == kFmtQ4_0)
        rc = launch_w<dev::PQ4_0>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, atomic, part);
    else if (fmt == kFmtQ5_0)
        rc = launch_w<dev::PQ5_0>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, atomic, part);
    else if (fmt == kFmtF16)
        rc = launch_w<dev::PF16>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, atomic, part);
    else
        rc = launch_w<dev::PQ8_0>(g, stream, A, Bb, C, M, N, K, rb, MT, NT, sps, remap, atomic, part);
    if (rc != 0 || !part) return rc;
    SplitSums sums;
    sums.part = part;
    sums.stride = mn;
    sums.S = ks;
    sums.N = N;
    sums.K = K;
    if (defer)
        *defer = sums;  // the consumer adds them up
    else
        launch_split_reduce(sums, C, M, stream);
    return 0;
}

}  // namespace detail
}  // namespace cri

// common.hpp -- device helpers shared by the gfx950 kernels.
//
// Everything here is written for CDNA4 wave64: cross-lane reductions use DPP
// row operations within 16-lane rows and ds_swizzle/bpermute across rows.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cri {
namespace dev {

// 16-byte vector whose address is only promised to be 4-byte aligned: the
// backend emits global_load_dwordx4, which gfx950 accepts at dword alignment.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ u32x4 ld_u32x4(const uint8_t* p) {  // p % 4 == 0
    u32x4_a4 v = *reinterpret_cast<const u32x4_a4*>(p);
    return u32x4{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ u32x4 ld_u32x4_a16(const uint8_t* p) {  // p % 16 == 0
    return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) {  // p % 4 == 0
    return *reinterpret_cast<const uint32_t*>(p);
}
__device__ __forceinline__ f32x4 ld_f32x4(const float* p) {  // p % 4 == 0 (bytes)
    f32x4_a4 v = *reinterpret_cast<const f32x4_a4*>(p);
    return f32x4{v.x, v.y, v.z, v.w};
}

// IEEE binary16 held in the low / high 16 bits of a dword, widened exactly.
__device__ __forceinline__ float h_lo(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w)));
}
__device__ __forceinline__ float h_hi(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}

// A small unsigned integer v < 1024 placed in the low or high half of a dword
// with nothing else in that half is the binary16 subnormal v * 2^-24, so
// fma(h(w), x, acc) multiplies by v exactly; the 2^24 is folded into the
// block scale.  The backend turns fma(fpext(half), f32, f32) into a single
// v_fma_mix_f32, so each weight costs one VALU op after masking.
constexpr float kTwo24 = 16777216.0f;

// Signed byte b of a dword, as float (exact).
__device__ __forceinline__ float sbyte(uint32_t w, int b) {
    return static_cast<float>(static_cast<int8_t>(w >> (8 * b)));
}
// Unsigned byte b of a dword, as float (exact; v_cvt_f32_ubyteN).
__device__ __forceinline__ float ubyte(uint32_t w, int b) {
    return static_cast<float>((w >> (8 * b)) & 0xFFu);
}

// Funnel shift: bytes [s, s+4) of the 8-byte little-endian pair (lo, hi).
__device__ __forceinline__ uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t s) {
    return __builtin_amdgcn_alignbyte(hi, lo, s);
}

__device__ __forceinline__ uint32_t ubfe(uint32_t v, uint32_t off, uint32_t width) {
    return __builtin_amdgcn_ubfe(v, off, width);
}

// ---- cross-lane reductions -------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// DPP control words (CDNA ISA, DPP_CTRL).
constexpr int kQuadPerm1032 = 0xB1;  // lane i <- lane i^1 within a quad
constexpr int kQuadPerm2301 = 0x4E;  // lane i <- lane i^2 within a quad
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;

__device__ __forceinline__ float swizzle_xor16(float v) {
    // ds_swizzle bit mode: and_mask=0x1F, or_mask=0, xor_mask=0x10
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}
__device__ __forceinline__ float shfl_xor32(float v) {
    const int lane = __lane_id();
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __builtin_bit_cast(int, v)));
}

// Sum over aligned groups of 2^log2n lanes (1 <= 2^log2n <= 64); every lane of
// the group receives the group total.
__device__ __forceinline__ float group_sum(float v, int log2n) {
    if (log2n >= 1) v += dpp<kQuadPerm1032>(v);
    if (log2n >= 2) v += dpp<kQuadPerm2301>(v);
    if (log2n >= 3) v += dpp<kRowHalfMirror>(v);
    if (log2n >= 4) v += dpp<kRowMirror>(v);
    if (log2n >= 5) v += swizzle_xor16(v);
    if (log2n >= 6) v += shfl_xor32(v);
    return v;
}

// Maximum over the whole wave; every lane receives it.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<kQuadPerm1032>(v));
    v = fmaxf(v, dpp<kQuadPerm2301>(v));
    v = fmaxf(v, dpp<kRowHalfMirror>(v));
    v = fmaxf(v, dpp<kRowMirror>(v));
    v = fmaxf(v, swizzle_xor16(v));
    v = fmaxf(v, shfl_xor32(v));
    return v;
}

template <int LOG2N>
__device__ __forceinline__ float group_sum_t(float v) {
    if constexpr (LOG2N >= 1) v += dpp<kQuadPerm1032>(v);
    if constexpr (LOG2N >= 2) v += dpp<kQuadPerm2301>(v);
    if constexpr (LOG2N >= 3) v += dpp<kRowHalfMirror>(v);
    if constexpr (LOG2N >= 4) v += dpp<kRowMirror>(v);
    if constexpr (LOG2N >= 5) v += swizzle_xor16(v);
    if constexpr (LOG2N >= 6) v += shfl_xor32(v);
    return v;
}

}  // namespace dev
}  // namespace cri

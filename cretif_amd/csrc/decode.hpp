// decode.hpp -- per-element decode of one quantized block, in the reference's
// own arithmetic (ref:src/kernels/dequantize.cu).  Every product involved is
// exact in binary32 (fp16 scale: 11 significant bits; codes: <= 13 bits), so
// the results are bit-identical to the reference whether or not the compiler
// contracts d*sc*q - dmin*mn into an FMA.
#pragma once

#include "common.hpp"
#include "internal.hpp"

namespace cri {
namespace dev {

__device__ __forceinline__ float half_at(const uint8_t* p) {
    const uint16_t h = static_cast<uint16_t>(p[0] | (p[1] << 8));
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// ref:src/kernels/dequantize.cu:45-47
__device__ __forceinline__ float decode_q8_0(const uint8_t* blk, int e) {
    return half_at(blk) * static_cast<float>(static_cast<int8_t>(blk[2 + e]));
}

// ref:src/kernels/dequantize.cu:84-100 (element e <- qs[e/2], low nibble for even e)
__device__ __forceinline__ float decode_q4_0(const uint8_t* blk, int e) {
    const uint8_t b = blk[2 + (e >> 1)];
    const int nib = (e & 1) ? (b >> 4) : (b & 0x0F);
    return half_at(blk) * static_cast<float>(nib - 8);
}

// ref:src/kernels/dequantize.cu:137-164
__device__ __forceinline__ float decode_q5_0(const uint8_t* blk, int e) {
    const uint32_t qh = static_cast<uint32_t>(blk[2]) | (static_cast<uint32_t>(blk[3]) << 8) |
                        (static_cast<uint32_t>(blk[4]) << 16) | (static_cast<uint32_t>(blk[5]) << 24);
    const int j = e & 15;
    const int low4 = (e < 16) ? (blk[6 + j] & 0x0F) : (blk[6 + j] >> 4);
    const int hb = static_cast<int>((qh >> e) & 1u);
    return half_at(blk) * static_cast<float>((low4 | (hb << 4)) - 16);
}

// ref:src/kernels/dequantize.cu:215-243
__device__ __forceinline__ float decode_q6_k(const uint8_t* blk, int e) {
    const int chunk = e >> 7, within = e & 127;
    const int quarter = within >> 5, l = within & 31;
    const int scale_idx = chunk * 8 + quarter * 2 + (l >> 4);
    const float sc = static_cast<float>(static_cast<int8_t>(blk[192 + scale_idx]));
    const int ql_off = (quarter & 1) * 32 + l + chunk * 64;
    const int qln = quarter < 2 ? (blk[ql_off] & 0x0F) : (blk[ql_off] >> 4);
    const int qhb = (blk[128 + l + chunk * 32] >> (quarter * 2)) & 0x03;
    const int q6 = (qln | (qhb << 4)) - 32;
    return half_at(blk + 208) * sc * static_cast<float>(q6);
}

// ref:src/kernels/dequantize.cu:289-324
__device__ __forceinline__ float decode_q4_k(const uint8_t* blk, int e) {
    const float d = half_at(blk), dmin = half_at(blk + 2);
    const uint8_t* s = blk + 4;
    const int sb = e >> 5;
    int sc, mn;
    if (sb < 4) {
        sc = s[sb] & 0x3F;
        mn = s[sb + 4] & 0x3F;
    } else {
        sc = (s[sb + 4] & 0x0F) | ((s[sb - 4] >> 6) << 4);
        mn = (s[sb + 4] >> 4) | ((s[sb] >> 6) << 4);
    }
    const int chunk64 = e >> 6, within = e & 63, l = within & 31;
    const uint8_t b = blk[16 + chunk64 * 32 + l];
    const int nib = within < 32 ? (b & 0x0F) : (b >> 4);
    return d * static_cast<float>(sc) * static_cast<float>(nib) - dmin * static_cast<float>(mn);
}

// Element k of a row of `fmt` weights starting at `row`.
__device__ __forceinline__ float decode_row_elem(int fmt, const uint8_t* row, int k) {
    switch (fmt) {
        case kFmtQ8_0: return decode_q8_0(row + (k >> 5) * 34, k & 31);
        case kFmtQ4_0: return decode_q4_0(row + (k >> 5) * 18, k & 31);
        case kFmtQ5_0: return decode_q5_0(row + (k >> 5) * 22, k & 31);
        case kFmtQ4_K: return decode_q4_k(row + (k >> 8) * 144, k & 255);
        case kFmtQ6_K: return decode_q6_k(row + (k >> 8) * 210, k & 255);
        case kFmtF16: return half_at(row + 2 * k);
        case kFmtF32: return reinterpret_cast<const float*>(row)[k];
    }
    return 0.0f;
}

}  // namespace dev
}  // namespace cri

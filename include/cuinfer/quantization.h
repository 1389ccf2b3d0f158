// quantization.h -- GGUF block layouts and standalone dequant entry points.
//
// Same packed layouts, names and sizes as ref:include/cuinfer/quantization.h:38-134
// (they are the GGUF on-disk format, so they cannot differ).  `__half` is
// HIP's binary16 type.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace cuinfer {

struct BlockQ8_0 {
    __half scale;
    int8_t qs[32];
};
static_assert(sizeof(BlockQ8_0) == 34, "BlockQ8_0 must be 34 bytes");

struct BlockQ4_0 {
    __half scale;
    uint8_t qs[16];  // element i <- qs[i/2], low nibble for even i
};
static_assert(sizeof(BlockQ4_0) == 18, "BlockQ4_0 must be 18 bytes");

struct BlockQ5_0 {
    __half scale;
    uint8_t qh[4];   // bit i = fifth bit of element i (little-endian u32)
    uint8_t qs[16];  // element i < 16: low nibble of qs[i]; i >= 16: high nibble of qs[i-16]
};
static_assert(sizeof(BlockQ5_0) == 22, "BlockQ5_0 must be 22 bytes");

struct BlockQ6_K {
    uint8_t ql[128];
    uint8_t qh[64];
    int8_t scales[16];
    __half d;
};
static_assert(sizeof(BlockQ6_K) == 210, "BlockQ6_K must be 210 bytes");

struct BlockQ4_K {
    __half d;
    __half dmin;
    uint8_t scales[12];
    uint8_t qs[128];
};
static_assert(sizeof(BlockQ4_K) == 144, "BlockQ4_K must be 144 bytes");

constexpr int Q8_0_BLOCK_SIZE = 32;
constexpr int Q4_0_BLOCK_SIZE = 32;
constexpr int Q5_0_BLOCK_SIZE = 32;
constexpr int Q4_K_BLOCK_SIZE = 256;
constexpr int Q6_K_BLOCK_SIZE = 256;

// dst[n_blocks * block_size] = dequant(src); device pointers; throw std::runtime_error on error.
void dequantize_q8_0(const void* src, float* dst, int n_blocks, hipStream_t stream = 0);
void dequantize_q4_0(const void* src, float* dst, int n_blocks, hipStream_t stream = 0);
void dequantize_q5_0(const void* src, float* dst, int n_blocks, hipStream_t stream = 0);
void dequantize_q6_k(const void* src, float* dst, int n_blocks, hipStream_t stream = 0);
void dequantize_q4_k(const void* src, float* dst, int n_blocks, hipStream_t stream = 0);

}  // namespace cuinfer

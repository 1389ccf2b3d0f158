// weights.h -- GGUF weights onto the device in the form the fused matmuls read.
//
// load_weight_quantized keeps the reference's behaviour
// (ref:src/model.cu:322-414): a 2-D tensor's raw GGUF blocks are uploaded
// unchanged as [N, K] (GGUF dims {K, N}); the per-tensor format comes from the
// tensor's type (Q4_K_M files mix Q4_K and Q6_K).  FP32 tensors are uploaded
// as [N, K] too, for matmul_transposed_b (the reference transposes them for
// its FP32 [K, N] matmul, which is not part of this library).
//
// load_lm_head returns output.weight, or token_embd.weight when the file ties
// the two -- kept in its file format.  The reference dequantizes a tied table
// to FP32 (1.05 GB for 128256 x 2048, ref:src/model.cu:603, 1027-1029), so its
// LM head streams 4-8x the bytes of the quantized GEMV this enables.
// embedding_lookup reads token rows straight from the same quantized table.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <string>

#include "dispatch.h"
#include "gguf_parser.h"
#include "tensor.h"

namespace cuinfer {

// GGML type of a tensor -> the library's weight format; throws for types the
// fused matmuls do not take (Q4_1, Q5_1, Q8_1, Q2_K, Q3_K, Q5_K).
WeightFormat ggml_type_to_weight_format(GGMLType type);

Tensor load_weight_quantized(const GGUFParser& parser, const std::string& name, WeightFormat& out_format);

// The LM head weight [vocab, dim] in its file format; *tied tells which tensor it is.
Tensor load_lm_head(const GGUFParser& parser, WeightFormat& out_format, bool* tied = nullptr);

// out[i, :] = dequant(table row ids[i]) for n_ids device token ids; rows of
// ids outside [0, vocab) are written as zeros.  Bit-identical to dequantizing
// the table and gathering the rows.
void embedding_lookup(const Tensor& table, WeightFormat format, const int32_t* ids, float* out, int n_ids,
                      hipStream_t stream = 0);

}  // namespace cuinfer

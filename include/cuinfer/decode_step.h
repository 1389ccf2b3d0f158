// decode_step.h -- one transformer step over M tokens with preallocated
// buffers, built on matmul_dispatch and captured as one HIP graph.
//
// The step is the layer loop of TransformerModel::forward's quantized path
// (ref:src/model.cu:831-1039): token embedding; per layer RMSNorm, the q/k/v
// projections, RoPE on q and k (ref:src/kernels/elementwise.cu:232-266), the
// KV-cache append (ref:src/kv_cache.cu:157-211), attention over the cache,
// the o projection, residual + RMSNorm, gate/up, SiLU * up, down, residual;
// then the final RMSNorm, the LM head and (optionally) the greedy token
// (argmax_sample, ref:src/embedding.cu:305-326).  Differences, each deliberate:
//   * every buffer is allocated once, at construction (the reference allocates
//     q/k/v, attn_concat and attn_out with Tensor::zeros inside the layer loop,
//     ref:src/model.cu:906-908, 937, 946, and two device words per argmax);
//   * q/k/v weights of one format are stored as one [q_dim + 2 kv_dim, dim]
//     matrix and gate/up as one [2 ffn, dim] matrix (GGUF rows are
//     independent, so stacking them is a byte concatenation): one launch each;
//   * for batches of up to 16 tokens the RMSNorm (with the residual add) and
//     SiLU * up are computed inside the next matmul's activation staging
//     (matmul_dispatch_rmsnorm / matmul_dispatch_swiglu);
//   * attention is a split online-softmax kernel for batches of up to 16 tokens
//     and, above that (a prompt), the reference's prefill flow of Q K^T and P V
//     through batched_matmul_gqa around a causal softmax (ref:src/attention.cu:
//     809-871); row m of the batch sees the first position() + m + 1 cache
//     positions, which is the reference's causal mask (ref:src/attention.cu:60-75)
//     for a multi-token call and its fused decode attention for one token;
//   * the sequence position lives in device memory and the step's own last
//     kernel advances it, so a captured step can be replayed for every
//     following token without being captured again.
//
// Weights are copied into the step's own device buffers from host or device
// memory (hipMemcpyDefault) in their GGUF [N, K] block layout.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <memory>
#include <vector>

#include "dispatch.h"
#include "tensor.h"

namespace cuinfer {

// The ModelConfig fields a step needs (ref:include/cuinfer/model.h:62-76),
// plus the largest batch (tokens per call) the buffers are sized for.
struct DecodeStepConfig {
    int n_layers = 0;
    int dim = 0;
    int n_heads = 0;
    int n_kv_heads = 0;
    int head_dim = 0;
    int intermediate_size = 0;
    int vocab_size = 0;
    int max_seq_len = 0;
    float rms_norm_eps = 1e-5f;
    float rope_theta = 10000.0f;
    int max_batch = 16;
};

// A weight matrix [N, K] in GGUF row order, in host or device memory.
struct WeightRef {
    WeightFormat format = WeightFormat::Q4_K;
    const void* data = nullptr;
};

// One layer's tensors (blk.N.* in a GGUF file); the norms are fp32 [dim].
struct LayerWeightsRef {
    const float* attn_norm = nullptr;
    const float* ffn_norm = nullptr;
    WeightRef q, k, v, o, gate, up, down;
};

class DecodeStep {
public:
    // Allocates the weights' and activations' buffers and the KV cache
    // (2 * n_layers * max_seq_len * n_kv_heads * head_dim floats).  Throws
    // std::invalid_argument for an inconsistent configuration.
    explicit DecodeStep(const DecodeStepConfig& cfg);
    ~DecodeStep();
    DecodeStep(const DecodeStep&) = delete;
    DecodeStep& operator=(const DecodeStep&) = delete;

    // The setters copy into new buffers and swap them in only when every copy succeeded (a
    // throw leaves the earlier tensors in place), and every setter discards a captured graph
    // (it holds the old buffers' addresses and kernel choices): replay() then throws until
    // capture() runs again.
    void set_layer(int layer, const LayerWeightsRef& w);
    // token embedding table [vocab, dim]: FP32 or any matmul format
    void set_token_embedding(const WeightRef& table);
    // final norm and LM head [vocab, dim]; lm_head == nullptr ties it to the
    // token table, kept in that table's format (an FP32 table multiplies
    // through matmul_transposed_b, as the reference's tied head does)
    void set_output(const float* output_norm, const WeightRef* lm_head);

    // Runs M tokens (1 <= M <= max_batch) at positions position() ..
    // position() + M - 1: token ids (device int32 [M]) -> logits (device fp32
    // [M, vocab]); next_ids (device int32 [M], may be null) receives the
    // argmax of each logits row.  Enqueued on `stream`; advances position().
    void forward(const int32_t* token_ids, int M, float* logits, int32_t* next_ids, hipStream_t stream = 0);
    // A prompt the way the reference's generate() consumes it (ref:src/model.cu:1063-1078): every
    // layer runs on the M tokens (the caches take their keys and values, position() advances by
    // M), and the final RMSNorm, the LM head and the argmax run for the last row only: logits
    // (device fp32 [vocab]) of token M - 1, next_id (device int32 [1], may be null) its argmax.
    // forward() computes every row's logits as the reference's forward() does; this skips the
    // M - 1 rows generate() never reads.
    void prefill(const int32_t* token_ids, int M, float* logits, int32_t* next_id, hipStream_t stream = 0);
    // forward() that also writes the residual stream entering each layer and the final norm:
    // hidden_taps (device fp32 [n_layers + 1, M, dim]) slice i = the hidden state layer i
    // reads (slice n_layers: the one the final RMSNorm reads), each added up from its pending
    // residual the way the next RMSNorm adds it.  The same kernels run as in forward(), plus
    // one small kernel per slice; for checking a step layer by layer.
    void forward_taps(const int32_t* token_ids, int M, float* logits, int32_t* next_ids, float* hidden_taps,
                      hipStream_t stream = 0);

    // Captures forward(token_ids, M, logits, next_ids) on `stream` (not the
    // null stream) as one HIP graph, replacing any earlier capture; nothing
    // runs and position() is unchanged.  replay() launches it on `stream`:
    // each replay is one more step of M tokens (next_ids may be token_ids, so
    // replays generate greedily).
    void capture(const int32_t* token_ids, int M, float* logits, int32_t* next_ids, hipStream_t stream);
    void replay(hipStream_t stream);

    int position() const { return pos_host_; }
    // sets the device position counter (reset = 0) with a kernel on `stream`
    void set_position(int pos, hipStream_t stream = 0);

    float* k_cache(int layer);  // [max_seq_len, n_kv_heads, head_dim]
    float* v_cache(int layer);
    const DecodeStepConfig& config() const { return cfg_; }
    size_t weight_bytes() const;  // every weight and norm byte held on the device
    // the weight bytes one step of M tokens reads: every layer's matrices and norms, the final
    // norm and LM head, and M rows of the token table (all of it when the head is tied to it)
    size_t step_weight_bytes(int M) const;
    int captured_batch() const { return graph_m_; }

private:
    struct Layer;
    void enqueue(const int32_t* token_ids, int M, float* logits, int32_t* next_ids, hipStream_t stream,
                 float* taps = nullptr, bool last_only = false);
    void check_ready() const;
    void check_call(const int32_t* token_ids, int M, float* logits, int32_t* next_ids, const char* what) const;
    void drop_graph();
    void attn_block(Layer& L, int li, int M, int& cur, const float*& res, hipStream_t s);
    void ffn_block(Layer& L, int li, int M, int& cur, const float*& res, hipStream_t s);
    // the consumer of layer li's FFN output (the next q/k/v or the LM head) is a batch-1 GEMV
    // that can add the down projection's K-split partial sums itself
    bool next_takes_split(int li) const;
    // RMSNorm(h + res) times W for one token with res as res_splits_ partial sums
    void norm_matmul_splitres(const float* h, const float* norm_w, float* h_out, const Tensor& W, WeightFormat f,
                              float* C, int N, hipStream_t s, const char* what);

    DecodeStepConfig cfg_;
    int q_dim_ = 0, kv_dim_ = 0;
    std::vector<std::unique_ptr<Layer>> layers_;
    Tensor tok_table_, out_norm_, lm_head_;
    WeightFormat tok_fmt_ = WeightFormat::FP32, lm_fmt_ = WeightFormat::FP32;
    bool tok_set_ = false, out_set_ = false, lm_tied_ = false;
    Tensor k_cache_, v_cache_, pos_dev_;
    Tensor hid_[2], normed_, qkv_, ctx_, attn_out_, ff_, act_, ffn_out_, attn_ws_, split_ws_, defer_ws_;
    Tensor argmax_part_, argmax_count_, rope_;
    // batches above 16 rows (a prompt): attention through batched_matmul_gqa in row blocks of up to
    // kPromptRows, on Q / K^T / V / scores / output workspaces (allocated when max_batch > 16)
    Tensor gqa_q_, gqa_k_, gqa_v_, gqa_s_, gqa_o_;
    bool capturing_ = false;  // enqueue() is recording a graph: shapes independent of the position
    // prompts (above 16 tokens) through the multi-row split attention (head_dim 64) instead of
    // batched_matmul_gqa around a materialized causal softmax
    bool prompt_mrow_ = false;
    Tensor res_parts_;    // the down projection's K-split partial sums at one token
    int res_splits_ = 0;  // > 0: the pending residual is that many partial sums in res_parts_
    // 2..16 tokens: the pending residual as the unreduced partial sums of the o projection, and
    // for a prompt those of a K-split o or down projection (res_part_count_ partial sums
    // res_part_stride_ floats apart from res_part_; 0: the plain residual pointer); the next
    // RMSNorm row kernel adds them to the hidden state and normalizes, and the projections after
    // it take plain activations
    Tensor norm_ss_;  // the row kernel's per-row sums of squares, [16 splits][16 rows], splits 1.. zero
    const float* res_part_ = nullptr;
    long res_part_stride_ = 0;
    int res_part_count_ = 0;
    bool split_flow(int M) const;
    // a prompt (above 16 tokens) leaves the o and down projections' K-split partial sums for the
    // RMSNorm row kernel that follows them (dim % 4 == 0, dim <= 4096)
    bool prompt_defers(int M) const;
    void prompt_norm(float* h, const float* res, const float* w, int M, hipStream_t s, const char* what);
    int pos_host_ = 0;
    hipGraph_t graph_ = nullptr;
    hipGraphExec_t graph_exec_ = nullptr;
    int graph_m_ = 0;
};

}  // namespace cuinfer

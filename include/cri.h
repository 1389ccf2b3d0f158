/*
 * cri.h -- C ABI of the MI355X (gfx950) fused dequant+matmul library.
 *
 * Every entry point takes device pointers owned by the caller, enqueues its
 * kernels on `stream` (0 = the null stream) and returns without
 * synchronising.  The library allocates no device memory and keeps no state
 * between calls, so calls are re-entrant on any stream.
 *
 * Return value: CRI_OK (0) on success, otherwise a negative cri_status; the
 * thread-local message from cri_last_error_string() says what was wrong.
 * Unlike the reference (which silently truncates K/32 and K/256), shapes are
 * validated before anything is launched.  Errors that happen while a kernel
 * executes surface at the caller's next synchronisation, as in the reference.
 *
 * Conventions (ref:include/cuinfer/kernels/matmul_quant.h:1-22):
 *   A : fp32 [M, K] row-major activations
 *   B : [N, K] weights in GGUF row order: row n is K/bs consecutive blocks
 *   C : fp32 [M, N] row-major output, fully overwritten (never accumulated)
 *   A, B and C must not overlap.
 */
#ifndef CRI_H
#define CRI_H

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum cri_status {
    CRI_OK = 0,
    CRI_ERR_INVALID_ARGUMENT = -1, /* null pointer or negative dimension       */
    CRI_ERR_SHAPE = -2,            /* K not a multiple of the block size, etc. */
    CRI_ERR_ALIGNMENT = -3,        /* pointer misaligned for its element type  */
    CRI_ERR_LAUNCH = -4,           /* the HIP runtime rejected a launch        */
    CRI_ERR_UNSUPPORTED = -5,      /* format id unknown                        */
    CRI_ERR_FILE = -6              /* GGUF file missing, unreadable, malformed */
} cri_status;

/* Weight formats; the numbering is shared with cri_matmul()/cri_dequantize(). */
typedef enum cri_format {
    CRI_Q8_0 = 0,
    CRI_Q4_0 = 1,
    CRI_Q5_0 = 2,
    CRI_Q4_K = 3,
    CRI_Q6_K = 4,
    CRI_FP16 = 5,
    CRI_FP32 = 6 /* only for cri_embedding_rows and cri_gguf_tensor.format */
} cri_format;

/* ---- fused dequant + matmul: C[M,N] = A[M,K] * dequant(B[N,K])^T ---------- */

/* replaces cuinfer::matmul_q8_0, ref:include/cuinfer/kernels/matmul_quant.h:37 (K % 32 == 0) */
int cri_matmul_q8_0(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t stream);
/* replaces cuinfer::matmul_q4_0, ref:include/cuinfer/kernels/matmul_quant.h:50 (K % 32 == 0) */
int cri_matmul_q4_0(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t stream);
/* replaces cuinfer::matmul_q5_0, ref:include/cuinfer/kernels/matmul_quant.h:63 (K % 32 == 0) */
int cri_matmul_q5_0(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t stream);
/* replaces cuinfer::matmul_q4_k, ref:include/cuinfer/kernels/matmul_quant.h:76 (K % 256 == 0) */
int cri_matmul_q4_k(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t stream);
/* replaces cuinfer::matmul_q6_k, ref:include/cuinfer/kernels/matmul_quant.h:88 (K % 256 == 0) */
int cri_matmul_q6_k(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t stream);
/* replaces cuinfer::matmul_fp16, ref:include/cuinfer/kernels/matmul_quant.h:104 (K % 32 == 0,
 * as the reference requires; B must be 2-byte aligned) */
int cri_matmul_fp16(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t stream);
/* format-switched form of the six above; mirrors the switch of matmul_dispatch,
 * ref:src/model.cu:797-825 (FP32 weights are not part of this library) */
int cri_matmul(int format, const float* A, const void* B, float* C, int M, int N, int K, hipStream_t stream);
/* cri_matmul with a caller workspace (no counterpart in the reference, whose matmuls take none):
 * the products whose K cri_matmul splits over workgroups with fp32 atomics -- 9..16 rows, and
 * above 16 rows the prefill GEMM's shapes with few output tiles (K % 256 == 0, e.g.
 * 512 x 2048 x 8192) -- store the partial sums in the workspace instead and add them in split
 * order in a second launch, so C has the same bits on every call (and the prefill shapes skip
 * the atomics and the zero fill: 512 x 2048 x 8192 Q4_K 41.1 -> 37.3 us).  Every other shape runs as
 * cri_matmul: 1..8 rows and unsplit products are deterministic there; above 16 rows with
 * K % 256 != 0 the k range may still be split with atomics.  workspace: device memory, 16-byte
 * aligned, at least cri_matmul_workspace_bytes(format, M, N, K) bytes; where it is used C must be
 * 16-byte aligned and N a multiple of 4 (CRI_ERR_ALIGNMENT otherwise).  Calls sharing a workspace
 * must be ordered on one stream. */
int cri_matmul_ws(int format, const float* A, const void* B, float* C, int M, int N, int K, void* workspace,
                  long long workspace_bytes, hipStream_t stream);
/* bytes of workspace cri_matmul_ws uses for this shape (0 when it uses none; a negative
 * cri_status for invalid arguments) */
long long cri_matmul_workspace_bytes(int format, int M, int N, int K);

/* ---- standalone dequant: dst[n_blocks * bs] = dequant(src) --------------- */

/* replaces cuinfer::dequantize_q8_0, ref:include/cuinfer/quantization.h:145 */
int cri_dequantize_q8_0(const void* src, float* dst, int n_blocks, hipStream_t stream);
/* replaces cuinfer::dequantize_q4_0, ref:include/cuinfer/quantization.h:152 */
int cri_dequantize_q4_0(const void* src, float* dst, int n_blocks, hipStream_t stream);
/* replaces cuinfer::dequantize_q5_0, ref:include/cuinfer/quantization.h:159 */
int cri_dequantize_q5_0(const void* src, float* dst, int n_blocks, hipStream_t stream);
/* replaces cuinfer::dequantize_q6_k, ref:include/cuinfer/quantization.h:166 */
int cri_dequantize_q6_k(const void* src, float* dst, int n_blocks, hipStream_t stream);
/* replaces cuinfer::dequantize_q4_k, ref:include/cuinfer/quantization.h:173 */
int cri_dequantize_q4_k(const void* src, float* dst, int n_blocks, hipStream_t stream);

/* ---- fp32 neighbours of the path ----------------------------------------- */

/* C[M,N] = A[M,K] * B[N,K]^T, all fp32; replaces cuinfer::matmul_transposed_b,
 * ref:include/cuinfer/embedding.h:136-137 (any K >= 1) */
int cri_matmul_transposed_b(const float* A, const float* B, float* C, int M, int N, int K,
                            hipStream_t stream);

/* C[h] = A[h] * B[h / (n_heads / n_kv_heads)] with A [n_heads, M, K],
 * B [n_kv_heads, K, N], C [n_heads, M, N], all fp32; replaces
 * cuinfer::batched_matmul_gqa, ref:include/cuinfer/attention.h:79-82
 * (n_heads % n_kv_heads == 0 is checked here; the reference checks it only in
 * AttentionBlock, ref:src/attention.cu:534-539) */
int cri_batched_matmul_gqa(const float* A, const float* B, float* C, int n_heads, int n_kv_heads,
                           int M, int N, int K, hipStream_t stream);

/* out[h, :] = softmax(scale * Q[h, :] . K[t, h / G, :] over t < kv_len) V[t, h / G, :]
 * for one query token, G = n_heads / n_kv_heads; Q [n_heads, head_dim],
 * K_cache / V_cache [>= kv_len, n_kv_heads, head_dim] (position stride
 * n_kv_heads * head_dim), out [n_heads, head_dim], all fp32; replaces
 * cuinfer::fused_decode_attention, ref:include/cuinfer/attention.h:161-167
 * (kernel ref:src/attention.cu:410-511).  Checked here: n_heads % n_kv_heads
 * == 0, kv_len >= 1 (the reference returns NaN for an empty cache) and
 * head_dim <= 256. */
int cri_fused_decode_attention(const float* Q, const float* K_cache, const float* V_cache, float* output,
                               int n_heads, int n_kv_heads, int head_dim, int kv_len, float scale,
                               hipStream_t stream);

/* Split form of cri_fused_decode_attention, with no counterpart in the
 * reference: for callers that can keep a device workspace (a decode loop or a
 * captured graph).  The cache positions are split over workgroups that each
 * read their K/V rows once for all the query heads of a KV head and write a
 * partial softmax state (max, sum, accumulator) per head to `workspace`; a
 * second kernel merges them.  The result equals cri_fused_decode_attention's
 * to fp32 rounding.  `workspace`: device memory, 16-byte aligned; the call
 * uses at most cri_fused_decode_attention_workspace_size() bytes of it (fewer
 * chunks when workspace_bytes is smaller; CRI_ERR_SHAPE below one record per
 * head).  Calls that share a workspace must be ordered on one stream.  Shapes
 * the split kernel does not take (head_dim > 128, head_dim % 4 != 0, Q/K/V not
 * 16-byte aligned) run cri_fused_decode_attention and leave the workspace
 * untouched. */
int cri_fused_decode_attention_ws(const float* Q, const float* K_cache, const float* V_cache, float* output,
                                  int n_heads, int n_kv_heads, int head_dim, int kv_len, float scale,
                                  void* workspace, long long workspace_bytes, hipStream_t stream);
/* No counterpart in the reference: cri_fused_decode_attention_ws without a
 * workspace argument and without any allocation, for callers that cannot call
 * hipMalloc (code under HIP graph capture, tight serving loops, harnesses that
 * forbid it).  The partial records live in a static device array of 1 MiB per
 * GPU (held until the process ends; every record is written before it is read,
 * so nothing needs clearing): fewer position chunks are used when a shape's
 * records would not fit, and CRI_ERR_SHAPE is returned when one record per head,
 * n_heads * (head_dim + 4) * 4 bytes, exceeds 1 MiB.  Needs 4 | head_dim <= 128
 * and 16-byte aligned Q, K_cache, V_cache (CRI_ERR_UNSUPPORTED otherwise).
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (different streams, or host threads) race and must be ordered by the caller.
 * The result equals cri_fused_decode_attention_ws's for the same shape. */
int cri_fused_decode_attention_noalloc(const float* Q, const float* K_cache, const float* V_cache, float* output,
                                       int n_heads, int n_kv_heads, int head_dim, int kv_len, float scale,
                                       hipStream_t stream);
/* Prompt attention over the [kv_len, n_kv_heads, head_dim] caches, the reference's prefill flow
 * (AttentionBlock::forward_from_qkv after the cache append, ref:src/attention.cu:809-871: Q K^T and
 * P V through batched_matmul_gqa around scale, causal mask and softmax): M query rows (already
 * rotated) at Q + m * ldq, [n_heads * head_dim] each, at positions pos .. pos + M - 1; row m
 * attends to cache positions [0, pos + m]; output row m at output + m * n_heads * head_dim.  The
 * caches must hold rows 0 .. pos + M - 1 (rows past them are never read into the products).
 * head_dim a multiple of 4 up to 128, ldq a multiple of 4; K_cache, V_cache, output and the
 * workspace 16-byte aligned; workspace_bytes at least
 * cri_prefill_attention_workspace_bytes(M, n_heads, n_kv_heads, head_dim, pos + M). */
int cri_prefill_attention(const float* Q, int ldq, const float* K_cache, const float* V_cache, float* output, int M,
                          int n_heads, int n_kv_heads, int head_dim, int pos, float scale, void* workspace,
                          long long workspace_bytes, hipStream_t stream);
long long cri_prefill_attention_workspace_bytes(int M, int n_heads, int n_kv_heads, int head_dim, int kv_len);
/* Workspace bytes cri_fused_decode_attention_ws uses for this shape (0 for an
 * empty problem; a negative cri_status for invalid arguments). */
long long cri_fused_decode_attention_workspace_size(int n_heads, int n_kv_heads, int head_dim, int kv_len);

/* ---- neighbour fusions: the activation computed while the matmul stages it -- */

/* C[M,N] = normed[M,K] * dequant(B[N,K])^T with v = hidden + residual and
 * normed = v * norm_weight * rsqrt(mean_k(v^2) + eps), the RMSNorm that feeds
 * q/k/v and gate/up (ref:src/kernels/elementwise.cu:463-513, called at
 * ref:src/model.cu:961-967 and :1012-1018 before matmul_dispatch).  v is also
 * written to hidden_out [M, K] when it is not null; hidden_out must not overlap
 * hidden or residual (checked).  residual may be null (plain RMSNorm).  No
 * counterpart in the reference: it replaces a rmsnorm_residual launch and the
 * normed buffer.  Decode batches only (1 <= M <= 16; CRI_ERR_UNSUPPORTED
 * above), every format; fp32 accuracy as cri_matmul at M <= 16. */
int cri_matmul_rmsnorm(int format, const float* hidden, const float* residual, const float* norm_weight,
                       float* hidden_out, const void* B, float* C, int M, int N, int K, float eps,
                       hipStream_t stream);
/* C[M,N] = (silu(gate) * up)[M,K] * dequant(B[N,K])^T, silu(x) = x / (1 + exp(-x)):
 * the FFN down projection of ref:src/model.cu:996-1002 with its silu and
 * multiply launches folded in.  gate and up rows are `ld` floats apart (ld >= K;
 * gate = buf, up = buf + inter, ld = 2 * inter reads a fused gate/up output).
 * No counterpart in the reference.  Decode batches only (1 <= M <= 16). */
int cri_matmul_swiglu(int format, const float* gate, const float* up, int ld, const void* B, float* C, int M,
                      int N, int K, hipStream_t stream);

/* Standalone forms, for batches the fused prologues do not take.
 * replaces cuinfer::rmsnorm_residual, ref:include/cuinfer/kernels/elementwise.h:107
 * (output may alias input; residual may be null) */
int cri_rmsnorm_residual(const float* input, const float* residual, const float* weight, float* output,
                         float* normed, int rows, int n, float eps, hipStream_t stream);
/* out = silu(gate) * up over n elements: cuinfer::silu then cuinfer::multiply,
 * ref:include/cuinfer/kernels/elementwise.h:23 and :75 (out may alias gate or up) */
int cri_silu_mul(const float* gate, const float* up, float* out, long long n, hipStream_t stream);

/* ---- GGUF files: the weights' on-disk format -------------------------------
 * A reader with the reference's parsing rules (ref:src/gguf_parser.cpp; the C++
 * class is cuinfer::GGUFParser in cuinfer/gguf_parser.h), for hosts that bind C.
 * The file is memory-mapped; names and strings returned stay valid until
 * cri_gguf_close.  A tensor's data lying past the end of the file is rejected at
 * open (CRI_ERR_FILE). */
typedef struct cri_gguf cri_gguf;
typedef struct cri_gguf_tensor {
    const char* name;
    int ggml_type;         /* GGML type tag (0 F32, 1 F16, 2 Q4_0, 6 Q5_0, 8 Q8_0, 12 Q4_K, 14 Q6_K, ...) */
    int format;            /* cri_format of the data, CRI_FP32, or -1 for types the matmuls do not take */
    int n_dims;
    long long dims[8];     /* dims[0] innermost: a [N, K] weight is {K, N} */
    long long n_elements;
    long long byte_size;   /* -1 for a GGML type this reader does not know */
    long long data_offset; /* bytes from the start of the file */
} cri_gguf_tensor;
typedef struct cri_gguf_model {
    char architecture[64]; /* general.architecture */
    unsigned context_length, embedding_length, block_count, head_count, head_count_kv, feed_forward_length,
        rope_dimension_count, vocab_size; /* bit i of `missing` set: field i (in this order) absent */
    float rope_freq_base;  /* default 10000 */
    float rms_norm_eps;    /* default 1e-5 */
    int tie_word_embeddings; /* 1 when there is no output.weight */
    unsigned missing;
} cri_gguf_model;
/* replaces cuinfer::GGUFParser::GGUFParser, ref:include/cuinfer/gguf_parser.h:165 */
int cri_gguf_open(const char* path, cri_gguf** out);
void cri_gguf_close(cri_gguf* file);
int cri_gguf_version(const cri_gguf* file);
long long cri_gguf_tensor_count(const cri_gguf* file);
long long cri_gguf_metadata_count(const cri_gguf* file);
/* index of the named tensor, or -1 (find_tensor, ref:include/cuinfer/gguf_parser.h:236) */
int cri_gguf_find_tensor(const cri_gguf* file, const char* name);
int cri_gguf_tensor_info(const cri_gguf* file, int index, cri_gguf_tensor* out);
/* host pointer into the mapping (tensor_data, ref:include/cuinfer/gguf_parser.h:240) */
const void* cri_gguf_tensor_data(const cri_gguf* file, int index);
/* GGUF value type tag of a metadata key, or -1 */
int cri_gguf_metadata_type(const cri_gguf* file, const char* key);
/* typed getters: CRI_ERR_SHAPE for a missing key or another type (get_*, ref:include/cuinfer/gguf_parser.h:197-201) */
int cri_gguf_get_u32(const cri_gguf* file, const char* key, unsigned* out);
int cri_gguf_get_i32(const cri_gguf* file, const char* key, int* out);
int cri_gguf_get_u64(const cri_gguf* file, const char* key, unsigned long long* out);
int cri_gguf_get_f32(const cri_gguf* file, const char* key, float* out);
int cri_gguf_get_string(const cri_gguf* file, const char* key, const char** out);
long long cri_gguf_get_array_length(const cri_gguf* file, const char* key);
/* the model helpers, ref:include/cuinfer/gguf_parser.h:208-230 */
int cri_gguf_model_params(const cri_gguf* file, cri_gguf_model* out);
/* the tensor's raw bytes to device memory; returns when the copy is done
 * (the upload of load_weight_quantized, ref:src/model.cu:406-411) */
int cri_gguf_upload(const cri_gguf* file, int index, void* device_dst, long long dst_bytes, hipStream_t stream);

/* out[i, :] = dequant(row ids[i] of table [vocab, dim]) in fp32, bit-identical to
 * dequantize + gather; ids outside [0, vocab) give zero rows.  format: a
 * cri_format or CRI_FP32.  Lets the token embedding stay in its file format
 * when the LM head reuses it (the reference dequantizes the tied table to
 * FP32, ref:src/model.cu:603); no counterpart in the reference. */
int cri_embedding_rows(int format, const void* table, const int* ids, float* out, int n_ids, int dim, int vocab,
                       hipStream_t stream);

/* ---- the decode step: TransformerModel::forward's layer loop ---------------
 * A decoder owns its weights (copied in), activation buffers, KV cache
 * [n_layers][max_seq_len, n_kv_heads, head_dim] and workspace, all allocated at
 * create; forward and replay allocate nothing.  The C++ class is
 * cuinfer::DecodeStep (cuinfer/decode_step.h).  It replaces the quantized path
 * of TransformerModel::forward, ref:src/model.cu:831-1039 (embedding, per layer
 * RMSNorm, q/k/v, RoPE, KV append, attention, o, residual + RMSNorm, gate/up,
 * SiLU * up, down, residual; final RMSNorm, LM head) and the greedy
 * argmax_sample, ref:src/embedding.cu:305-326.  Batch row m of a call at
 * position p attends to cache positions [0, p + m] (the reference's causal
 * mask; one token: its fused decode attention).  The position is kept in
 * device memory, so a captured step replays correctly token after token. */
typedef struct cri_decoder cri_decoder;
typedef struct cri_decoder_config {
    int n_layers, dim, n_heads, n_kv_heads, head_dim, ffn_dim, vocab_size, max_seq_len;
    int max_batch; /* tokens per call, 1..65535 (up to 16 use the fused norm prologues) */
    float rms_norm_eps, rope_theta;
} cri_decoder_config;
/* one layer's tensors; weights [N, K] in GGUF row order, in host or device memory
 * (copied at set time); norms fp32 [dim]; formats: cri_format, not CRI_FP32 */
typedef struct cri_decoder_layer {
    const float* attn_norm;
    const float* ffn_norm;
    int q_format, k_format, v_format, o_format, gate_format, up_format, down_format;
    const void *q, *k, *v, *o, *gate, *up, *down;
} cri_decoder_layer;
int cri_decoder_create(const cri_decoder_config* config, cri_decoder** out);
void cri_decoder_destroy(cri_decoder* dec);
int cri_decoder_set_layer(cri_decoder* dec, int layer, const cri_decoder_layer* weights);
/* token table [vocab, dim]: a cri_format or CRI_FP32 */
int cri_decoder_set_embedding(cri_decoder* dec, int format, const void* table);
/* final norm fp32 [dim] and LM head [vocab, dim]; format -1 ties the head to the token table */
int cri_decoder_set_output(cri_decoder* dec, const float* output_norm, int format, const void* lm_head);
/* M tokens (device int32 [M]) at positions position() .. +M-1 -> logits (device fp32 [M, vocab]);
 * next_ids (device int32 [M] or NULL) <- argmax of each logits row (ties: the smallest index).
 * CRI_ERR_SHAPE when position() + M would exceed max_seq_len. */
int cri_decoder_forward(cri_decoder* dec, const int* token_ids, int M, float* logits, int* next_ids,
                        hipStream_t stream);
/* A prompt as the reference's generate() consumes it (ref:src/model.cu:1063-1078, which runs
 * forward() and reads only the last row's logits): every layer runs on the M tokens (caches
 * appended, position advanced by M), the final RMSNorm, LM head and argmax for token M - 1 only:
 * logits (device fp32 [vocab]), next_id (device int32 [1] or NULL).  No counterpart in the
 * reference's API (its forward() always returns every row). */
int cri_decoder_prefill(cri_decoder* dec, const int* token_ids, int M, float* logits, int* next_id,
                        hipStream_t stream);
/* capture the same call as one HIP graph on a non-null stream (nothing runs), and replay it:
 * each replay is one more step of M tokens; next_ids == token_ids generates greedily */
/* cri_decoder_forward that also writes the residual stream entering each layer and the final
 * norm: hidden_taps (device fp32 [n_layers + 1, M, dim]) slice i = the hidden state layer i
 * reads (slice n_layers: the final RMSNorm's input).  Same kernels as cri_decoder_forward plus
 * one small kernel per slice; for checking a step layer by layer.  Has no counterpart in the
 * reference (its forward keeps no per-layer state). */
int cri_decoder_forward_taps(cri_decoder* dec, const int* token_ids, int M, float* logits, int* next_ids,
                             float* hidden_taps, hipStream_t stream);
/* any cri_decoder_set_* call discards a captured graph (replay then fails until the next capture) */
int cri_decoder_capture(cri_decoder* dec, const int* token_ids, int M, float* logits, int* next_ids,
                        hipStream_t stream);
int cri_decoder_replay(cri_decoder* dec, hipStream_t stream);
/* the sequence position (0 = empty cache); set with a kernel on `stream` */
int cri_decoder_set_position(cri_decoder* dec, int pos, hipStream_t stream);
int cri_decoder_position(const cri_decoder* dec);
/* the layer's K and V cache, [max_seq_len, n_kv_heads, head_dim] fp32 device memory */
int cri_decoder_kv_cache(cri_decoder* dec, int layer, float** k_cache, float** v_cache);
long long cri_decoder_weight_bytes(const cri_decoder* dec);
/* weight bytes one step of M tokens reads: every layer's matrices and norms, the final norm and
 * LM head, and M token-table rows (the whole table when the head is tied to it) */
long long cri_decoder_step_weight_bytes(const cri_decoder* dec, int M);

/* ---- diagnostics ---------------------------------------------------------- */

/* Reads n_bytes (a multiple of 16) at src (16-byte aligned) once with 16-byte
 * loads and nothing else: the achievable streaming-read bandwidth that the
 * GEMV rooflines are read against.  sink (one device word) is written only if
 * the XOR of the words one thread reads (four 16-byte chunks, 4096 bytes apart)
 * equals 0x9E3779B9.  A measurement aid with no counterpart in the reference. */
int cri_stream_read(const void* src, long long n_bytes, unsigned* sink, hipStream_t stream);

/* cri_stream_read with the launch shape as parameters, for sweeping it:
 * loads_per_thread (1, 2, 4, 8 or 16) 16-byte loads in flight per thread;
 * grid_blocks 0 covers the buffer once with one pass per thread, otherwise
 * that many workgroups of 256 threads stride over it.  cri_stream_read is
 * (4, 0).  A measurement aid with no counterpart in the reference. */
int cri_stream_read_ex(const void* src, long long n_bytes, unsigned* sink, int loads_per_thread, int grid_blocks,
                       hipStream_t stream);

/* Writes the GPU's constant 100 MHz clock (wall_clock64) to *dst (device, 8-byte
 * aligned) from a one-wave kernel on `stream`: timestamps between the kernels of
 * a captured graph, where events cannot be recorded.  A measurement aid with no
 * counterpart in the reference. */
int cri_timestamp(unsigned long long* dst, hipStream_t stream);

/* Message for the last non-zero status returned on this thread ("" if none). */
const char* cri_last_error_string(void);
/* Bytes per block / elements per block of a format (0 if unknown). */
int cri_block_bytes(int format);
int cri_block_elems(int format);
/* Library ABI version (major * 10000 + minor * 100 + patch). */
int cri_version(void);

#ifdef __cplusplus
}
#endif
#endif /* CRI_H */

// internal.hpp -- launchers shared between the kernel translation units and
// the C ABI (abi.cpp).  Launchers assume the ABI has validated every shape,
// pointer and alignment requirement; they only enqueue kernels.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

namespace cri {

// Format ids; identical to cri_format in include/cri.h, plus fp32 weights for
// the transposed-B GEMV.
enum : int { kFmtQ8_0 = 0, kFmtQ4_0 = 1, kFmtQ5_0 = 2, kFmtQ4_K = 3, kFmtQ6_K = 4, kFmtF16 = 5, kFmtF32 = 6 };

inline int block_elems(int fmt) {
    switch (fmt) {
        case kFmtQ8_0: case kFmtQ4_0: case kFmtQ5_0: return 32;
        case kFmtQ4_K: case kFmtQ6_K: return 256;
        case kFmtF16: case kFmtF32: return 1;
    }
    return 0;
}
inline int block_bytes(int fmt) {
    switch (fmt) {
        case kFmtQ8_0: return 34;
        case kFmtQ4_0: return 18;
        case kFmtQ5_0: return 22;
        case kFmtQ4_K: return 144;
        case kFmtQ6_K: return 210;
        case kFmtF16: return 2;
        case kFmtF32: return 4;
    }
    return 0;
}
inline long row_bytes(int fmt, int K) { return static_cast<long>(K / block_elems(fmt)) * block_bytes(fmt); }

// Activation prologue of the fused decode matmuls: the A operand is computed
// from its neighbours' outputs while it is staged, instead of by separate
// elementwise launches (ref:src/model.cu:960-1010 runs rmsnorm_residual, silu
// and multiply between the GEMVs).
//   kActPlain   : x[m][k] = a[m*lda + k]
//   kActSwiGLU  : x[m][k] = silu(a[m*lda + k]) * b[m*lda + k]            (gate, up)
//   kActRMSNorm : v = a[m*lda + k] + b[m*lda + k] (b may be null), x = v * w[k],
//                 the output row m scaled by 1/sqrt(mean_k v^2 + eps), and v
//                 written to h_out[m*K + k] when h_out is not null
//   kActSwiGLU2 : SwiGLU of gate/up outputs left as the two partial sums of an
//                 RMSNorm matmul whose K was split over workgroups (SplitSums):
//                 g = f_m (a[off] + a[off + split]), u likewise from b, with
//                 f_m = 1/sqrt((w[m] + w[16 + m] + ... nss terms) / kn + eps) (w: the
//                 splits' sums of squares; w null: f_m = 1, a plain gate/up), then silu(g) * u;
//                 split = 0: one partial sum (g = f_m a[off])
//   kActRMSNormS: kActRMSNorm with the residual left as kn (<= 4) partial sums of a K
//                 split: r = b[off] + b[off + split] + ... in split order (the batch-1 GEMV)
enum : int { kActPlain = 0, kActSwiGLU = 1, kActRMSNorm = 2, kActSwiGLU2 = 3, kActRMSNormS = 4 };
constexpr int kResMaxSplits = 4;
struct ActIn {
    const float* a;
    const float* b;
    const float* w;
    float* h_out;
    long lda;
    float eps;
    long split = 0;  // kActSwiGLU2, kActRMSNormS: floats between consecutive partial sums
    int kn = 0;      // kActSwiGLU2: K of the RMSNorm; kActRMSNormS: number of partial sums
    int nss = 2;     // kActSwiGLU2: sums of squares added for the row factor (w[16 s + m], s < nss <= 4)
};

// The q/k/v projection's outputs at one decode position, rotated and appended in the GEMV's
// epilogue: columns [0, qd) are q (rotated, to the output), [qd, qd + kvd) k (rotated, to
// kc + pos kvd) and [qd + kvd, qd + 2 kvd) v (to vc + pos kvd); pos = *pos_dev; rot: the
// [max_seq, half] table of (cos, sin) pairs of the RoPE kernel (half = head_dim / 2).
struct RopeOut {
    const int* pos = nullptr;
    const float* rot = nullptr;
    float* kc = nullptr;
    float* vc = nullptr;
    int qd = 0, kvd = 0, half = 0;
};

// A decode-batch matmul whose K split over workgroups is left unreduced for its consumer:
// C[m][n] = (part[m N + n] + part[stride + m N + n] + ... in split order) * f_m, with
// f_m = 1/sqrt(sum over splits of ssq[s * 16 + m] / K + eps) when ssq is not null (RMSNorm),
// else 1.  S = 0: C itself was written.
struct SplitSums {
    const float* part = nullptr;
    const float* ssq = nullptr;
    long stride = 0;
    int S = 0, N = 0, K = 0;
    float eps = 0.0f;
    int nss = 0;  // sums of squares added for the row factor (0: S of them)
};

namespace detail {

// Launcher status: 0 = enqueued; kDeclined = this kernel does not take the shape
// (the caller may try another); kFailed = the HIP runtime refused a set-up call
// or the launch (the caller reports CRI_ERR_LAUNCH and tries nothing else).
constexpr int kDeclined = -1;
constexpr int kFailed = -4;

// Target number of resident waves for the GEMV grid (MI355X: 256 CUs).
constexpr long kGemvTargetWaves = 2048;

// batch-1 GEMV (gemv.hip); the _act form takes an activation prologue
bool gemv_supported(int fmt, int K, const void* W);
int launch_gemv(int fmt, const float* x, const void* W, float* y, int N, int K, hipStream_t stream);
int launch_gemv2(int fmt, const float* x, const void* W, float* y, int M, int N, int K, hipStream_t stream);
int launch_gemv_act(int mode, int fmt, const ActIn& act, const void* W, float* y, int N, int K, hipStream_t stream);
// batch-1 GEMV with K split into `splits` parts (grid.y), part s written to y + s N (partial
// sums for a kActRMSNormS consumer); plain or SwiGLU prologue, K / splits a multiple of 256
int launch_gemv_ksplit(int mode, int fmt, const ActIn& act, const void* W, float* y, int N, int K, int splits,
                       hipStream_t stream);
// the RMSNorm-prologue GEMV of a fused q/k/v projection with RoPE and the cache append in its
// epilogue (RopeOut); kDeclined when the layout does not put each rotated pair in one wave
// (split_res: the residual arrives as partial sums, kActRMSNormS)
int launch_gemv_rope(int fmt, const ActIn& act, const void* W, float* q_out, int N, int K, const RopeOut& rope,
                     hipStream_t stream, bool split_res = false);

// batch-1 GEMV with K sliced over the waves of a workgroup (gemv_slice.hip; Q4_K: two waves up to
// 2048 x 2048, four above), for K in
// {1024, 2048, 4096, 8192} and dword-aligned weights; plain or SwiGLU prologue (kDeclined otherwise)
bool slice_gemv_supported(int fmt, int N, int K, const void* W);
int launch_slice_gemv(int mode, int fmt, const ActIn& act, const void* W, float* y, int N, int K, hipStream_t stream);

// 1 <= M <= 16 fused dequant matmul on the matrix cores (mfma_skinny.hip)
bool skinny_supported(int fmt, int M, int K, const void* B);
int launch_skinny(int fmt, const float* A, const void* B, float* C, int M, int N, int K, hipStream_t stream);
// ws (optional, skinny_workspace_floats(M, N) floats, 16-byte aligned): the partial sums of a K
// split over workgroups are stored there and a second launch adds them in a fixed order
// (deterministic; the RMSNorm prologue splits too).  Without it a split (plain and SwiGLU
// prologues, several activation chunks) adds into C with fp32 atomics.  Calls sharing one
// workspace must be ordered on one stream.
// defer (with ws): when the launch splits K into defer_S partial sums (any count for defer_S
// = 0), the reduction is not launched and *defer describes the partial sums; otherwise
// defer->S = 0 and C holds the result.
int launch_skinny_act(int mode, int fmt, const ActIn& act, const void* B, float* C, int M, int N, int K,
                      hipStream_t stream, float* ws = nullptr, long ws_floats = 0, SplitSums* defer = nullptr,
                      int defer_S = 0);
long skinny_workspace_floats(int M, int N);
// whether launch_skinny_act without a workspace splits K over workgroups with fp32 atomics (plain
// activations, M rows); with a workspace those partial sums are added in a fixed order instead
bool skinny_atomic_split(int M, int K);
// cri_matmul / cri_matmul_swiglu / cri_matmul_rmsnorm with that workspace (abi.cpp); return a cri_status
int matmul_split_ws(int fmt, const float* A, const void* B, float* C, int M, int N, int K, float* ws, long ws_floats,
                    hipStream_t s, SplitSums* defer = nullptr, int defer_S = 0);
int matmul_rmsnorm_split_ws(int fmt, const float* hidden, const float* residual, const float* norm_weight,
                            float* hidden_out, const void* B, float* C, int M, int N, int K, float eps, float* ws,
                            long ws_floats, hipStream_t s, SplitSums* defer = nullptr, int defer_S = 0);
// RMSNorm(hidden + residual) times B for one token, the residual given as `splits` partial sums
// `split` floats apart (kActRMSNormS); hidden_out as in cri_matmul_rmsnorm
int matmul_rmsnorm_splitres(int fmt, const float* hidden, const float* res_parts, int splits, long split,
                            const float* norm_weight, float* hidden_out, const void* B, float* C, int N, int K,
                            float eps, hipStream_t s);
// the SwiGLU matmul of gate/up outputs left as two partial sums (kActSwiGLU2; gu.S = 1: one,
// the whole product without its row factor): gate at gu.part, up at gu.part + up_off, the row
// factor from gu.ssq (null: none)
int matmul_swiglu2_split_ws(int fmt, const SplitSums& gu, long up_off, int ld, const void* B, float* C, int M, int N,
                            int K, float* ws, long ws_floats, hipStream_t s, SplitSums* defer = nullptr,
                            int defer_S = 0);
int matmul_swiglu_split_ws(int fmt, const float* gate, const float* up, int ld, const void* B, float* C, int M, int N,
                           int K, float* ws, long ws_floats, hipStream_t s, SplitSums* defer = nullptr,
                           int defer_S = 0);

// multi-token fused dequant GEMM on the matrix cores, fp16 operands (mfma_gemm.hip)
bool mfma_gemm_supported(int fmt, int M, int N, int K, const void* A, const void* B);
int launch_mfma_gemm(int fmt, const float* A, const void* B, float* C, int M, int N, int K, hipStream_t stream);

// multi-token GEMM with weights decoded straight into MFMA operands, Q4_K, Q6_K and Q8_0 (prefill.hip)
bool prefill_supported(int fmt, int M, int N, int K, const void* A, const void* B);
// A K split over workgroups (few tiles) adds into a zero-filled C with fp32 atomics, or, given a
// workspace of at least kPrefillSplitFloats floats (16-byte aligned, N % 4 == 0), stores its
// partial sums there: left for the consumer with defer (defer->S > 0; defer_S: the count it
// takes, 0 any), else added up into C (16-byte aligned) in split order by a second launch.
int launch_prefill(int fmt, const float* A, const void* B, float* C, int M, int N, int K, hipStream_t stream,
                   float* ws = nullptr, long ws_floats = 0, SplitSums* defer = nullptr, int defer_S = 0);
// K splits of the prefill GEMM are chosen so that tiles x splits < 512; so at most this many
// partial-sum floats (512 tiles of 64 x 256); splits past 16 take the atomics
constexpr long kPrefillSplitFloats = 512L * 64 * 256;
// C[M, F] = SiLU(A gate^T) * (A up^T) for a stacked gate/up matrix B of 2F rows (gate first), the
// product and the elementwise step in one launch (the SiLU * up of the separate kernel, bit for
// bit); kDeclined where the tiles would need a K split (short prompts) or the kernel does not apply
int launch_prefill_swiglu(int fmt, const float* A, const void* B, float* C, int M, int F, int K, hipStream_t stream);
// floats of partial sums launch_prefill stores in a workspace for this shape (0: no K split)
long prefill_workspace_floats(int M, int N, int K);
// C = the S partial sums of p added in split order (times p's RMSNorm row factor); M N % 4 == 0,
// C and p.part 16-byte aligned, p.stride % 4 == 0 (mfma_skinny.hip)
int launch_split_reduce(const SplitSums& p, float* C, int M, hipStream_t stream);

// any-M fused dequant matmul, element-wise decode (generic.hip)
int launch_generic_matmul(int fmt, const float* A, const void* B, float* C, int M, int N, int K,
                          hipStream_t stream);
int launch_generic_matmul_act(int mode, int fmt, const ActIn& act, const void* B, float* C, int M, int N, int K,
                              hipStream_t stream);

// standalone neighbours (elementwise.hip): the reference's rmsnorm_residual and silu + multiply
int launch_rmsnorm_residual(const float* input, const float* residual, const float* weight, float* output,
                            float* normed, int rows, int n, float eps, hipStream_t stream);
int launch_silu_mul(const float* gate, const float* up, float* out, long n, hipStream_t stream);
// rmsnorm_residual with the residual as the partial sums of a split decode-batch matmul
// (r.S = 0: none); rows of up to 4096 floats, 16-byte aligned (else kDeclined).  row_ss (not
// null): normed = (h + r) * weight without the row factor, and each row is cut into
// kNormParts column ranges whose sums of squares go to row_ss[16 part + row] (the layout of
// SplitSums.ssq; the consumer adds kNormParts of them), n % (4 kNormParts) == 0
constexpr int kNormParts = 4;
int launch_split_norm(const float* h, const SplitSums& r, const float* weight, float* output, float* normed, int rows,
                      int n, float eps, hipStream_t stream, float* row_ss = nullptr);
// token rows of a (quantized) embedding table, dequantized (elementwise.hip)
int launch_stream_read(const void* src, long n_bytes, uint32_t* sink, hipStream_t stream);
// the device's 100 MHz wall clock written to *dst (probe.hip)
int launch_timestamp(unsigned long long* dst, hipStream_t stream);
// per 16-byte loads per thread in flight (1, 2, 4, 8, 16); grid_blocks 0: one pass of a grid
// covering the buffer, else that many blocks of 256 threads striding over it
int launch_stream_read_ex(const void* src, long n_bytes, uint32_t* sink, int per, long grid_blocks,
                          hipStream_t stream);
int launch_embedding_rows(int fmt, const void* table, const int* ids, float* out, int n_ids, int dim, int vocab,
                          hipStream_t stream);

// standalone dequant (dequant.hip)
int launch_dequant(int fmt, const void* src, float* dst, long n_blocks, hipStream_t stream);

// C[0..n) = 0 with a kernel (no hipMemsetAsync, so the call can be captured in a graph)
void launch_fill_zero(float* C, long n, hipStream_t stream);

// fp32 neighbours (fp32ops.hip)
int launch_transposed_b(const float* A, const float* B, float* C, int M, int N, int K, hipStream_t stream);
int launch_gqa(const float* A, const float* B, float* C, int n_heads, int n_kv_heads, int M, int N, int K,
               hipStream_t stream);

// fused decode attention over the [kv_len, n_kv_heads, head_dim] cache (attention.hip)
constexpr int kDecodeAttnMaxHeadDim = 256;
int launch_decode_attention(const float* Q, const float* K, const float* V, float* out, int n_heads, int n_kv_heads,
                            int head_dim, int kv_len, float scale, hipStream_t stream);
// split over positions with partial results in a caller workspace (head_dim <= 128, 4 | head_dim,
// 16-byte aligned Q/K/V); returns -2 when the workspace cannot hold one record per head
constexpr int kDecodeAttnSplitMaxHeadDim = 128;
bool decode_attention_split_supported(const float* Q, const float* K, const float* V, int head_dim);
long decode_attention_workspace_bytes(int n_heads, int n_kv_heads, int head_dim, int kv_len);
int launch_decode_attention_split(const float* Q, const float* K, const float* V, float* out, int n_heads,
                                  int n_kv_heads, int head_dim, int kv_len, float scale, float* ws, long ws_bytes,
                                  hipStream_t stream);
// the split form for `rows` consecutive query tokens (row m at Q + m*ldq, output at out + m*ldo):
// row m attends to the first kv0 + m positions (+ *kv_dev when kv_dev is not null);
// nchunks chunks per row (decode_attention_rows_chunks gives the count suited to `rows` rows at
// max_kv_len: ~256 workgroups per row for one row; for the multi-row form one 32-position tile
// per wave of a four-wave workgroup, up to 16 chunks); ws holds rows * n_heads * nchunks records
// of head_dim + 4 floats
int decode_attention_rows_chunks(int n_heads, int n_kv_heads, int head_dim, int max_kv_len, int rows);
// true where `rows` query rows take the multi-row (matrix-core) kernel
bool decode_attention_rows_mrow(int rows, int head_dim);
int launch_decode_attention_rows(const float* Q, long ldq, const float* K, const float* V, float* out, long ldo,
                                 int rows, int n_heads, int n_kv_heads, int head_dim, const int* kv_dev, int kv0,
                                 int nchunks, float scale, float* ws, hipStream_t stream);

// cri_fused_decode_attention_noalloc: its records live in a file-scope device array of this
// many bytes (attention.hip); noalloc_scratch gives the current device's address of it
constexpr long kNoallocScratchBytes = 1L << 20;
int noalloc_scratch(float** out);

// decode step neighbours (step_kernels.hip)
// RoPE of the rows' q and k at positions *pos + m (ref:src/kernels/elementwise.cu:232-266),
// q rotated in place, rotated k and v written to the caches' rows *pos + m
// (KVCache::append, ref:src/kv_cache.cu:157-211); caches [max_seq, n_kv_heads, head_dim];
// rot: the (cos, sin) table [max_seq, head_dim / 2] of fp32 pairs
// qkv (optional, S > 0): the q/k/v projection left as partial sums; q, k and v are then its
// columns [0, ..), [kcol, ..) and [vcol, ..), reduced here, and q is written to q (row m at
// q + m*ldq) rotated
int launch_rope_append(float* q, long ldq, const float* k, long ldk, const float* v, long ldv, int rows, int n_heads,
                       int n_kv_heads, int head_dim, const float* rot, const int* pos, float* k_cache, float* v_cache,
                       hipStream_t stream, const SplitSums* qkv = nullptr, int kcol = 0, int vcol = 0);
// out[m] = index of the largest logits[m][i], the smallest index among equal maxima, NaN ignored
// (kernel_argmax, ref:src/embedding.cu:155-200); rows are cut into argmax_slices(n) slices whose
// (value, index) go to part (2 floats each, rows * slices); counters: rows zeroed words (re-zeroed
// by the kernel); *pos += pos_add at the end when pos is not null
int argmax_slices(int n);
int launch_argmax_rows(const float* logits, long ld, int rows, int n, int* out, float* part, unsigned* counters,
                       int* pos, int pos_add, hipStream_t stream);
// *pos += delta / *pos = value
int launch_pos_add(int* pos, int delta, hipStream_t stream);
int launch_pos_set(int* pos, int value, hipStream_t stream);
// Prompt attention over the [T, Hkv, D] caches through batched_matmul_gqa, as the reference's
// prefill (ref:src/attention.cu:809-871): q rows [M][ldq] -> ctx rows [M][H D] for the batch rows
// m0 .. m0 + M - 1 of a step at position *pos (row m0 + m sees cache positions <= *pos + m0 + m).
// Workspaces: qh and oh H M D floats, kt and vh Hkv D T4, sc H M T4 (T4 % 4 == 0, T4 >= *pos + m0 +
// M when it runs; cache rows past that are not read into the products).  kDeclined for an
// unsupported shape.
int launch_prefill_attention(const float* q, long ldq, const float* kc, const float* vc, float* ctx, int m0, int M,
                             int H, int Hkv, int D, int T4, const int* pos, float scale, float* qh, float* kt,
                             float* vh, float* sc, float* oh, hipStream_t stream);
// rows per launch_prefill_attention call of the C ABI and the decode step (the scores workspace
// holds n_heads x this many rows x the cache length)
constexpr int kPromptRows = 512;
// out[rows, n] = h + the pending residual r (r.S partial sums r.stride floats apart, rows r.N
// floats apart, added in split order; r.S = 0: none): a step's layer taps
int launch_hidden_tap(const float* h, const SplitSums& r, float* out, int rows, int n, hipStream_t stream);

}  // namespace detail
}  // namespace cri

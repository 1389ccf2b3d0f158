/*
 * oracle.h -- CPU restatement of CRETIF's fused dequant+matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (cretif_amd/, include/)
 * may link, import or call this code.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg use it, and only as the checker or as the
 * timed CPU baseline.
 *
 * Every function names the reference file:line whose arithmetic it restates
 * (paths relative to the reference repository root).  Arithmetic is plain
 * IEEE binary32 compiled with -O2 -ffp-contract=off, matching the reference
 * host build (ISO C++17, no contraction).
 *
 * Parity pinning (each function is checked by tests/test_oracle_*.py):
 *   orc_half_to_float / orc_float_to_half : exhaustive vs numpy float16.
 *   orc_dequantize_*    : reference KATs (SingleBlock, all-0x88), the loop-form
 *                         CPU references of tests/test_dequantize.cu restated
 *                         independently in numpy, quantize->dequantize round
 *                         trips bounded by half a quantization step, and all
 *                         2^k codes per field.
 *   orc_matmul_*        : fp64 brute force with an error bound, exact-integer
 *                         KATs (every partial sum exact), linearity, one-hot.
 *   orc_decode_attention*: the two reference formulations against each other,
 *                         an fp64 brute force with an error bound, and closed
 *                         forms (kv_len 1 -> V[0]; equal scores -> mean of V;
 *                         one dominant score -> its V row; a position
 *                         permutation leaves the output unchanged).
 *   orc_rmsnorm_residual, orc_silu_mul: fp64 numpy, closed forms (a constant
 *                         row normalises to c / sqrt(c^2 + eps); silu(0) = 0,
 *                         silu(x) -> x and -> 0 at the ends), the residual sum
 *                         exact, scale invariance of the normed row.
 *   orc_rope            : pos 0 is the identity (bit-exact), each pair keeps its
 *                         norm, pair 0 turns by exactly pos radians, a turn by
 *                         p then q equals a turn by p + q (fp64 numpy), and the
 *                         whole map against an fp64 numpy rotation.
 *   orc_argmax          : numpy argmax on rows without NaN, ties to the first
 *                         index, NaN skipped, all -inf / NaN -> 0.
 *   orc_quantize_*      : bit-exact vs the numpy quantizers in cretif_amd/quant.py
 *                         (written separately) and round-trip error bounds.
 */
#ifndef CRETIF_ORACLE_H
#define CRETIF_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* format ids (same numbering as cri_format in include/cri.h) */
enum { ORC_Q8_0 = 0, ORC_Q4_0 = 1, ORC_Q5_0 = 2, ORC_Q4_K = 3, ORC_Q6_K = 4, ORC_FP16 = 5 };

int      orc_block_elems(int fmt);
int      orc_block_bytes(int fmt);

float    orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f);
void     orc_half_to_float_array(const uint16_t* src, float* dst, int64_t n);
void     orc_float_to_half_array(const float* src, uint16_t* dst, int64_t n);

/* standalone dequant: index form of ref:src/kernels/dequantize.cu */
void orc_dequantize_q8_0(const void* src, float* dst, int64_t n_blocks);
void orc_dequantize_q4_0(const void* src, float* dst, int64_t n_blocks);
void orc_dequantize_q5_0(const void* src, float* dst, int64_t n_blocks);
void orc_dequantize_q6_k(const void* src, float* dst, int64_t n_blocks);
void orc_dequantize_q4_k(const void* src, float* dst, int64_t n_blocks);
void orc_dequantize_fp16(const void* src, float* dst, int64_t n_elems);
/* generic: fmt id, n_elems = n_blocks * block_elems */
void orc_dequantize(int fmt, const void* src, float* dst, int64_t n_elems);

/* C[M,N] = A[M,K] * B[N,K]^T, sequential fp32 (ref:tests/test_matmul_quant.cu:30-41) */
void orc_matmul_bt(const float* A, const float* B, float* C, int M, int N, int K);
/* dequant(B) then orc_matmul_bt, row by row; only rows [n0, n1) of C are written */
void orc_matmul_quant_rows(int fmt, const float* A, const void* Bq, float* C,
                           int M, int N, int K, int n0, int n1);
void orc_matmul_quant(int fmt, const float* A, const void* Bq, float* C, int M, int N, int K);
/* ref:tests/test_embedding.cu:98-109 */
void orc_matmul_transposed_b(const float* A, const float* B, float* C, int M, int N, int K);
/* ref:tests/test_attention.cu:76-85 (cpu_matmul) + :399-407 (GQA mapping) */
void orc_batched_matmul_gqa(const float* A, const float* B, float* C,
                            int n_heads, int n_kv_heads, int M, int N, int K);

/* one-token decode attention, cache layout [kv_len, n_kv_heads, head_dim]:
 * two-pass softmax of ref:tests/test_attention.cu:972-1008 (+ cpu_softmax :110-122) */
void orc_decode_attention(const float* Q, const float* Kc, const float* Vc, float* out,
                          int n_heads, int n_kv_heads, int head_dim, int kv_len, float scale);
/* the reference kernel's online recurrence, ref:src/attention.cu:446-493 */
void orc_decode_attention_online(const float* Q, const float* Kc, const float* Vc, float* out,
                                 int n_heads, int n_kv_heads, int head_dim, int kv_len, float scale);

/* the matmuls' elementwise neighbours: ref:src/kernels/elementwise.cu:463-504, :93-99 + :300-305 */
void orc_rmsnorm_residual(const float* input, const float* residual, const float* weight, float* output,
                          float* normed, int rows, int n, float eps);
void orc_silu_mul(const float* gate, const float* up, float* out, int64_t n);

/* RoPE of n_heads heads of one token in place, ref:src/kernels/elementwise.cu:232-257 */
void orc_rope(float* qk, int pos, int head_dim, int n_heads, float theta);
/* argmax with the reference kernel's tie and NaN rules, ref:src/embedding.cu:155-200 */
int32_t orc_argmax(const float* x, int n);

/* host quantizers restated from ref:tests/test_matmul_quant.cu */
void orc_quantize_q8_0(const float* x, void* dst, int64_t n);        /* :46-71   */
void orc_quantize_q4_0(const float* x, void* dst, int64_t n);        /* :74-102  */
void orc_quantize_q5_0(const float* x, void* dst, int64_t n);        /* :410-460 */
void orc_quantize_q6_k(const float* x, void* dst, int64_t n);        /* :611-686 */
void orc_quantize_q4_k_simple(const float* x, void* dst, int64_t n); /* :107-184 */
/* asymmetric Q4_K quantizer (own; nonzero dmin and mins, GGML packing) */
void orc_quantize_q4_k_asym(const float* x, void* dst, int64_t n);

/* deterministic block makers, ref:tests/test_dequantize.cu:135-208 */
void orc_make_q8_0_blocks(void* dst, int n_blocks);
void orc_make_q4_0_blocks(void* dst, int n_blocks);
void orc_make_q6_k_blocks(void* dst, int n_blocks);
void orc_make_q4_k_blocks(void* dst, int n_blocks);

/* LCG uniform[-1,1], ref:tests/test_matmul_quant.cu:187-195 */
void orc_random_matrix_lcg(float* dst, int64_t n, uint32_t seed);
/* own generator: splitmix64 + Box-Muller, N(0, sigma^2) */
void orc_randn(float* dst, int64_t n, uint64_t seed, float sigma);

#ifdef __cplusplus
}
#endif
#endif

/*
 * oracle.c -- CPU restatement of CRETIF's dequant + matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Compiled with
 *   gcc -O2 -std=c99 -ffp-contract=off -fPIC -shared
 * so every float expression is evaluated as written, one IEEE binary32
 * rounding per operation, like the reference's host-side CPU references.
 *
 * Block layouts (byte offsets; ref:include/cuinfer/quantization.h:38-126):
 *   Q8_0  34 B : f16 d @0, int8 qs[32] @2
 *   Q4_0  18 B : f16 d @0, u8 qs[16] @2
 *   Q5_0  22 B : f16 d @0, u8 qh[4] @2, u8 qs[16] @6
 *   Q6_K 210 B : u8 ql[128] @0, u8 qh[64] @128, int8 scales[16] @192, f16 d @208
 *   Q4_K 144 B : f16 d @0, f16 dmin @2, u8 scales[12] @4, u8 qs[128] @16
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

int orc_block_elems(int fmt) {
    switch (fmt) {
        case ORC_Q8_0: case ORC_Q4_0: case ORC_Q5_0: return 32;
        case ORC_Q4_K: case ORC_Q6_K: return 256;
        case ORC_FP16: return 1;
    }
    return 0;
}

int orc_block_bytes(int fmt) {
    switch (fmt) {
        case ORC_Q8_0: return 34;
        case ORC_Q4_0: return 18;
        case ORC_Q5_0: return 22;
        case ORC_Q4_K: return 144;
        case ORC_Q6_K: return 210;
        case ORC_FP16: return 2;
    }
    return 0;
}

/* ---------------------------------------------------------------------------
 * IEEE-754 binary16 <-> binary32, written from the format definition
 * (1 sign bit, 5 exponent bits with bias 15, 10 fraction bits).
 * ------------------------------------------------------------------------- */

static float bits_to_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t float_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float orc_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in binary32 */
        float v = ldexpf((float)m, -24);
        return sign ? -v : v;
    }
    if (e == 31) {
        /* inf (m == 0) or NaN (payload kept in the top fraction bits) */
        return bits_to_float(sign | 0x7F800000u | (m << 13));
    }
    return bits_to_float(sign | ((e - 15u + 127u) << 23) | (m << 13));
}

uint16_t orc_float_to_half(float f) {
    const uint32_t x = float_to_bits(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu)); /* NaN */
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {
        /* result is subnormal (or zero): round |f| * 2^24 to nearest, ties to even.
         * The scaling is exact (power of two) and |f| * 2^24 < 1024. */
        float scaled = ldexpf(bits_to_float(ax), 24);
        float r = rintf(scaled); /* default rounding mode: nearest-even */
        return (uint16_t)(sign | (uint16_t)r);
    }
    /* normal: rebias the exponent, round the 23-bit fraction to 10 bits (RNE) */
    uint32_t e = ((ax >> 23) - 127u + 15u);
    uint32_t m = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* carry may bump the exponent */
    return (uint16_t)(sign | h);
}

void orc_half_to_float_array(const uint16_t* src, float* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_half_to_float(src[i]);
}

void orc_float_to_half_array(const float* src, uint16_t* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_float_to_half(src[i]);
}

static float rd_half(const uint8_t* p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return orc_half_to_float(h);
}

static void wr_half(uint8_t* p, float f) {
    uint16_t h = orc_float_to_half(f);
    memcpy(p, &h, 2);
}

/* ---------------------------------------------------------------------------
 * Standalone dequant, per-element index form.
 * ------------------------------------------------------------------------- */

/* ref:src/kernels/dequantize.cu:34-48 */
void orc_dequantize_q8_0(const void* src, float* dst, int64_t n_blocks) {
    const uint8_t* s = (const uint8_t*)src;
    for (int64_t b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = s + b * 34;
        const float scale = rd_half(blk);
        for (int i = 0; i < 32; ++i) {
            const int8_t q = (int8_t)blk[2 + i];
            dst[b * 32 + i] = scale * (float)q;
        }
    }
}

/* ref:src/kernels/dequantize.cu:73-101 -- element i <- qs[i/2], low nibble if i even */
void orc_dequantize_q4_0(const void* src, float* dst, int64_t n_blocks) {
    const uint8_t* s = (const uint8_t*)src;
    for (int64_t b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = s + b * 18;
        const float scale = rd_half(blk);
        for (int i = 0; i < 32; ++i) {
            const uint8_t packed = blk[2 + i / 2];
            const int nib = (i % 2 == 0) ? (packed & 0x0F) : (packed >> 4);
            dst[b * 32 + i] = scale * (float)(nib - 8);
        }
    }
}

/* ref:src/kernels/dequantize.cu:126-165 */
void orc_dequantize_q5_0(const void* src, float* dst, int64_t n_blocks) {
    const uint8_t* s = (const uint8_t*)src;
    for (int64_t b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = s + b * 22;
        const float scale = rd_half(blk);
        const uint8_t* qh = blk + 2;
        const uint8_t* qs = blk + 6;
        const uint32_t qh32 = (uint32_t)qh[0] | ((uint32_t)qh[1] << 8) |
                              ((uint32_t)qh[2] << 16) | ((uint32_t)qh[3] << 24);
        for (int i = 0; i < 32; ++i) {
            const int half = i / 16, j = i % 16;
            const int low4 = half == 0 ? (qs[j] & 0x0F) : (qs[j] >> 4);
            const int hb = (int)((qh32 >> i) & 1u);
            const int q5 = low4 | (hb << 4);
            dst[b * 32 + i] = scale * (float)(q5 - 16);
        }
    }
}

/* ref:src/kernels/dequantize.cu:204-244 */
void orc_dequantize_q6_k(const void* src, float* dst, int64_t n_blocks) {
    const uint8_t* s = (const uint8_t*)src;
    for (int64_t b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = s + b * 210;
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const int8_t* sc = (const int8_t*)(blk + 192);
        const float d = rd_half(blk + 208);
        for (int e = 0; e < 256; ++e) {
            const int chunk = e / 128, within = e % 128;
            const int quarter = within / 32, l = within % 32;
            const int scale_idx = chunk * 8 + quarter * 2 + l / 16;
            const float scf = (float)sc[scale_idx];
            const int ql_off = (quarter & 1) * 32 + l + chunk * 64;
            const int qln = quarter < 2 ? (ql[ql_off] & 0x0F) : (ql[ql_off] >> 4);
            const int qhb = (qh[l + chunk * 32] >> (quarter * 2)) & 0x03;
            const int q6 = (qln | (qhb << 4)) - 32;
            dst[b * 256 + e] = d * scf * (float)q6;
        }
    }
}

/* ref:src/kernels/dequantize.cu:298-305, the GGML get_scale_min_k4 packing */
static void q4k_scale_min(const uint8_t* scales, int j, int* sc, int* mn) {
    if (j < 4) {
        *sc = scales[j] & 0x3F;
        *mn = scales[j + 4] & 0x3F;
    } else {
        *sc = (scales[j + 4] & 0x0F) | ((scales[j - 4] >> 6) << 4);
        *mn = (scales[j + 4] >> 4) | ((scales[j] >> 6) << 4);
    }
}

/* ref:src/kernels/dequantize.cu:278-325 */
void orc_dequantize_q4_k(const void* src, float* dst, int64_t n_blocks) {
    const uint8_t* s = (const uint8_t*)src;
    for (int64_t b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = s + b * 144;
        const float d = rd_half(blk);
        const float dmin = rd_half(blk + 2);
        const uint8_t* scales = blk + 4;
        const uint8_t* qs = blk + 16;
        for (int e = 0; e < 256; ++e) {
            int sc, mn;
            q4k_scale_min(scales, e / 32, &sc, &mn);
            const int chunk64 = e / 64, within = e % 64, l = within % 32;
            const uint8_t byte = qs[chunk64 * 32 + l];
            const int nib = within < 32 ? (byte & 0x0F) : (byte >> 4);
            dst[b * 256 + e] = d * (float)sc * (float)nib - dmin * (float)mn;
        }
    }
}

/* ref:src/kernels/matmul_quant.cu:539 (__half2float per element) */
void orc_dequantize_fp16(const void* src, float* dst, int64_t n_elems) {
    orc_half_to_float_array((const uint16_t*)src, dst, n_elems);
}

void orc_dequantize(int fmt, const void* src, float* dst, int64_t n_elems) {
    const int64_t nb = n_elems / orc_block_elems(fmt);
    switch (fmt) {
        case ORC_Q8_0: orc_dequantize_q8_0(src, dst, nb); break;
        case ORC_Q4_0: orc_dequantize_q4_0(src, dst, nb); break;
        case ORC_Q5_0: orc_dequantize_q5_0(src, dst, nb); break;
        case ORC_Q4_K: orc_dequantize_q4_k(src, dst, nb); break;
        case ORC_Q6_K: orc_dequantize_q6_k(src, dst, nb); break;
        case ORC_FP16: orc_dequantize_fp16(src, dst, n_elems); break;
    }
}

/* ---------------------------------------------------------------------------
 * Matmuls.
 * ------------------------------------------------------------------------- */

/* ref:tests/test_matmul_quant.cu:30-41 -- sequential fp32 sum over k */
void orc_matmul_bt(const float* A, const float* B, float* C, int M, int N, int K) {
    for (int i = 0; i < M; ++i) {
        for (int j = 0; j < N; ++j) {
            float sum = 0.0f;
            for (int k = 0; k < K; ++k) sum += A[(int64_t)i * K + k] * B[(int64_t)j * K + k];
            C[(int64_t)i * N + j] = sum;
        }
    }
}

/* dequant(B) + orc_matmul_bt, one B row at a time: the per-element arithmetic
 * is the same as dequantizing the whole tensor first (ref:tests/test_matmul_quant.cu:332-373). */
void orc_matmul_quant_rows(int fmt, const float* A, const void* Bq, float* C,
                           int M, int N, int K, int n0, int n1) {
    const int be = orc_block_elems(fmt);
    const int64_t row_bytes = (int64_t)(K / be) * orc_block_bytes(fmt);
    float* w = (float*)malloc(sizeof(float) * (size_t)K);
    if (!w) return;
    (void)N;
    for (int n = n0; n < n1; ++n) {
        orc_dequantize(fmt, (const uint8_t*)Bq + (int64_t)n * row_bytes, w, K);
        for (int i = 0; i < M; ++i) {
            float sum = 0.0f;
            const float* a = A + (int64_t)i * K;
            for (int k = 0; k < K; ++k) sum += a[k] * w[k];
            C[(int64_t)i * N + n] = sum;
        }
    }
    free(w);
}

void orc_matmul_quant(int fmt, const float* A, const void* Bq, float* C, int M, int N, int K) {
    orc_matmul_quant_rows(fmt, A, Bq, C, M, N, K, 0, N);
}

/* ref:tests/test_embedding.cu:98-109 */
void orc_matmul_transposed_b(const float* A, const float* B, float* C, int M, int N, int K) {
    orc_matmul_bt(A, B, C, M, N, K);
}

/* ref:tests/test_attention.cu:76-85 (cpu_matmul, B is [K,N]) and :399-407 */
void orc_batched_matmul_gqa(const float* A, const float* B, float* C,
                            int n_heads, int n_kv_heads, int M, int N, int K) {
    const int groups = n_heads / n_kv_heads;
    for (int h = 0; h < n_heads; ++h) {
        const int kv = h / groups;
        const float* a = A + (int64_t)h * M * K;
        const float* b = B + (int64_t)kv * K * N;
        float* c = C + (int64_t)h * M * N;
        for (int i = 0; i < M; ++i)
            for (int j = 0; j < N; ++j) {
                float sum = 0.0f;
                for (int k = 0; k < K; ++k) sum += a[(int64_t)i * K + k] * b[(int64_t)k * N + j];
                c[(int64_t)i * N + j] = sum;
            }
    }
}

/* Decode attention of one query token over the [kv_len, n_kv_heads, head_dim]
 * cache, as the reference's CPU test computes it: ref:tests/test_attention.cu:972-1008
 * (cpu_fused_decode_attention) with cpu_softmax (:110-122).  Scores are
 * sequential fp32 dot products times scale, the softmax subtracts the max
 * (starting from -FLT_MAX) and divides each exp by the sum, and the V sum runs
 * over positions in order. */
void orc_decode_attention(const float* Q, const float* Kc, const float* Vc, float* out,
                          int n_heads, int n_kv_heads, int head_dim, int kv_len, float scale) {
    const int groups = n_heads / n_kv_heads;
    const int64_t kv_dim = (int64_t)n_kv_heads * head_dim;
    float* scores = (float*)malloc(sizeof(float) * (size_t)(kv_len > 0 ? kv_len : 1));
    float* w = (float*)malloc(sizeof(float) * (size_t)(kv_len > 0 ? kv_len : 1));
    for (int h = 0; h < n_heads; ++h) {
        const int kvh = h / groups;
        const float* q = Q + (int64_t)h * head_dim;
        for (int t = 0; t < kv_len; ++t) {
            float dot = 0.0f;
            for (int d = 0; d < head_dim; ++d) dot += q[d] * Kc[t * kv_dim + (int64_t)kvh * head_dim + d];
            scores[t] = dot * scale;
        }
        float max_val = -3.40282347e+38f; /* -FLT_MAX */
        for (int t = 0; t < kv_len; ++t)
            if (scores[t] > max_val) max_val = scores[t];
        float sum_exp = 0.0f;
        for (int t = 0; t < kv_len; ++t) sum_exp += expf(scores[t] - max_val);
        for (int t = 0; t < kv_len; ++t) w[t] = expf(scores[t] - max_val) / sum_exp;
        for (int d = 0; d < head_dim; ++d) {
            float val = 0.0f;
            for (int t = 0; t < kv_len; ++t) val += w[t] * Vc[t * kv_dim + (int64_t)kvh * head_dim + d];
            out[(int64_t)h * head_dim + d] = val;
        }
    }
    free(scores);
    free(w);
}

/* The same attention by the reference kernel's single-pass recurrence,
 * ref:src/attention.cu:446-493: per position, score = dot * scale, running max
 * m, correction = exp(m_old - m_new), p = exp(score - m_new),
 * sum = sum * correction + p, acc[d] = acc[d] * correction + p * V[d]; finally
 * acc[d] * (1 / sum).  The dot is sequential here (the kernel's block
 * reduction order is not portable). */
void orc_decode_attention_online(const float* Q, const float* Kc, const float* Vc, float* out,
                                 int n_heads, int n_kv_heads, int head_dim, int kv_len, float scale) {
    const int groups = n_heads / n_kv_heads;
    const int64_t kv_dim = (int64_t)n_kv_heads * head_dim;
    float* acc = (float*)malloc(sizeof(float) * (size_t)(head_dim > 0 ? head_dim : 1));
    for (int h = 0; h < n_heads; ++h) {
        const int kvh = h / groups;
        const float* q = Q + (int64_t)h * head_dim;
        float max_score = -INFINITY, sum_exp = 0.0f;
        for (int d = 0; d < head_dim; ++d) acc[d] = 0.0f;
        for (int t = 0; t < kv_len; ++t) {
            const float* k = Kc + t * kv_dim + (int64_t)kvh * head_dim;
            const float* v = Vc + t * kv_dim + (int64_t)kvh * head_dim;
            float dot = 0.0f;
            for (int d = 0; d < head_dim; ++d) dot += q[d] * k[d];
            const float score = dot * scale;
            const float old_max = max_score;
            const float new_max = fmaxf(old_max, score);
            const float correction = expf(old_max - new_max);
            const float exp_score = expf(score - new_max);
            max_score = new_max;
            sum_exp = sum_exp * correction + exp_score;
            for (int d = 0; d < head_dim; ++d) acc[d] = acc[d] * correction + exp_score * v[d];
        }
        const float inv_sum = 1.0f / sum_exp;
        for (int d = 0; d < head_dim; ++d) out[(int64_t)h * head_dim + d] = acc[d] * inv_sum;
    }
    free(acc);
}

/* RMSNorm with a residual, ref:src/kernels/elementwise.cu:463-504 per row:
 * v = input + residual (residual may be NULL), output = v, sum of v^2 (here in
 * index order; the kernel's tree order is not portable), factor =
 * 1 / sqrt(sum / n + eps) (the kernel's rsqrtf), normed = output * weight * factor. */
void orc_rmsnorm_residual(const float* input, const float* residual, const float* weight, float* output,
                          float* normed, int rows, int n, float eps) {
    for (int r = 0; r < rows; ++r) {
        const float* in = input + (int64_t)r * n;
        const float* res = residual ? residual + (int64_t)r * n : NULL;
        float* out = output + (int64_t)r * n;
        float* nrm = normed + (int64_t)r * n;
        float ss = 0.0f;
        for (int i = 0; i < n; ++i) {
            const float v = in[i] + (res ? res[i] : 0.0f);
            out[i] = v;
            ss += v * v;
        }
        const float mean_sq = ss / (float)n;
        const float f = 1.0f / sqrtf(mean_sq + eps);
        for (int i = 0; i < n; ++i) nrm[i] = out[i] * weight[i] * f;
    }
}

/* silu then multiply, ref:src/kernels/elementwise.cu:93-99 and :300-305 */
void orc_silu_mul(const float* gate, const float* up, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float x = gate[i];
        const float s = x / (1.0f + expf(-x));
        out[i] = s * up[i];
    }
}

/* RoPE of one token's heads in place, ref:src/kernels/elementwise.cu:232-257:
 * pair i of a head (elements 2i, 2i+1) turns by pos / theta^(2i / head_dim),
 * with the reference's fp32 expressions for the frequency and the angle. */
void orc_rope(float* qk, int pos, int head_dim, int n_heads, float theta) {
    const int half = head_dim / 2;
    for (int h = 0; h < n_heads; ++h) {
        for (int i = 0; i < half; ++i) {
            const float freq = 1.0f / powf(theta, (2.0f * (float)i) / (float)head_dim);
            const float ang = (float)pos * freq;
            const float c = cosf(ang), s = sinf(ang);
            float* p = qk + (int64_t)h * head_dim + 2 * i;
            const float x0 = p[0], x1 = p[1];
            p[0] = x0 * c - x1 * s;
            p[1] = x0 * s + x1 * c;
        }
    }
}

/* Greedy token, ref:src/embedding.cu:155-200 (kernel_argmax): the largest value
 * (NaN never compares larger), the smallest index among equal maxima, starting
 * from (-FLT_MAX, 0) -- so a row of -inf / NaN gives 0. */
int32_t orc_argmax(const float* x, int n) {
    float best = -3.402823466e38f;
    int32_t bi = 0;
    for (int i = 0; i < n; ++i) {
        if (x[i] > best) {
            best = x[i];
            bi = i;
        }
    }
    return bi;
}

/* ---------------------------------------------------------------------------
 * Host quantizers (ref:tests/test_matmul_quant.cu).  std::round is roundf
 * (half away from zero); __float2half is round-to-nearest-even.
 * ------------------------------------------------------------------------- */

static float block_amax(const float* x, int n) {
    float amax = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float a = fabsf(x[i]);
        amax = amax < a ? a : amax; /* std::max(amax, |x|) */
    }
    return amax;
}

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* :46-71 */
void orc_quantize_q8_0(const float* x, void* dst, int64_t n) {
    uint8_t* out = (uint8_t*)dst;
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* v = x + b * 32;
        uint8_t* blk = out + b * 34;
        float scale = block_amax(v, 32) / 127.0f;
        if (scale == 0.0f) scale = 1.0f;
        wr_half(blk, scale);
        const float inv = 1.0f / scale;
        for (int i = 0; i < 32; ++i) {
            int q = (int)roundf(v[i] * inv);
            blk[2 + i] = (uint8_t)(int8_t)clampi(q, -128, 127);
        }
    }
}

/* :74-102 (element i -> qs[i/2], low nibble for even i) */
void orc_quantize_q4_0(const float* x, void* dst, int64_t n) {
    uint8_t* out = (uint8_t*)dst;
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* v = x + b * 32;
        uint8_t* blk = out + b * 18;
        float scale = block_amax(v, 32) / 8.0f;
        if (scale == 0.0f) scale = 1.0f;
        wr_half(blk, scale);
        const float inv = 1.0f / scale;
        for (int i = 0; i < 32; i += 2) {
            int v0 = clampi((int)roundf(v[i] * inv) + 8, 0, 15);
            int v1 = clampi((int)roundf(v[i + 1] * inv) + 8, 0, 15);
            blk[2 + i / 2] = (uint8_t)(v0 | (v1 << 4));
        }
    }
}

/* :410-460 */
void orc_quantize_q5_0(const float* x, void* dst, int64_t n) {
    uint8_t* out = (uint8_t*)dst;
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* v = x + b * 32;
        uint8_t* blk = out + b * 22;
        float scale = block_amax(v, 32) / 16.0f;
        if (scale == 0.0f) scale = 1.0f;
        wr_half(blk, scale);
        const float inv = 1.0f / scale;
        uint32_t qh = 0;
        uint8_t* qs = blk + 6;
        memset(qs, 0, 16);
        for (int i = 0; i < 32; ++i) {
            const int q = clampi((int)roundf(v[i] * inv) + 16, 0, 31);
            const int low4 = q & 0x0F, hb = (q >> 4) & 1;
            if (i < 16) qs[i] = (uint8_t)((qs[i] & 0xF0) | low4);
            else qs[i - 16] = (uint8_t)((qs[i - 16] & 0x0F) | (low4 << 4));
            if (hb) qh |= 1u << i;
        }
        blk[2] = (uint8_t)(qh & 0xFF);
        blk[3] = (uint8_t)((qh >> 8) & 0xFF);
        blk[4] = (uint8_t)((qh >> 16) & 0xFF);
        blk[5] = (uint8_t)((qh >> 24) & 0xFF);
    }
}

/* :611-686 */
void orc_quantize_q6_k(const float* x, void* dst, int64_t n) {
    uint8_t* out = (uint8_t*)dst;
    for (int64_t b = 0; b < n / 256; ++b) {
        const float* v = x + b * 256;
        uint8_t* blk = out + b * 210;
        memset(blk, 0, 210);
        uint8_t* ql = blk;
        uint8_t* qh = blk + 128;
        int8_t* scales = (int8_t*)(blk + 192);
        const float amax = block_amax(v, 256);
        float sub_amax[16];
        for (int g = 0; g < 16; ++g) sub_amax[g] = block_amax(v + g * 16, 16);
        const float d = amax > 0 ? amax / (32.0f * 31.0f) : 1.0f;
        wr_half(blk + 208, d);
        const float inv_d = 1.0f / d;
        int8_t sc[16];
        for (int g = 0; g < 16; ++g) {
            const float sub_scale = sub_amax[g] > 0 ? sub_amax[g] / 31.0f : 0.0f;
            /* the reference casts to int8_t first, then clamps to [-127, 127] */
            const int s = clampi((int)(int8_t)roundf(sub_scale * inv_d), -127, 127);
            sc[g] = (int8_t)s;
            scales[g] = (int8_t)s;
        }
        for (int g16 = 0; g16 < 16; ++g16) {
            const float eff = d * (float)sc[g16];
            const float inv_eff = eff != 0.0f ? 1.0f / eff : 0.0f;
            for (int i = 0; i < 16; ++i) {
                const int e = g16 * 16 + i;
                const int q6 = clampi((int)roundf(v[e] * inv_eff) + 32, 0, 63);
                const int low4 = q6 & 0x0F, high2 = (q6 >> 4) & 0x03;
                const int chunk = e / 128, within = e % 128;
                const int quarter = within / 32, l = within % 32;
                const int ql_off = (quarter & 1) * 32 + l + chunk * 64;
                if (quarter < 2) ql[ql_off] = (uint8_t)((ql[ql_off] & 0xF0) | low4);
                else ql[ql_off] = (uint8_t)((ql[ql_off] & 0x0F) | (low4 << 4));
                qh[l + chunk * 32] |= (uint8_t)(high2 << (quarter * 2));
            }
        }
    }
}

/* :107-184 (dmin = 0, mins = 0; negative values clamp to nibble 0) */
void orc_quantize_q4_k_simple(const float* x, void* dst, int64_t n) {
    uint8_t* out = (uint8_t*)dst;
    for (int64_t b = 0; b < n / 256; ++b) {
        const float* v = x + b * 256;
        uint8_t* blk = out + b * 144;
        uint8_t* scales = blk + 4;
        uint8_t* qs = blk + 16;
        float d_val = block_amax(v, 256) / (15.0f * 63.0f);
        if (d_val == 0.0f) d_val = 1e-6f;
        wr_half(blk, d_val);
        wr_half(blk + 2, 0.0f);
        memset(scales, 0, 12);
        for (int sb = 0; sb < 8; ++sb) {
            const float sb_max = block_amax(v + sb * 32, 32);
            float r = roundf(sb_max / (d_val * 15.0f));
            const uint8_t sc = (uint8_t)(63.0f < r ? 63.0f : r);
            if (sb < 4) {
                scales[sb] = (uint8_t)((scales[sb] & 0xC0) | (sc & 0x3F));
            } else {
                scales[sb + 4] = (uint8_t)((scales[sb + 4] & 0xF0) | (sc & 0x0F));
                scales[sb - 4] = (uint8_t)((scales[sb - 4] & 0x3F) | ((sc >> 4) << 6));
            }
        }
        memset(qs, 0, 128);
        const float dh = rd_half(blk);
        for (int c = 0; c < 4; ++c) {
            int sc_lo, sc_hi, dummy;
            q4k_scale_min(scales, 2 * c, &sc_lo, &dummy);
            q4k_scale_min(scales, 2 * c + 1, &sc_hi, &dummy);
            const float eff_lo = dh * (float)sc_lo, eff_hi = dh * (float)sc_hi;
            const float inv_lo = eff_lo > 0 ? 1.0f / eff_lo : 0.0f;
            const float inv_hi = eff_hi > 0 ? 1.0f / eff_hi : 0.0f;
            for (int l = 0; l < 32; ++l) {
                const int vlo = clampi((int)roundf(v[c * 64 + l] * inv_lo), 0, 15);
                const int vhi = clampi((int)roundf(v[c * 64 + l + 32] * inv_hi), 0, 15);
                qs[c * 32 + l] = (uint8_t)(vlo | (vhi << 4));
            }
        }
    }
}

/* Own asymmetric Q4_K quantizer: per 32-element sub-block, scale = (max - min)/15
 * and min offset = -min (min clamped to <= 0); 6-bit sc/mn relative to
 * d = max(scale)/63 and dmin = max(offset)/63; nibble = round((x + dmin*mn)/(d*sc))
 * with the fp16-rounded d/dmin.  Packing follows the decode of
 * ref:src/kernels/dequantize.cu:298-319. */
void orc_quantize_q4_k_asym(const float* x, void* dst, int64_t n) {
    uint8_t* out = (uint8_t*)dst;
    for (int64_t b = 0; b < n / 256; ++b) {
        const float* v = x + b * 256;
        uint8_t* blk = out + b * 144;
        uint8_t* scales = blk + 4;
        uint8_t* qs = blk + 16;
        float sub_scale[8], sub_min[8];
        float max_scale = 0.0f, max_min = 0.0f;
        for (int s = 0; s < 8; ++s) {
            float lo = v[s * 32], hi = v[s * 32];
            for (int i = 1; i < 32; ++i) {
                const float t = v[s * 32 + i];
                lo = t < lo ? t : lo;
                hi = t > hi ? t : hi;
            }
            if (lo > 0.0f) lo = 0.0f;
            sub_scale[s] = (hi - lo) / 15.0f;
            sub_min[s] = -lo;
            max_scale = sub_scale[s] > max_scale ? sub_scale[s] : max_scale;
            max_min = sub_min[s] > max_min ? sub_min[s] : max_min;
        }
        const float d = max_scale / 63.0f;
        const float dmin = max_min / 63.0f;
        const float inv_d = d > 0.0f ? 1.0f / d : 0.0f;
        const float inv_m = dmin > 0.0f ? 1.0f / dmin : 0.0f;
        int sc[8], mn[8];
        for (int s = 0; s < 8; ++s) {
            sc[s] = clampi((int)roundf(sub_scale[s] * inv_d), 0, 63);
            mn[s] = clampi((int)roundf(sub_min[s] * inv_m), 0, 63);
        }
        for (int j = 0; j < 4; ++j) {
            scales[j] = (uint8_t)((sc[j] & 0x3F) | ((sc[j + 4] >> 4) << 6));
            scales[j + 4] = (uint8_t)((mn[j] & 0x3F) | ((mn[j + 4] >> 4) << 6));
            scales[j + 8] = (uint8_t)((sc[j + 4] & 0x0F) | ((mn[j + 4] & 0x0F) << 4));
        }
        wr_half(blk, d);
        wr_half(blk + 2, dmin);
        const float dq = rd_half(blk), dmq = rd_half(blk + 2);
        memset(qs, 0, 128);
        for (int e = 0; e < 256; ++e) {
            const int s = e / 32;
            const float eff = dq * (float)sc[s];
            const float off = dmq * (float)mn[s];
            const int q = eff > 0.0f ? clampi((int)roundf((v[e] + off) / eff), 0, 15) : 0;
            const int chunk64 = e / 64, within = e % 64, l = within % 32;
            if (within < 32) qs[chunk64 * 32 + l] |= (uint8_t)q;
            else qs[chunk64 * 32 + l] |= (uint8_t)(q << 4);
        }
    }
}

/* ---------------------------------------------------------------------------
 * Deterministic block makers, ref:tests/test_dequantize.cu:135-208.
 * ------------------------------------------------------------------------- */

void orc_make_q8_0_blocks(void* dst, int n_blocks) {
    uint8_t* out = (uint8_t*)dst;
    for (int b = 0; b < n_blocks; ++b) {
        uint8_t* blk = out + b * 34;
        wr_half(blk, 0.1f * (float)(b + 1));
        for (int i = 0; i < 32; ++i) blk[2 + i] = (uint8_t)(int8_t)((i * 7 + b * 13) % 255 - 127);
    }
}

void orc_make_q4_0_blocks(void* dst, int n_blocks) {
    uint8_t* out = (uint8_t*)dst;
    for (int b = 0; b < n_blocks; ++b) {
        uint8_t* blk = out + b * 18;
        wr_half(blk, 0.05f * (float)(b + 1));
        for (int i = 0; i < 16; ++i) {
            const uint8_t lo = (uint8_t)((i + b) % 16), hi = (uint8_t)((i * 3 + b * 5) % 16);
            blk[2 + i] = (uint8_t)(lo | (hi << 4));
        }
    }
}

void orc_make_q6_k_blocks(void* dst, int n_blocks) {
    uint8_t* out = (uint8_t*)dst;
    for (int b = 0; b < n_blocks; ++b) {
        uint8_t* blk = out + b * 210;
        wr_half(blk + 208, 0.02f * (float)(b + 1));
        for (int i = 0; i < 16; ++i) blk[192 + i] = (uint8_t)(int8_t)((i * 3 + b) % 127 - 63);
        for (int i = 0; i < 128; ++i) {
            const uint8_t lo = (uint8_t)((i + b) % 16), hi = (uint8_t)((i * 3 + b) % 16);
            blk[i] = (uint8_t)(lo | (hi << 4));
        }
        for (int i = 0; i < 64; ++i) blk[128 + i] = (uint8_t)((i + b * 7) % 256);
    }
}

void orc_make_q4_k_blocks(void* dst, int n_blocks) {
    uint8_t* out = (uint8_t*)dst;
    for (int b = 0; b < n_blocks; ++b) {
        uint8_t* blk = out + b * 144;
        wr_half(blk, 0.03f * (float)(b + 1));
        wr_half(blk + 2, 0.01f * (float)(b + 1));
        for (int i = 0; i < 12; ++i) blk[4 + i] = (uint8_t)((i * 17 + b * 11) % 256);
        for (int i = 0; i < 128; ++i) {
            const uint8_t lo = (uint8_t)((i + b * 3) % 16), hi = (uint8_t)((i * 5 + b) % 16);
            blk[16 + i] = (uint8_t)(lo | (hi << 4));
        }
    }
}

/* ---------------------------------------------------------------------------
 * Data generators.
 * ------------------------------------------------------------------------- */

/* ref:tests/test_matmul_quant.cu:187-195 */
void orc_random_matrix_lcg(float* dst, int64_t n, uint32_t seed) {
    uint32_t state = seed;
    for (int64_t i = 0; i < n; ++i) {
        state = state * 1103515245u + 12345u;
        dst[i] = ((float)(state & 0xFFFFu) / 32768.0f) - 1.0f;
    }
}

static uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* splitmix64 -> two 53-bit uniforms in (0,1] -> Box-Muller in double */
void orc_randn(float* dst, int64_t n, uint64_t seed, float sigma) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        const double u1 = ((double)(splitmix64(&s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        const double u2 = ((double)(splitmix64(&s) >> 11)) * (1.0 / 9007199254740992.0);
        const double r = sqrt(-2.0 * log(u1));
        dst[i] = (float)(r * cos(two_pi * u2)) * sigma;
        if (i + 1 < n) dst[i + 1] = (float)(r * sin(two_pi * u2)) * sigma;
    }
}

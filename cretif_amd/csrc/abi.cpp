// abi.cpp -- the extern "C" boundary declared in include/cri.h.
//
// Validates every argument before anything is enqueued (the reference
// launches unconditionally and truncates K/32 and K/256 silently,
// ref:src/kernels/matmul_quant.cu:77-78, 322-323), picks a kernel, and turns
// HIP launch failures into CRI_ERR_LAUNCH with a message.
#include "../../include/cri.h"

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <algorithm>
#include <string>

#include "internal.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int status, const char* fn, const std::string& what) {
    g_last_error = std::string(fn) + ": " + what;
    return status;
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int check_launch(const char* fn) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(CRI_ERR_LAUNCH, fn, std::string("kernel launch failed: ") + hipGetErrorString(e));
    return CRI_OK;
}

// Clears an error an earlier, unrelated HIP call left pending, so that check_launch
// reports only the status of this call's own launches.
void clear_pending_error() { (void)hipGetLastError(); }

// A specialised launcher either enqueued its kernels (0), declined the shape
// (kDeclined: the element-wise kernel takes it) or hit a runtime failure
// (kFailed: reported, never retried on another kernel).
int finish_matmul(int rc, const char* fn) {
    if (rc == cri::detail::kFailed) {
        const hipError_t e = hipGetLastError();
        return fail(CRI_ERR_LAUNCH, fn,
                    std::string("kernel set-up or launch failed: ") +
                        (e != hipSuccess ? hipGetErrorString(e) : "hipFuncSetAttribute/hipGetDevice refused"));
    }
    if (rc != 0) return fail(CRI_ERR_UNSUPPORTED, fn, "no kernel for this shape");
    return check_launch(fn);
}

constexpr long kMaxElems = (1L << 40);

// Batches above this many rows are prefill: they run on the fp16-operand MFMA
// GEMM (stated tolerance 1e-3); smaller batches keep fp32-accurate kernels.
constexpr int kPrefillMinM = 16;

int fill_zero(float* C, long n, hipStream_t stream, const char* fn);

int matmul_impl(int fmt, const float* A, const void* B, float* C, int M, int N, int K, hipStream_t stream,
                const char* fn, float* ws = nullptr, long ws_floats = 0, cri::SplitSums* defer = nullptr,
                int defer_S = 0) {
    if (defer) defer->S = 0;
    if (M < 0 || N < 0 || K < 0)
        return fail(CRI_ERR_INVALID_ARGUMENT, fn,
                    "negative dimension (M=" + std::to_string(M) + ", N=" + std::to_string(N) +
                        ", K=" + std::to_string(K) + ")");
    const int be = cri::block_elems(fmt);
    if (K % be != 0)
        return fail(CRI_ERR_SHAPE, fn,
                    "K=" + std::to_string(K) + " is not a multiple of the block size " + std::to_string(be));
    if (M == 0 || N == 0) return CRI_OK;
    if (!A || !B || !C) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null pointer");
    if (!aligned(A, 4) || !aligned(C, 4)) return fail(CRI_ERR_ALIGNMENT, fn, "A and C must be 4-byte aligned");
    if (fmt == cri::kFmtF16 && !aligned(B, 2)) return fail(CRI_ERR_ALIGNMENT, fn, "FP16 B must be 2-byte aligned");
    if (static_cast<long>(M) * K > kMaxElems || static_cast<long>(M) * N > kMaxElems)
        return fail(CRI_ERR_SHAPE, fn, "problem too large");
    clear_pending_error();
    if (K == 0) return fill_zero(C, static_cast<long>(M) * N, stream, fn);
    int rc;
    // batches of two (Q8_0, Q4_0, Q5_0, Q6_K) or up to four (the 32-element formats) as row
    // pairs on the two-row GEMV: measured faster than the skinny MFMA kernel there
    // (8192 x 2048 at M = 4: Q4_0 11.7 -> 9.3 us, Q5_0 16.7 -> 9.5, Q8_0 12.0 -> 10.4); from
    // M = 8, and for Q6_K from M = 4, the skinny kernel is faster
    const bool fmt32 = fmt == cri::kFmtQ8_0 || fmt == cri::kFmtQ4_0 || fmt == cri::kFmtQ5_0;
    if (((M >= 2 && M <= 4 && fmt32) || (M == 2 && fmt == cri::kFmtQ6_K)) && K <= 4096 &&
        cri::detail::gemv_supported(fmt, K, B))
        rc = cri::detail::launch_gemv2(fmt, A, B, C, M, N, K, stream);
    else if (cri::detail::skinny_supported(fmt, M, K, B))
        rc = cri::detail::launch_skinny_act(cri::kActPlain, fmt, cri::ActIn{A, nullptr, nullptr, nullptr, K, 0.0f}, B,
                                            C, M, N, K, stream, ws, ws_floats, defer, defer_S);
    else if (M == 1 && cri::detail::slice_gemv_supported(fmt, N, K, B))
        rc = cri::detail::launch_slice_gemv(cri::kActPlain, fmt, cri::ActIn{A, nullptr, nullptr, nullptr, K, 0.0f}, B,
                                            C, N, K, stream);
    else if (M == 1 && cri::detail::gemv_supported(fmt, K, B))
        rc = cri::detail::launch_gemv(fmt, A, B, C, N, K, stream);
    else if (M > kPrefillMinM && cri::detail::prefill_supported(fmt, M, N, K, A, B))
        rc = cri::detail::launch_prefill(fmt, A, B, C, M, N, K, stream, ws, ws_floats, defer, defer_S);
    else if (M > kPrefillMinM && cri::detail::mfma_gemm_supported(fmt, M, N, K, A, B))
        rc = cri::detail::launch_mfma_gemm(fmt, A, B, C, M, N, K, stream);
    else if (M <= 16 && fmt32 && K <= 4096 && cri::detail::gemv_supported(fmt, K, B))
        // small batches whose K is not a multiple of 256 (no skinny kernel): row pairs on the two-row GEMV
        rc = cri::detail::launch_gemv2(fmt, A, B, C, M, N, K, stream);
    else
        rc = cri::detail::kDeclined;
    if (rc == cri::detail::kDeclined) rc = cri::detail::launch_generic_matmul(fmt, A, B, C, M, N, K, stream);
    return finish_matmul(rc, fn);
}

int dequant_impl(int fmt, const void* src, float* dst, int n_blocks, hipStream_t stream, const char* fn) {
    if (n_blocks < 0) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "negative n_blocks");
    if (n_blocks == 0) return CRI_OK;
    if (!src || !dst) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null pointer");
    if (!aligned(dst, 4)) return fail(CRI_ERR_ALIGNMENT, fn, "dst must be 4-byte aligned");
    clear_pending_error();
    if (cri::detail::launch_dequant(fmt, src, dst, n_blocks, stream) != 0)
        return fail(CRI_ERR_UNSUPPORTED, fn, "unknown format");
    return check_launch(fn);
}

}  // namespace

void cri_internal_set_error(const char* msg) { g_last_error = msg; }

namespace {
int fill_zero(float* C, long n, hipStream_t stream, const char* fn) {
    clear_pending_error();
    cri::detail::launch_fill_zero(C, n, stream);
    return check_launch(fn);
}
}  // namespace

extern "C" {

int cri_matmul_q8_0(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t s) {
    return matmul_impl(cri::kFmtQ8_0, A, B, C, M, N, K, s, "cri_matmul_q8_0");
}
int cri_matmul_q4_0(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t s) {
    return matmul_impl(cri::kFmtQ4_0, A, B, C, M, N, K, s, "cri_matmul_q4_0");
}
int cri_matmul_q5_0(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t s) {
    return matmul_impl(cri::kFmtQ5_0, A, B, C, M, N, K, s, "cri_matmul_q5_0");
}
int cri_matmul_q4_k(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t s) {
    return matmul_impl(cri::kFmtQ4_K, A, B, C, M, N, K, s, "cri_matmul_q4_k");
}
int cri_matmul_q6_k(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t s) {
    return matmul_impl(cri::kFmtQ6_K, A, B, C, M, N, K, s, "cri_matmul_q6_k");
}
int cri_matmul_fp16(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t s) {
    // The reference requires K % 32 == 0 for FP16 too (ref:include/cuinfer/kernels/matmul_quant.h:102).
    if (K >= 0 && K % 32 != 0)
        return fail(CRI_ERR_SHAPE, "cri_matmul_fp16", "K=" + std::to_string(K) + " is not a multiple of 32");
    return matmul_impl(cri::kFmtF16, A, B, C, M, N, K, s, "cri_matmul_fp16");
}
int cri_matmul(int format, const float* A, const void* B, float* C, int M, int N, int K, hipStream_t s) {
    switch (format) {
        case CRI_Q8_0: return cri_matmul_q8_0(A, B, C, M, N, K, s);
        case CRI_Q4_0: return cri_matmul_q4_0(A, B, C, M, N, K, s);
        case CRI_Q5_0: return cri_matmul_q5_0(A, B, C, M, N, K, s);
        case CRI_Q4_K: return cri_matmul_q4_k(A, B, C, M, N, K, s);
        case CRI_Q6_K: return cri_matmul_q6_k(A, B, C, M, N, K, s);
        case CRI_FP16: return cri_matmul_fp16(A, B, C, M, N, K, s);
    }
    return fail(CRI_ERR_UNSUPPORTED, "cri_matmul", "unknown format id " + std::to_string(format));
}

long long cri_matmul_workspace_bytes(int format, int M, int N, int K) {
    if (format < CRI_Q8_0 || format > CRI_FP16 || M < 0 || N < 0 || K < 0) return CRI_ERR_INVALID_ARGUMENT;
    if (M < 2 || N == 0 || K == 0) return 0;
    // above 16 rows: the prefill kernel's K split (formats and K it takes; the other kernels split nothing
    // a workspace would hold)
    if (M > kPrefillMinM)
        return K % 256 == 0 ? static_cast<long long>(cri::detail::prefill_workspace_floats(M, N, K)) * 4 : 0;
    return static_cast<long long>(cri::detail::skinny_workspace_floats(M, N)) * 4;
}

int cri_matmul_ws(int format, const float* A, const void* B, float* C, int M, int N, int K, void* workspace,
                  long long workspace_bytes, hipStream_t s) {
    const char* fn = "cri_matmul_ws";
    if (format < CRI_Q8_0 || format > CRI_FP16)
        return fail(CRI_ERR_UNSUPPORTED, fn, "unknown format id " + std::to_string(format));
    if (format == CRI_FP16 && K >= 0 && K % 32 != 0)
        return fail(CRI_ERR_SHAPE, fn, "K=" + std::to_string(K) + " is not a multiple of 32");
    float* ws = nullptr;
    long ws_floats = 0;
    if (M >= 2 && M <= 16 && N > 0 && K > 0) {
        // the K split's partial sums go to the workspace and are added in split order (the same bits
        // on every call); its reduction stores C as 16-byte vectors
        const long long need = cri_matmul_workspace_bytes(format, M, N, K);
        if (!workspace || workspace_bytes < need)
            return fail(CRI_ERR_INVALID_ARGUMENT, fn,
                        "workspace of at least " + std::to_string(need) + " bytes needed (cri_matmul_workspace_bytes)");
        if (!aligned(workspace, 16) || !aligned(C, 16) || N % 4 != 0)
            return fail(CRI_ERR_ALIGNMENT, fn, "workspace and C must be 16-byte aligned and N a multiple of 4");
        // used only where cri_matmul would add partial sums with atomics; elsewhere its kernel
        // choice is already deterministic and as fast or faster (8192 x 2048 at 16 rows: 9.7 us
        // unsplit against 11.1 split with a workspace)
        if (cri::detail::skinny_atomic_split(M, K)) {
            ws = static_cast<float*>(workspace);
            ws_floats = static_cast<long>(workspace_bytes / 4);
        }
    } else if (M > kPrefillMinM && N > 0 && K > 0) {
        // the prefill GEMM's K split (few output tiles, e.g. 512 x 2048 x 8192): its partial sums go
        // to the workspace and a second launch adds them in split order, in place of atomics into a
        // zero-filled C (the same bits on every call)
        const long long need = cri_matmul_workspace_bytes(format, M, N, K);
        if (need > 0 && cri::detail::prefill_supported(format, M, N, K, A, B)) {
            if (!workspace || workspace_bytes < need)
                return fail(CRI_ERR_INVALID_ARGUMENT, fn,
                            "workspace of at least " + std::to_string(need) +
                                " bytes needed (cri_matmul_workspace_bytes)");
            if (!aligned(workspace, 16) || !aligned(C, 16) || N % 4 != 0)
                return fail(CRI_ERR_ALIGNMENT, fn, "workspace and C must be 16-byte aligned and N a multiple of 4");
            ws = static_cast<float*>(workspace);
            ws_floats = static_cast<long>(workspace_bytes / 4);
        }
    }
    // the format ids of cri.h are the library's internal ones
    return matmul_impl(format, A, B, C, M, N, K, s, fn, ws, ws_floats);
}

int cri_dequantize_q8_0(const void* src, float* dst, int n_blocks, hipStream_t s) {
    return dequant_impl(cri::kFmtQ8_0, src, dst, n_blocks, s, "cri_dequantize_q8_0");
}
int cri_dequantize_q4_0(const void* src, float* dst, int n_blocks, hipStream_t s) {
    return dequant_impl(cri::kFmtQ4_0, src, dst, n_blocks, s, "cri_dequantize_q4_0");
}
int cri_dequantize_q5_0(const void* src, float* dst, int n_blocks, hipStream_t s) {
    return dequant_impl(cri::kFmtQ5_0, src, dst, n_blocks, s, "cri_dequantize_q5_0");
}
int cri_dequantize_q6_k(const void* src, float* dst, int n_blocks, hipStream_t s) {
    return dequant_impl(cri::kFmtQ6_K, src, dst, n_blocks, s, "cri_dequantize_q6_k");
}
int cri_dequantize_q4_k(const void* src, float* dst, int n_blocks, hipStream_t s) {
    return dequant_impl(cri::kFmtQ4_K, src, dst, n_blocks, s, "cri_dequantize_q4_k");
}

int cri_matmul_transposed_b(const float* A, const float* B, float* C, int M, int N, int K, hipStream_t s) {
    const char* fn = "cri_matmul_transposed_b";
    if (M < 0 || N < 0 || K < 0) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "negative dimension");
    if (M == 0 || N == 0) return CRI_OK;
    if (!A || !B || !C) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null pointer");
    if (!aligned(A, 4) || !aligned(B, 4) || !aligned(C, 4))
        return fail(CRI_ERR_ALIGNMENT, fn, "A, B and C must be 4-byte aligned");
    if (static_cast<long>(M) * K > kMaxElems || static_cast<long>(N) * K > kMaxElems)
        return fail(CRI_ERR_SHAPE, fn, "problem too large");
    if (K == 0) return fill_zero(C, static_cast<long>(M) * N, s, fn);
    clear_pending_error();
    if (cri::detail::launch_transposed_b(A, B, C, M, N, K, s) != 0)
        return fail(CRI_ERR_UNSUPPORTED, fn, "no kernel for this shape");
    return check_launch(fn);
}

int cri_batched_matmul_gqa(const float* A, const float* B, float* C, int n_heads, int n_kv_heads, int M, int N,
                           int K, hipStream_t s) {
    const char* fn = "cri_batched_matmul_gqa";
    if (n_heads < 0 || n_kv_heads < 0 || M < 0 || N < 0 || K < 0)
        return fail(CRI_ERR_INVALID_ARGUMENT, fn, "negative dimension");
    if (n_heads == 0 || M == 0 || N == 0) return CRI_OK;
    if (n_kv_heads == 0 || n_heads % n_kv_heads != 0)
        return fail(CRI_ERR_SHAPE, fn,
                    "n_heads=" + std::to_string(n_heads) + " is not a multiple of n_kv_heads=" +
                        std::to_string(n_kv_heads));
    if (!A || !B || !C) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null pointer");
    if (!aligned(A, 4) || !aligned(B, 4) || !aligned(C, 4))
        return fail(CRI_ERR_ALIGNMENT, fn, "A, B and C must be 4-byte aligned");
    if (K == 0) return fill_zero(C, static_cast<long>(n_heads) * M * N, s, fn);
    clear_pending_error();
    if (cri::detail::launch_gqa(A, B, C, n_heads, n_kv_heads, M, N, K, s) != 0)
        return fail(CRI_ERR_UNSUPPORTED, fn, "no kernel for this shape");
    return check_launch(fn);
}

int cri_fused_decode_attention(const float* Q, const float* K_cache, const float* V_cache, float* output,
                               int n_heads, int n_kv_heads, int head_dim, int kv_len, float scale, hipStream_t s) {
    const char* fn = "cri_fused_decode_attention";
    if (n_heads < 0 || n_kv_heads < 0 || head_dim < 0 || kv_len < 0)
        return fail(CRI_ERR_INVALID_ARGUMENT, fn, "negative dimension");
    if (n_heads == 0 || head_dim == 0) return CRI_OK;
    if (n_kv_heads == 0 || n_heads % n_kv_heads != 0)
        return fail(CRI_ERR_SHAPE, fn,
                    "n_heads=" + std::to_string(n_heads) + " is not a multiple of n_kv_heads=" +
                        std::to_string(n_kv_heads));
    // the reference divides by an empty softmax sum (NaN output) for kv_len == 0
    if (kv_len == 0) return fail(CRI_ERR_SHAPE, fn, "kv_len must be at least 1");
    if (head_dim > cri::detail::kDecodeAttnMaxHeadDim)
        return fail(CRI_ERR_SHAPE, fn,
                    "head_dim=" + std::to_string(head_dim) + " exceeds " +
                        std::to_string(cri::detail::kDecodeAttnMaxHeadDim));
    if (!Q || !K_cache || !V_cache || !output) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null pointer");
    if (!aligned(Q, 4) || !aligned(K_cache, 4) || !aligned(V_cache, 4) || !aligned(output, 4))
        return fail(CRI_ERR_ALIGNMENT, fn, "Q, K_cache, V_cache and output must be 4-byte aligned");
    if (static_cast<long>(kv_len) * n_kv_heads * head_dim > kMaxElems)
        return fail(CRI_ERR_SHAPE, fn, "problem too large");
    clear_pending_error();
    if (cri::detail::launch_decode_attention(Q, K_cache, V_cache, output, n_heads, n_kv_heads, head_dim, kv_len,
                                             scale, s) != 0)
        return fail(CRI_ERR_UNSUPPORTED, fn, "no kernel for this shape");
    return check_launch(fn);
}

namespace {

bool overlaps(const void* a, long abytes, const void* b, long bbytes) {
    if (!a || !b || abytes <= 0 || bbytes <= 0) return false;
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + static_cast<uintptr_t>(bbytes) && y < x + static_cast<uintptr_t>(abytes);
}

// Batches up to this many rows take the fused activation prologues (decode).
constexpr int kFusedMaxM = 16;

int fused_matmul(int mode, int fmt, const cri::ActIn& act, const void* B, float* C, int M, int N, int K,
                 hipStream_t stream, const char* fn, float* ws = nullptr, long ws_floats = 0,
                 cri::SplitSums* defer = nullptr, int defer_S = 0) {
    if (defer) defer->S = 0;
    if (fmt < cri::kFmtQ8_0 || fmt > cri::kFmtF16) return fail(CRI_ERR_UNSUPPORTED, fn, "unknown format id");
    if (M < 0 || N < 0 || K < 0) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "negative dimension");
    const int be = cri::block_elems(fmt);
    if (K % be != 0 || (fmt == cri::kFmtF16 && K % 32 != 0))
        return fail(CRI_ERR_SHAPE, fn, "K=" + std::to_string(K) + " is not a multiple of the block size");
    if (M == 0 || N == 0) return CRI_OK;
    if (M > kFusedMaxM)
        return fail(CRI_ERR_UNSUPPORTED, fn,
                    "the fused prologue serves decode batches (M <= 16); for M=" + std::to_string(M) +
                        " run cri_rmsnorm_residual / cri_silu_mul, then cri_matmul");
    if (!B || !C) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null pointer");
    if (!aligned(C, 4)) return fail(CRI_ERR_ALIGNMENT, fn, "C must be 4-byte aligned");
    if (fmt == cri::kFmtF16 && !aligned(B, 2)) return fail(CRI_ERR_ALIGNMENT, fn, "FP16 B must be 2-byte aligned");
    clear_pending_error();
    if (mode == cri::kActRMSNormS) {  // one token on the batch-1 GEMV only
        if (M == 1 && cri::detail::gemv_supported(fmt, K, B))
            return finish_matmul(cri::detail::launch_gemv_act(mode, fmt, act, B, C, N, K, stream), fn);
        return fail(CRI_ERR_UNSUPPORTED, fn, "a split residual is taken by the batch-1 GEMV only");
    }
    int rc = cri::detail::kDeclined;
    // SwiGLU at one row: the K-sliced GEMV where each lane's activations are its own (K = 8192:
    // 2048 x 8192 Q4_K 4.97 us against 6.73 on the batch-1 GEMV); it recomputes the prologue in
    // every lane, so with an RMSNorm prologue (three loads per activation) the batch-1 GEMV, which
    // stages it once per workgroup, is faster (16384 x 2048: 7.1 against 8.1 us)
    if (M == 1 && mode == cri::kActSwiGLU && K == 8192 && cri::detail::slice_gemv_supported(fmt, N, K, B))
        rc = cri::detail::launch_slice_gemv(mode, fmt, act, B, C, N, K, stream);
    if (rc == cri::detail::kDeclined && cri::detail::skinny_supported(fmt, M, K, B))
        rc = cri::detail::launch_skinny_act(mode, fmt, act, B, C, M, N, K, stream, ws, ws_floats, defer, defer_S);
    if (rc == cri::detail::kDeclined && mode == cri::kActSwiGLU2)
        return fail(CRI_ERR_UNSUPPORTED, fn, "the two-split SwiGLU prologue runs on the skinny kernel only");
    if (rc == cri::detail::kDeclined && M == 1 && cri::detail::gemv_supported(fmt, K, B))
        rc = cri::detail::launch_gemv_act(mode, fmt, act, B, C, N, K, stream);
    if (rc == cri::detail::kDeclined) rc = cri::detail::launch_generic_matmul_act(mode, fmt, act, B, C, M, N, K, stream);
    return finish_matmul(rc, fn);
}

}  // namespace

namespace {
int rmsnorm_impl(int format, const float* hidden, const float* residual, const float* norm_weight,
                 float* hidden_out, const void* B, float* C, int M, int N, int K, float eps, hipStream_t s,
                 const char* fn, float* ws, long ws_floats, cri::SplitSums* defer = nullptr, int defer_S = 0) {
    if (defer) defer->S = 0;
    if (M > 0 && N > 0 && K == 0) return fail(CRI_ERR_SHAPE, fn, "K=0: the RMS of an empty row is undefined");
    if (M > 0 && N > 0 && K > 0) {
        if (!hidden || !norm_weight) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null hidden or norm_weight");
        if (!aligned(hidden, 4) || !aligned(residual, 4) || !aligned(norm_weight, 4) || !aligned(hidden_out, 4))
            return fail(CRI_ERR_ALIGNMENT, fn, "hidden, residual, norm_weight and hidden_out must be 4-byte aligned");
        const long bytes = static_cast<long>(M) * K * 4;
        if (overlaps(hidden_out, bytes, hidden, bytes) || overlaps(hidden_out, bytes, residual, bytes))
            return fail(CRI_ERR_INVALID_ARGUMENT, fn,
                        "hidden_out overlaps hidden or residual (other workgroups still read them)");
    }
    const cri::ActIn act{hidden, residual, norm_weight, hidden_out, K, eps};
    return fused_matmul(cri::kActRMSNorm, format, act, B, C, M, N, K, s, fn, ws, ws_floats, defer, defer_S);
}
}  // namespace

int cri_matmul_rmsnorm(int format, const float* hidden, const float* residual, const float* norm_weight,
                       float* hidden_out, const void* B, float* C, int M, int N, int K, float eps, hipStream_t s) {
    return rmsnorm_impl(format, hidden, residual, norm_weight, hidden_out, B, C, M, N, K, eps, s,
                        "cri_matmul_rmsnorm", nullptr, 0);
}

namespace {
int swiglu_impl(int format, const float* gate, const float* up, int ld, const void* B, float* C, int M, int N, int K,
                hipStream_t s, const char* fn, float* ws, long ws_floats, cri::SplitSums* defer = nullptr,
                int defer_S = 0) {
    if (M > 0 && N > 0 && K > 0) {
        if (!gate || !up) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null gate or up");
        if (ld < K) return fail(CRI_ERR_SHAPE, fn, "ld=" + std::to_string(ld) + " is below K=" + std::to_string(K));
        if (!aligned(gate, 4) || !aligned(up, 4)) return fail(CRI_ERR_ALIGNMENT, fn, "gate and up must be 4-byte aligned");
    }
    const cri::ActIn act{gate, up, nullptr, nullptr, ld, 0.0f};
    return fused_matmul(cri::kActSwiGLU, format, act, B, C, M, N, K, s, fn, ws, ws_floats, defer, defer_S);
}
}  // namespace

int cri_matmul_swiglu(int format, const float* gate, const float* up, int ld, const void* B, float* C, int M, int N,
                      int K, hipStream_t s) {
    return swiglu_impl(format, gate, up, ld, B, C, M, N, K, s, "cri_matmul_swiglu", nullptr, 0);
}

int cri_rmsnorm_residual(const float* input, const float* residual, const float* weight, float* output,
                         float* normed, int rows, int n, float eps, hipStream_t s) {
    const char* fn = "cri_rmsnorm_residual";
    if (rows < 0 || n < 0) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "negative dimension");
    if (rows == 0) return CRI_OK;
    if (n == 0) return fail(CRI_ERR_SHAPE, fn, "n=0: the RMS of an empty row is undefined");
    if (!input || !weight || !output || !normed) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null pointer");
    if (!aligned(input, 4) || !aligned(residual, 4) || !aligned(weight, 4) || !aligned(output, 4) ||
        !aligned(normed, 4))
        return fail(CRI_ERR_ALIGNMENT, fn, "all buffers must be 4-byte aligned");
    clear_pending_error();
    cri::detail::launch_rmsnorm_residual(input, residual, weight, output, normed, rows, n, eps, s);
    return check_launch(fn);
}

int cri_silu_mul(const float* gate, const float* up, float* out, long long n, hipStream_t s) {
    const char* fn = "cri_silu_mul";
    if (n < 0) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "negative n");
    if (n == 0) return CRI_OK;
    if (!gate || !up || !out) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null pointer");
    if (!aligned(gate, 4) || !aligned(up, 4) || !aligned(out, 4))
        return fail(CRI_ERR_ALIGNMENT, fn, "all buffers must be 4-byte aligned");
    clear_pending_error();
    cri::detail::launch_silu_mul(gate, up, out, static_cast<long>(n), s);
    return check_launch(fn);
}

int cri_stream_read(const void* src, long long n_bytes, unsigned* sink, hipStream_t s) {
    const char* fn = "cri_stream_read";
    if (n_bytes < 0 || n_bytes % 16 != 0)
        return fail(CRI_ERR_INVALID_ARGUMENT, fn, "n_bytes must be a non-negative multiple of 16");
    if (n_bytes == 0) return CRI_OK;
    if (!src || !sink) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null pointer");
    if (!aligned(src, 16) || !aligned(sink, 4)) return fail(CRI_ERR_ALIGNMENT, fn, "src must be 16-byte aligned");
    clear_pending_error();
    if (cri::detail::launch_stream_read(src, n_bytes, sink, s) != 0) return fail(CRI_ERR_SHAPE, fn, "too large");
    return check_launch(fn);
}

int cri_timestamp(unsigned long long* dst, hipStream_t s) {
    const char* fn = "cri_timestamp";
    if (!dst) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null pointer");
    if (!aligned(dst, 8)) return fail(CRI_ERR_ALIGNMENT, fn, "dst must be 8-byte aligned");
    clear_pending_error();
    cri::detail::launch_timestamp(dst, s);
    return check_launch(fn);
}

int cri_stream_read_ex(const void* src, long long n_bytes, unsigned* sink, int loads_per_thread, int grid_blocks,
                       hipStream_t s) {
    const char* fn = "cri_stream_read_ex";
    if (n_bytes < 0 || n_bytes % 16 != 0)
        return fail(CRI_ERR_INVALID_ARGUMENT, fn, "n_bytes must be a non-negative multiple of 16");
    if (grid_blocks < 0) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "negative grid_blocks");
    if (n_bytes == 0) return CRI_OK;
    if (!src || !sink) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null pointer");
    if (!aligned(src, 16) || !aligned(sink, 4)) return fail(CRI_ERR_ALIGNMENT, fn, "src must be 16-byte aligned");
    clear_pending_error();
    if (cri::detail::launch_stream_read_ex(src, n_bytes, sink, loads_per_thread, grid_blocks, s) != 0)
        return fail(CRI_ERR_INVALID_ARGUMENT, fn, "loads_per_thread must be 1, 2, 4, 8 or 16");
    return check_launch(fn);
}

long long cri_fused_decode_attention_workspace_size(int n_heads, int n_kv_heads, int head_dim, int kv_len) {
    const char* fn = "cri_fused_decode_attention_workspace_size";
    if (n_heads < 0 || n_kv_heads < 0 || head_dim < 0 || kv_len < 0)
        return fail(CRI_ERR_INVALID_ARGUMENT, fn, "negative dimension");
    if (n_heads == 0 || head_dim == 0 || kv_len == 0) return 0;
    if (n_kv_heads == 0 || n_heads % n_kv_heads != 0)
        return fail(CRI_ERR_SHAPE, fn, "n_heads is not a multiple of n_kv_heads");
    return cri::detail::decode_attention_workspace_bytes(n_heads, n_kv_heads, head_dim, kv_len);
}

int cri_fused_decode_attention_ws(const float* Q, const float* K_cache, const float* V_cache, float* output,
                                  int n_heads, int n_kv_heads, int head_dim, int kv_len, float scale, void* workspace,
                                  long long workspace_bytes, hipStream_t s) {
    const char* fn = "cri_fused_decode_attention_ws";
    if (workspace_bytes < 0) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "negative workspace size");
    if (n_heads < 0 || n_kv_heads < 0 || head_dim < 0 || kv_len < 0 || n_heads == 0 || head_dim == 0 || kv_len == 0 ||
        n_kv_heads == 0 || n_heads % n_kv_heads != 0 || head_dim > cri::detail::kDecodeAttnMaxHeadDim || !Q ||
        !K_cache || !V_cache || !output ||
        !cri::detail::decode_attention_split_supported(Q, K_cache, V_cache, head_dim)) {
        // argument errors, or a shape the split kernel does not take: the workspace-free form
        const int rc = cri_fused_decode_attention(Q, K_cache, V_cache, output, n_heads, n_kv_heads, head_dim, kv_len,
                                                  scale, s);
        if (rc != CRI_OK) {
            const size_t colon = g_last_error.find(':');
            g_last_error = std::string(fn) + (colon == std::string::npos ? ": " + g_last_error : g_last_error.substr(colon));
        }
        return rc;
    }
    if (!aligned(output, 4)) return fail(CRI_ERR_ALIGNMENT, fn, "output must be 4-byte aligned");
    if (!workspace) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null workspace");
    if (!aligned(workspace, 16)) return fail(CRI_ERR_ALIGNMENT, fn, "workspace must be 16-byte aligned");
    if (static_cast<long>(kv_len) * n_kv_heads * head_dim > kMaxElems) return fail(CRI_ERR_SHAPE, fn, "problem too large");
    clear_pending_error();
    const int rc = cri::detail::launch_decode_attention_split(Q, K_cache, V_cache, output, n_heads, n_kv_heads,
                                                              head_dim, kv_len, scale, static_cast<float*>(workspace),
                                                              static_cast<long>(workspace_bytes), s);
    if (rc == -2)
        return fail(CRI_ERR_SHAPE, fn,
                    "workspace of " + std::to_string(workspace_bytes) + " bytes holds less than one record per head (" +
                        std::to_string(static_cast<long>(n_heads) * (head_dim + 4) * 4) + " bytes)");
    if (rc != 0) return fail(CRI_ERR_UNSUPPORTED, fn, "no kernel for this shape");
    return check_launch(fn);
}

namespace {
// workspace layout of cri_prefill_attention: the position (16 bytes), then q heads and output heads
// (n_heads x rows x head_dim each), K^T and V heads (n_kv_heads x T4 x head_dim each), scores
// (n_heads x rows x T4), for rows = min(M, kPromptRows) and T4 = kv_len rounded up to 4
struct PrefillWs {
    long qh, oh, kt, vh, sc, total;  // float offsets after the 16-byte position slot; total bytes
};
PrefillWs prefill_ws(int M, int H, int Hkv, int D, int kv_len) {
    const long rows = std::min(M, cri::detail::kPromptRows), T4 = (static_cast<long>(kv_len) + 3) / 4 * 4;
    PrefillWs w;
    w.qh = 0;
    w.oh = w.qh + H * rows * D;
    w.kt = w.oh + H * rows * D;
    w.vh = w.kt + Hkv * T4 * D;
    w.sc = w.vh + Hkv * T4 * D;
    w.total = 16 + 4 * (w.sc + H * rows * T4);
    return w;
}
}  // namespace

long long cri_prefill_attention_workspace_bytes(int M, int n_heads, int n_kv_heads, int head_dim, int kv_len) {
    if (M < 1 || n_heads < 1 || n_kv_heads < 1 || head_dim < 1 || kv_len < 1) return 0;
    return prefill_ws(M, n_heads, n_kv_heads, head_dim, kv_len).total;
}

int cri_prefill_attention(const float* Q, int ldq, const float* K_cache, const float* V_cache, float* output, int M,
                          int n_heads, int n_kv_heads, int head_dim, int pos, float scale, void* workspace,
                          long long workspace_bytes, hipStream_t s) {
    const char* fn = "cri_prefill_attention";
    if (M < 0 || n_heads < 0 || n_kv_heads < 0 || head_dim < 0 || pos < 0 || workspace_bytes < 0)
        return fail(CRI_ERR_INVALID_ARGUMENT, fn, "negative argument");
    if (M == 0 || n_heads == 0) return CRI_OK;
    if (n_kv_heads == 0 || n_heads % n_kv_heads != 0)
        return fail(CRI_ERR_INVALID_ARGUMENT, fn, "n_heads is not a multiple of n_kv_heads");
    if (head_dim % 4 != 0 || head_dim < 4 || head_dim > cri::detail::kDecodeAttnSplitMaxHeadDim)
        return fail(CRI_ERR_UNSUPPORTED, fn, "head_dim must be a multiple of 4 in [4, 128]");
    if (ldq < n_heads * head_dim || ldq % 4 != 0)
        return fail(CRI_ERR_SHAPE, fn, "ldq must be a multiple of 4 and at least n_heads * head_dim");
    if (!Q || !K_cache || !V_cache || !output || !workspace) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null pointer");
    if (!aligned(Q, 4) || !aligned(K_cache, 16) || !aligned(V_cache, 16) || !aligned(output, 16) ||
        !aligned(workspace, 16))
        return fail(CRI_ERR_ALIGNMENT, fn, "Q must be 4-byte aligned, K_cache, V_cache, output and workspace 16-byte");
    const long kv_len = static_cast<long>(pos) + M;
    if (kv_len * n_kv_heads * head_dim > kMaxElems || static_cast<long>(M) * ldq > kMaxElems)
        return fail(CRI_ERR_SHAPE, fn, "problem too large");
    const PrefillWs w = prefill_ws(M, n_heads, n_kv_heads, head_dim, static_cast<int>(kv_len));
    if (workspace_bytes < w.total)
        return fail(CRI_ERR_SHAPE, fn, "workspace of " + std::to_string(workspace_bytes) + " bytes, " +
                                           std::to_string(w.total) + " needed");
    clear_pending_error();
    int* pos_dev = static_cast<int*>(workspace);
    float* base = reinterpret_cast<float*>(static_cast<char*>(workspace) + 16);
    if (cri::detail::launch_pos_set(pos_dev, pos, s) != 0) return fail(CRI_ERR_LAUNCH, fn, "launch failed");
    const int QD = n_heads * head_dim;
    for (int m0 = 0; m0 < M; m0 += cri::detail::kPromptRows) {
        const int mb = std::min(cri::detail::kPromptRows, M - m0);
        const int T4 = (pos + m0 + mb + 3) / 4 * 4;
        const int rc = cri::detail::launch_prefill_attention(
            Q + static_cast<long>(m0) * ldq, ldq, K_cache, V_cache, output + static_cast<long>(m0) * QD, m0, mb,
            n_heads, n_kv_heads, head_dim, T4, pos_dev, scale, base + w.qh, base + w.kt, base + w.vh, base + w.sc,
            base + w.oh, s);
        if (rc != 0) return fail(CRI_ERR_UNSUPPORTED, fn, "no kernel for this shape");
    }
    return check_launch(fn);
}

int cri_fused_decode_attention_noalloc(const float* Q, const float* K_cache, const float* V_cache, float* output,
                                       int n_heads, int n_kv_heads, int head_dim, int kv_len, float scale,
                                       hipStream_t s) {
    const char* fn = "cri_fused_decode_attention_noalloc";
    if (n_heads < 0 || n_kv_heads < 0 || head_dim < 0 || kv_len < 0)
        return fail(CRI_ERR_INVALID_ARGUMENT, fn, "negative dimension");
    if (n_heads == 0 || head_dim == 0) return CRI_OK;
    if (n_kv_heads == 0 || n_heads % n_kv_heads != 0)
        return fail(CRI_ERR_SHAPE, fn, "n_heads is not a multiple of n_kv_heads");
    if (kv_len == 0) return fail(CRI_ERR_SHAPE, fn, "kv_len must be at least 1");
    if (!Q || !K_cache || !V_cache || !output) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null pointer");
    if (!cri::detail::decode_attention_split_supported(Q, K_cache, V_cache, head_dim))
        return fail(CRI_ERR_UNSUPPORTED, fn,
                    "needs 4 | head_dim <= " + std::to_string(cri::detail::kDecodeAttnSplitMaxHeadDim) +
                        " and 16-byte aligned Q, K_cache, V_cache");
    if (!aligned(output, 4)) return fail(CRI_ERR_ALIGNMENT, fn, "output must be 4-byte aligned");
    if (static_cast<long>(kv_len) * n_kv_heads * head_dim > kMaxElems) return fail(CRI_ERR_SHAPE, fn, "problem too large");
    const long rec = static_cast<long>(n_heads) * (head_dim + 4) * 4;
    if (rec > cri::detail::kNoallocScratchBytes)
        return fail(CRI_ERR_SHAPE, fn,
                    "one partial record per head needs " + std::to_string(rec) + " bytes, more than the " +
                        std::to_string(cri::detail::kNoallocScratchBytes) + "-byte static scratch");
    clear_pending_error();
    float* ws = nullptr;
    if (cri::detail::noalloc_scratch(&ws) != 0)
        return fail(CRI_ERR_LAUNCH, fn, "hipGetSymbolAddress of the static scratch failed");
    const int rc = cri::detail::launch_decode_attention_split(Q, K_cache, V_cache, output, n_heads, n_kv_heads,
                                                              head_dim, kv_len, scale, ws,
                                                              cri::detail::kNoallocScratchBytes, s);
    if (rc != 0) return fail(CRI_ERR_UNSUPPORTED, fn, "no kernel for this shape");
    return check_launch(fn);
}

int cri_embedding_rows(int format, const void* table, const int* ids, float* out, int n_ids, int dim, int vocab,
                       hipStream_t s) {
    const char* fn = "cri_embedding_rows";
    if (format < CRI_Q8_0 || format > CRI_FP32) return fail(CRI_ERR_UNSUPPORTED, fn, "unknown format id");
    if (n_ids < 0 || dim < 0 || vocab < 0) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "negative dimension");
    if (n_ids == 0 || dim == 0) return CRI_OK;
    if (dim % cri::block_elems(format) != 0)
        return fail(CRI_ERR_SHAPE, fn, "dim=" + std::to_string(dim) + " is not a multiple of the block size");
    if (!table || !ids || !out) return fail(CRI_ERR_INVALID_ARGUMENT, fn, "null pointer");
    if (!aligned(ids, 4) || !aligned(out, 4)) return fail(CRI_ERR_ALIGNMENT, fn, "ids and out must be 4-byte aligned");
    if ((format == CRI_FP16 && !aligned(table, 2)) || (format == CRI_FP32 && !aligned(table, 4)))
        return fail(CRI_ERR_ALIGNMENT, fn, "table misaligned for its element type");
    clear_pending_error();
    cri::detail::launch_embedding_rows(format, table, ids, out, n_ids, dim, vocab, s);
    return check_launch(fn);
}

const char* cri_last_error_string(void) { return g_last_error.c_str(); }

int cri_block_bytes(int format) { return format >= 0 && format <= 5 ? cri::block_bytes(format) : 0; }
int cri_block_elems(int format) { return format >= 0 && format <= 5 ? cri::block_elems(format) : 0; }
int cri_version(void) { return 100; }

}  // extern "C"

// In-library callers that own a workspace (the decode step): the same products, with the
// skinny kernel's split partial sums reduced in a fixed order (deterministic).
namespace cri {
namespace detail {
int matmul_split_ws(int fmt, const float* A, const void* B, float* C, int M, int N, int K, float* ws, long ws_floats,
                    hipStream_t s, SplitSums* defer, int defer_S) {
    return matmul_impl(fmt, A, B, C, M, N, K, s, "matmul (decode step)", ws, ws_floats, defer, defer_S);
}
int matmul_swiglu_split_ws(int fmt, const float* gate, const float* up, int ld, const void* B, float* C, int M, int N,
                           int K, float* ws, long ws_floats, hipStream_t s, SplitSums* defer, int defer_S) {
    return swiglu_impl(fmt, gate, up, ld, B, C, M, N, K, s, "matmul_swiglu (decode step)", ws, ws_floats, defer,
                       defer_S);
}
int matmul_rmsnorm_split_ws(int fmt, const float* hidden, const float* residual, const float* norm_weight,
                            float* hidden_out, const void* B, float* C, int M, int N, int K, float eps, float* ws,
                            long ws_floats, hipStream_t s, SplitSums* defer, int defer_S) {
    return rmsnorm_impl(fmt, hidden, residual, norm_weight, hidden_out, B, C, M, N, K, eps, s,
                        "matmul_rmsnorm (decode step)", ws, ws_floats, defer, defer_S);
}
int matmul_rmsnorm_splitres(int fmt, const float* hidden, const float* res_parts, int splits, long split,
                            const float* norm_weight, float* hidden_out, const void* B, float* C, int N, int K,
                            float eps, hipStream_t s) {
    const char* fn = "matmul_rmsnorm with a split residual (decode step)";
    if (splits < 1 || splits > kResMaxSplits || split < K || !hidden || !res_parts || !norm_weight)
        return fail(CRI_ERR_INVALID_ARGUMENT, fn, "bad residual partial sums");
    cri::ActIn act{hidden, res_parts, norm_weight, hidden_out, K, eps};
    act.split = split;
    act.kn = splits;
    return fused_matmul(cri::kActRMSNormS, fmt, act, B, C, 1, N, K, s, fn);
}
int matmul_swiglu2_split_ws(int fmt, const SplitSums& gu, long up_off, int ld, const void* B, float* C, int M, int N,
                            int K, float* ws, long ws_floats, hipStream_t s, SplitSums* defer, int defer_S) {
    const char* fn = "matmul_swiglu2 (decode step)";
    if ((gu.S != 1 && gu.S != 2) || !gu.part || ld < K || up_off < K)
        return fail(CRI_ERR_INVALID_ARGUMENT, fn, "expects one or two partial sums of a gate/up matmul");
    cri::ActIn act{gu.part, gu.part + up_off, gu.ssq, nullptr, ld, gu.eps};
    act.split = gu.S == 2 ? gu.stride : 0;
    act.nss = gu.nss ? gu.nss : gu.S;
    if (act.nss < 1 || act.nss > cri::kResMaxSplits)
        return fail(CRI_ERR_INVALID_ARGUMENT, fn, "up to four sums of squares per row");
    act.kn = gu.K;
    return fused_matmul(cri::kActSwiGLU2, fmt, act, B, C, M, N, K, s, fn, ws, ws_floats, defer, defer_S);
}
}  // namespace detail
}  // namespace cri

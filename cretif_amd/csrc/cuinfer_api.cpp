// cuinfer_api.cpp -- the reference's C++ entry points on top of the C ABI.
//
// Each wrapper forwards to its cri_* function and throws std::runtime_error
// on a non-zero status, which is how the reference reports errors
// (CUINFER_CHECK_CUDA, ref:include/cuinfer/cuda_utils.h:12-20).
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <stdexcept>
#include <string>
#include <utility>

#include "../../include/cri.h"
#include "../../include/cuinfer/attention.h"
#include "../../include/cuinfer/dispatch.h"
#include "../../include/cuinfer/embedding.h"
#include "../../include/cuinfer/hip_utils.h"
#include "../../include/cuinfer/kernels/elementwise.h"
#include "../../include/cuinfer/kernels/matmul_quant.h"
#include "../../include/cuinfer/quantization.h"
#include "../../include/cuinfer/tensor.h"

namespace cuinfer {

void matmul_q8_0(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t s) {
    CUINFER_CHECK_CRI(cri_matmul_q8_0(A, B, C, M, N, K, s));
}
void matmul_q4_0(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t s) {
    CUINFER_CHECK_CRI(cri_matmul_q4_0(A, B, C, M, N, K, s));
}
void matmul_q5_0(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t s) {
    CUINFER_CHECK_CRI(cri_matmul_q5_0(A, B, C, M, N, K, s));
}
void matmul_q4_k(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t s) {
    CUINFER_CHECK_CRI(cri_matmul_q4_k(A, B, C, M, N, K, s));
}
void matmul_q6_k(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t s) {
    CUINFER_CHECK_CRI(cri_matmul_q6_k(A, B, C, M, N, K, s));
}
void matmul_fp16(const float* A, const void* B, float* C, int M, int N, int K, hipStream_t s) {
    CUINFER_CHECK_CRI(cri_matmul_fp16(A, B, C, M, N, K, s));
}

void dequantize_q8_0(const void* src, float* dst, int n, hipStream_t s) {
    CUINFER_CHECK_CRI(cri_dequantize_q8_0(src, dst, n, s));
}
void dequantize_q4_0(const void* src, float* dst, int n, hipStream_t s) {
    CUINFER_CHECK_CRI(cri_dequantize_q4_0(src, dst, n, s));
}
void dequantize_q5_0(const void* src, float* dst, int n, hipStream_t s) {
    CUINFER_CHECK_CRI(cri_dequantize_q5_0(src, dst, n, s));
}
void dequantize_q6_k(const void* src, float* dst, int n, hipStream_t s) {
    CUINFER_CHECK_CRI(cri_dequantize_q6_k(src, dst, n, s));
}
void dequantize_q4_k(const void* src, float* dst, int n, hipStream_t s) {
    CUINFER_CHECK_CRI(cri_dequantize_q4_k(src, dst, n, s));
}

void matmul_transposed_b(const float* A, const float* B, float* C, int M, int N, int K, hipStream_t s) {
    CUINFER_CHECK_CRI(cri_matmul_transposed_b(A, B, C, M, N, K, s));
}

void batched_matmul_gqa(const float* A, const float* B, float* C, int n_heads, int n_kv_heads, int M, int N, int K,
                        hipStream_t s) {
    CUINFER_CHECK_CRI(cri_batched_matmul_gqa(A, B, C, n_heads, n_kv_heads, M, N, K, s));
}

void fused_decode_attention(const float* Q, const float* K_cache, const float* V_cache, float* output, int n_heads,
                            int n_kv_heads, int head_dim, int kv_len, float scale, hipStream_t s) {
    CUINFER_CHECK_CRI(cri_fused_decode_attention(Q, K_cache, V_cache, output, n_heads, n_kv_heads, head_dim, kv_len,
                                                 scale, s));
}

void prefill_attention(const float* Q, int ldq, const float* K_cache, const float* V_cache, float* output, int M,
                       int n_heads, int n_kv_heads, int head_dim, int pos, float scale, hipStream_t stream) {
    const long long bytes = cri_prefill_attention_workspace_bytes(M, n_heads, n_kv_heads, head_dim, pos + M);
    Tensor ws = Tensor::empty({std::max<int64_t>(1, (bytes + 3) / 4)});
    CUINFER_CHECK_CRI(cri_prefill_attention(Q, ldq, K_cache, V_cache, output, M, n_heads, n_kv_heads, head_dim, pos,
                                            scale, ws.data(), bytes, stream));
    // the workspace is released when this returns: wait for the kernels that use it
    CUINFER_CHECK_HIP(hipStreamSynchronize(stream));
}

// ---------------------------------------------------------------- dispatch
const char* weight_format_name(WeightFormat fmt) {
    switch (fmt) {
        case WeightFormat::FP32: return "FP32";
        case WeightFormat::FP16: return "FP16";
        case WeightFormat::Q8_0: return "Q8_0";
        case WeightFormat::Q4_0: return "Q4_0";
        case WeightFormat::Q5_0: return "Q5_0";
        case WeightFormat::Q4_K: return "Q4_K";
        case WeightFormat::Q6_K: return "Q6_K";
    }
    return "UNKNOWN";
}

WeightFormat weight_format_of(DType dtype) {
    switch (dtype) {
        case DType::FP16: return WeightFormat::FP16;
        case DType::Q8_0: return WeightFormat::Q8_0;
        case DType::Q4_0: return WeightFormat::Q4_0;
        case DType::Q5_0: return WeightFormat::Q5_0;
        case DType::Q4_K: return WeightFormat::Q4_K;
        case DType::Q6_K: return WeightFormat::Q6_K;
        default: return WeightFormat::FP32;
    }
}

static int format_id(WeightFormat format, const char* fn) {
    switch (format) {
        case WeightFormat::FP16: return CRI_FP16;
        case WeightFormat::Q8_0: return CRI_Q8_0;
        case WeightFormat::Q4_0: return CRI_Q4_0;
        case WeightFormat::Q5_0: return CRI_Q5_0;
        case WeightFormat::Q4_K: return CRI_Q4_K;
        case WeightFormat::Q6_K: return CRI_Q6_K;
        default: break;
    }
    throw std::invalid_argument(std::string(fn) + ": FP32 weights ([K,N] pre-transposed) are not handled here");
}

// The matmuls read the weight as N rows of K/bs consecutive blocks from weight.data(): a strided
// view (for example a column slice of a quantized tensor) or a tensor holding fewer than N*K
// elements would be read wrongly or past its end, so both are rejected before anything runs.
static void check_weight(const Tensor& weight, int N, int K, const char* fn) {
    if (!weight.is_contiguous())
        throw std::invalid_argument(std::string(fn) + ": the weight tensor is a strided view; the matmul reads "
                                    "N x K contiguous elements");
    if (weight.dtype() != DType::FP32 && N > 0 && K > 0 &&
        weight.numel() < static_cast<int64_t>(N) * static_cast<int64_t>(K))
        throw std::invalid_argument(std::string(fn) + ": the weight tensor holds " + std::to_string(weight.numel()) +
                                    " elements, fewer than N x K = " +
                                    std::to_string(static_cast<int64_t>(N) * K));
}

void matmul_dispatch(const float* A, const Tensor& weight, float* C, int M, int N, int K, WeightFormat format,
                     hipStream_t s) {
    check_weight(weight, N, K, "matmul_dispatch");
    CUINFER_CHECK_CRI(cri_matmul(format_id(format, "matmul_dispatch"), A, weight.data(), C, M, N, K, s));
}

void matmul_dispatch_rmsnorm(const float* hidden, const float* residual, const float* norm_weight, float* hidden_out,
                             const Tensor& weight, float* C, int M, int N, int K, WeightFormat format, float eps,
                             hipStream_t s) {
    check_weight(weight, N, K, "matmul_dispatch_rmsnorm");
    CUINFER_CHECK_CRI(cri_matmul_rmsnorm(format_id(format, "matmul_dispatch_rmsnorm"), hidden, residual, norm_weight,
                                         hidden_out, weight.data(), C, M, N, K, eps, s));
}

void matmul_dispatch_swiglu(const float* gate, const float* up, int ld, const Tensor& weight, float* C, int M, int N,
                            int K, WeightFormat format, hipStream_t s) {
    check_weight(weight, N, K, "matmul_dispatch_swiglu");
    CUINFER_CHECK_CRI(cri_matmul_swiglu(format_id(format, "matmul_dispatch_swiglu"), gate, up, ld, weight.data(), C,
                                        M, N, K, s));
}

void rmsnorm_residual(const float* input, const float* residual, const float* weight, float* output, float* normed,
                      int rows, int n, float eps, hipStream_t s) {
    CUINFER_CHECK_CRI(cri_rmsnorm_residual(input, residual, weight, output, normed, rows, n, eps, s));
}

void silu_mul(const float* gate, const float* up, float* out, long long n, hipStream_t s) {
    CUINFER_CHECK_CRI(cri_silu_mul(gate, up, out, n, s));
}

// ---------------------------------------------------------------- Tensor
void Tensor::compute_shape_and_stride(const std::vector<int64_t>& shape, std::array<int64_t, 4>& out_shape,
                                      std::array<int64_t, 4>& out_stride) {
    if (shape.empty() || shape.size() > 4)
        throw std::invalid_argument("Tensor shape must have 1-4 dimensions, got " + std::to_string(shape.size()));
    out_shape.fill(1);
    const int off = 4 - static_cast<int>(shape.size());
    for (size_t i = 0; i < shape.size(); ++i) {
        if (shape[i] <= 0) throw std::invalid_argument("Tensor: dimensions must be positive");
        out_shape[off + i] = shape[i];
    }
    int64_t n = 1;
    for (int64_t d : out_shape)
        if (__builtin_mul_overflow(n, d, &n)) throw std::invalid_argument("Tensor: element count overflows int64");
    out_stride[3] = 1;
    for (int i = 2; i >= 0; --i) out_stride[i] = out_stride[i + 1] * out_shape[i + 1];
}

Tensor::Tensor() = default;

Tensor::Tensor(std::vector<int64_t> shape, DType dtype) : dtype_(dtype), owning_(true) {
    compute_shape_and_stride(shape, shape_, stride_);
    if (dtype_is_quantized(dtype) && shape_[3] % dtype_block_elements(dtype) != 0)
        throw std::invalid_argument(std::string("Tensor: innermost dimension is not a multiple of the ") +
                                    dtype_name(dtype) + " block size");
    const size_t bytes = size_bytes();
    if (bytes > 0) CUINFER_CHECK_HIP(hipMalloc(&data_, bytes));
}

Tensor::Tensor(void* data, std::array<int64_t, 4> shape, std::array<int64_t, 4> stride, DType dtype)
    : data_(data), shape_(shape), stride_(stride), dtype_(dtype), owning_(false) {}

Tensor::~Tensor() {
    if (owning_ && data_) (void)hipFree(data_);
    data_ = nullptr;
}

Tensor::Tensor(Tensor&& o) noexcept
    : data_(o.data_), shape_(o.shape_), stride_(o.stride_), dtype_(o.dtype_), owning_(o.owning_) {
    // the moved-from tensor is empty: no data, every dimension 1 (ref:src/tensor.cu:69-100)
    o.data_ = nullptr;
    o.shape_.fill(1);
    o.stride_.fill(1);
    o.owning_ = false;
}

Tensor& Tensor::operator=(Tensor&& o) noexcept {
    if (this != &o) {
        if (owning_ && data_) (void)hipFree(data_);
        data_ = o.data_;
        shape_ = o.shape_;
        stride_ = o.stride_;
        dtype_ = o.dtype_;
        owning_ = o.owning_;
        o.data_ = nullptr;
        o.shape_.fill(1);
        o.stride_.fill(1);
        o.owning_ = false;
    }
    return *this;
}

Tensor Tensor::from_host(const void* host, std::vector<int64_t> shape, DType dtype) {
    Tensor t(std::move(shape), dtype);
    t.copy_from_host(host, t.size_bytes());
    return t;
}

Tensor Tensor::zeros(std::vector<int64_t> shape, DType dtype) {
    Tensor t(std::move(shape), dtype);
    if (t.size_bytes()) CUINFER_CHECK_HIP(hipMemset(t.data_, 0, t.size_bytes()));
    return t;
}

Tensor Tensor::empty(std::vector<int64_t> shape, DType dtype) { return Tensor(std::move(shape), dtype); }

Tensor Tensor::view(int64_t dim, int64_t start, int64_t end) const {
    if (dim < 0 || dim >= 4) throw std::out_of_range("view(): dim must be in [0, 3]");
    if (start < 0 || end > shape_[dim] || start >= end) throw std::out_of_range("view(): invalid range");
    size_t byte_offset;
    if (dtype_is_quantized(dtype_)) {
        const int64_t elems = start * stride_[dim];
        const int be = dtype_block_elements(dtype_);
        if (elems % be != 0 || (dim == 3 && ((end - start) % be != 0)))
            throw std::invalid_argument("view(): quantised slice must fall on block boundaries");
        byte_offset = static_cast<size_t>(elems / be) * dtype_block_bytes(dtype_);
    } else {
        byte_offset = static_cast<size_t>(start * stride_[dim]) * dtype_size(dtype_);
    }
    auto ns = shape_;
    ns[dim] = end - start;
    return Tensor(static_cast<char*>(data_) + byte_offset, ns, stride_, dtype_);
}

Tensor Tensor::reshape(std::vector<int64_t> new_shape) const {
    if (!is_contiguous()) throw std::runtime_error("reshape(): tensor must be contiguous");
    if (new_shape.empty() || new_shape.size() > 4)
        throw std::invalid_argument("reshape(): shape must have 1-4 dimensions, got " +
                                    std::to_string(new_shape.size()));
    std::array<int64_t, 4> s, st;
    compute_shape_and_stride(new_shape, s, st);
    if (s[0] * s[1] * s[2] * s[3] != numel()) throw std::invalid_argument("reshape(): element count mismatch");
    return Tensor(data_, s, st, dtype_);
}

Tensor Tensor::clone() const {
    if (!is_contiguous()) throw std::runtime_error("clone(): tensor must be contiguous");
    std::vector<int64_t> s(shape_.begin(), shape_.end());
    Tensor t(s, dtype_);
    if (size_bytes()) CUINFER_CHECK_HIP(hipMemcpy(t.data_, data_, size_bytes(), hipMemcpyDeviceToDevice));
    return t;
}

void Tensor::copy_from_host(const void* host, size_t bytes) {
    if (bytes > size_bytes()) throw std::invalid_argument("copy_from_host(): more bytes than the tensor holds");
    if (bytes) CUINFER_CHECK_HIP(hipMemcpy(data_, host, bytes, hipMemcpyHostToDevice));
}

void Tensor::copy_to_host(void* host, size_t bytes) const {
    if (bytes > size_bytes()) throw std::invalid_argument("copy_to_host(): more bytes than the tensor holds");
    if (bytes) CUINFER_CHECK_HIP(hipMemcpy(host, data_, bytes, hipMemcpyDeviceToHost));
}

int64_t Tensor::numel() const { return shape_[0] * shape_[1] * shape_[2] * shape_[3]; }

size_t Tensor::size_bytes() const {
    if (dtype_is_quantized(dtype_))
        return static_cast<size_t>(numel() / dtype_block_elements(dtype_)) * dtype_block_bytes(dtype_);
    return static_cast<size_t>(numel()) * dtype_size(dtype_);
}

int Tensor::ndim() const {
    int lead = 0;
    while (lead < 3 && shape_[lead] == 1) ++lead;
    return 4 - lead;
}

bool Tensor::is_contiguous() const {
    int64_t expect = 1;
    for (int i = 3; i >= 0; --i) {
        if (shape_[i] != 1 && stride_[i] != expect) return false;
        expect *= shape_[i];
    }
    return true;
}

int64_t Tensor::shape(int dim) const {
    if (dim < 0 || dim >= 4) throw std::out_of_range("shape(): dim out of range");
    return shape_[dim];
}

int64_t Tensor::stride(int dim) const {
    if (dim < 0 || dim >= 4) throw std::out_of_range("stride(): dim out of range");
    return stride_[dim];
}

}  // namespace cuinfer

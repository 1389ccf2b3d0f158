// tensor.h -- device tensor with GGUF block-aware sizes.
//
// Keeps the reference's DType enum, helpers and Tensor interface
// (ref:include/cuinfer/tensor.h:14-231) so weights uploaded by existing call
// sites can be handed to the matmul entry points unchanged.  One deliberate
// difference: view() on a quantised tensor slices whole rows by bytes
// (the reference computes a zero offset there, ref:src/tensor.cu:152-155),
// and rejects slices that do not fall on block boundaries.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace cuinfer {

enum class DType { FP32, FP16, INT8, Q8_0, Q4_0, Q5_0, Q4_K, Q6_K };

inline size_t dtype_size(DType d) {
    switch (d) {
        case DType::FP32: return 4;
        case DType::FP16: return 2;
        case DType::INT8: return 1;
        default: return 0;  // block-quantised: use dtype_block_bytes / dtype_block_elements
    }
}
inline bool dtype_is_quantized(DType d) {
    return d == DType::Q8_0 || d == DType::Q4_0 || d == DType::Q5_0 || d == DType::Q4_K || d == DType::Q6_K;
}
inline int dtype_block_elements(DType d) {
    switch (d) {
        case DType::Q8_0: case DType::Q4_0: case DType::Q5_0: return 32;
        case DType::Q4_K: case DType::Q6_K: return 256;
        default: return 1;
    }
}
inline size_t dtype_block_bytes(DType d) {
    switch (d) {
        case DType::FP32: return 4;
        case DType::FP16: return 2;
        case DType::INT8: return 1;
        case DType::Q8_0: return 34;
        case DType::Q4_0: return 18;
        case DType::Q5_0: return 22;
        case DType::Q4_K: return 144;
        case DType::Q6_K: return 210;
    }
    return 0;
}
inline const char* dtype_name(DType d) {
    switch (d) {
        case DType::FP32: return "FP32";
        case DType::FP16: return "FP16";
        case DType::INT8: return "INT8";
        case DType::Q8_0: return "Q8_0";
        case DType::Q4_0: return "Q4_0";
        case DType::Q5_0: return "Q5_0";
        case DType::Q4_K: return "Q4_K";
        case DType::Q6_K: return "Q6_K";
    }
    return "UNKNOWN";
}

// Move-only RAII device buffer with a right-aligned 4-D shape.
class Tensor {
public:
    Tensor();
    explicit Tensor(std::vector<int64_t> shape, DType dtype = DType::FP32);
    ~Tensor();
    Tensor(Tensor&& other) noexcept;
    Tensor& operator=(Tensor&& other) noexcept;
    Tensor(const Tensor&) = delete;
    Tensor& operator=(const Tensor&) = delete;

    static Tensor from_host(const void* host_data, std::vector<int64_t> shape, DType dtype = DType::FP32);
    static Tensor zeros(std::vector<int64_t> shape, DType dtype = DType::FP32);
    static Tensor empty(std::vector<int64_t> shape, DType dtype = DType::FP32);

    Tensor view(int64_t dim, int64_t start, int64_t end) const;
    Tensor reshape(std::vector<int64_t> new_shape) const;
    Tensor clone() const;
    void copy_from_host(const void* host_data, size_t bytes);
    void copy_to_host(void* host_data, size_t bytes) const;

    int64_t numel() const;
    size_t size_bytes() const;
    int ndim() const;
    bool is_contiguous() const;

    void* data() { return data_; }
    const void* data() const { return data_; }
    template <typename T>
    T* data_as() { return static_cast<T*>(data_); }
    template <typename T>
    const T* data_as() const { return static_cast<const T*>(data_); }

    const std::array<int64_t, 4>& shape() const { return shape_; }
    const std::array<int64_t, 4>& stride() const { return stride_; }
    int64_t shape(int dim) const;
    int64_t stride(int dim) const;
    DType dtype() const { return dtype_; }
    bool is_owning() const { return owning_; }

private:
    Tensor(void* data, std::array<int64_t, 4> shape, std::array<int64_t, 4> stride, DType dtype);
    static void compute_shape_and_stride(const std::vector<int64_t>& shape, std::array<int64_t, 4>& out_shape,
                                         std::array<int64_t, 4>& out_stride);
    void* data_ = nullptr;
    std::array<int64_t, 4> shape_ = {1, 1, 1, 1};
    std::array<int64_t, 4> stride_ = {1, 1, 1, 1};
    DType dtype_ = DType::FP32;
    bool owning_ = false;
};

}  // namespace cuinfer

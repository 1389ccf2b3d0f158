// C++ host check of cuinfer::Tensor, the drop-in for the reference's Tensor
// (ref:include/cuinfer/tensor.h, ref:src/tensor.cu), following the reference's
// own test list (ref:tests/test_tensor.cu:12-230: create and shape, host round
// trip, zeros, clone, move semantics, view, reshape, dtypes) plus the error
// behaviour of shapes, views and reshapes.  Built and run by
// tests/test_tensor_cpp.py.  Test infrastructure only.
//
//   tensor_check cpu   checks that allocate no device memory; prints "ok"
//   tensor_check gpu   the reference's list on device tensors; prints "ok"
#include <cmath>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "cuinfer/dispatch.h"
#include "cuinfer/tensor.h"

using cuinfer::DType;
using cuinfer::Tensor;

static int g_failures = 0;

#define CHECK(c)                                                                \
    do {                                                                        \
        if (!(c)) {                                                             \
            std::fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
            ++g_failures;                                                       \
        }                                                                       \
    } while (0)

template <class E, class F>
static bool throws(F&& f) {
    try {
        f();
    } catch (const E&) {
        return true;
    } catch (...) {
        return false;
    }
    return false;
}

// ---------------------------------------------------------------- no device memory
static void cpu_checks() {
    // a default tensor: no data, every dimension 1
    Tensor t;
    CHECK(t.data() == nullptr);
    CHECK(!t.is_owning());
    CHECK(t.numel() == 1);
    CHECK(t.ndim() == 1);
    CHECK(t.is_contiguous());

    // shapes: 1-4 positive dimensions whose product fits int64
    CHECK(throws<std::invalid_argument>([] { Tensor x(std::vector<int64_t>{}); }));
    CHECK(throws<std::invalid_argument>([] { Tensor x({1, 1, 1, 1, 1}); }));
    CHECK(throws<std::invalid_argument>([] { Tensor x({4, 0}); }));
    CHECK(throws<std::invalid_argument>([] { Tensor x({-2, 8}); }));
    CHECK(throws<std::invalid_argument>([] { Tensor x({int64_t(1) << 40, int64_t(1) << 40}); }));
    // a quantized innermost dimension is whole blocks
    CHECK(throws<std::invalid_argument>([] { Tensor x({2, 48}, DType::Q8_0); }));
    CHECK(throws<std::invalid_argument>([] { Tensor x({2, 512 + 32}, DType::Q4_K); }));

    // reshape: 1-4 dimensions, same element count (ref:src/tensor.cu:170-173)
    CHECK(throws<std::invalid_argument>([&] { (void)t.reshape({1, 1, 1, 1, 1}); }));
    CHECK(throws<std::invalid_argument>([&] { (void)t.reshape(std::vector<int64_t>{}); }));
    CHECK(throws<std::invalid_argument>([&] { (void)t.reshape({2}); }));
    Tensor r = t.reshape({1, 1});
    CHECK(r.numel() == 1 && !r.is_owning());

    // view and accessor ranges
    CHECK(throws<std::out_of_range>([&] { (void)t.view(4, 0, 1); }));
    CHECK(throws<std::out_of_range>([&] { (void)t.view(-1, 0, 1); }));
    CHECK(throws<std::out_of_range>([&] { (void)t.view(3, 0, 2); }));
    CHECK(throws<std::out_of_range>([&] { (void)t.view(3, 1, 1); }));
    CHECK(throws<std::out_of_range>([&] { (void)t.shape(4); }));
    CHECK(throws<std::out_of_range>([&] { (void)t.stride(-1); }));

    // moving a default tensor leaves both empty
    Tensor m(std::move(t));
    CHECK(m.data() == nullptr && t.data() == nullptr && t.numel() == 1);

    // dtype tables (ref:include/cuinfer/quantization.h block layouts)
    CHECK(cuinfer::dtype_size(DType::FP32) == 4 && cuinfer::dtype_size(DType::FP16) == 2 &&
          cuinfer::dtype_size(DType::INT8) == 1);
    CHECK(cuinfer::dtype_block_bytes(DType::Q8_0) == 34 && cuinfer::dtype_block_elements(DType::Q8_0) == 32);
    CHECK(cuinfer::dtype_block_bytes(DType::Q4_0) == 18 && cuinfer::dtype_block_elements(DType::Q4_0) == 32);
    CHECK(cuinfer::dtype_block_bytes(DType::Q5_0) == 22 && cuinfer::dtype_block_elements(DType::Q5_0) == 32);
    CHECK(cuinfer::dtype_block_bytes(DType::Q4_K) == 144 && cuinfer::dtype_block_elements(DType::Q4_K) == 256);
    CHECK(cuinfer::dtype_block_bytes(DType::Q6_K) == 210 && cuinfer::dtype_block_elements(DType::Q6_K) == 256);
    CHECK(!cuinfer::dtype_is_quantized(DType::FP16) && cuinfer::dtype_is_quantized(DType::Q6_K));
    CHECK(std::string(cuinfer::dtype_name(DType::Q4_K)) == "Q4_K");
}

// ---------------------------------------------------------------- device tensors
static std::vector<float> iota(int n) {
    std::vector<float> v(n);
    for (int i = 0; i < n; ++i) v[i] = static_cast<float>(i);
    return v;
}

static void gpu_checks() {
    {  // CreateAndShape (ref:tests/test_tensor.cu:12-36)
        Tensor t({32, 768});
        CHECK(t.shape(0) == 1 && t.shape(1) == 1 && t.shape(2) == 32 && t.shape(3) == 768);
        CHECK(t.numel() == 32 * 768);
        CHECK(t.size_bytes() == 32 * 768 * sizeof(float));
        CHECK(t.ndim() == 2);
        CHECK(t.dtype() == DType::FP32);
        CHECK(t.is_owning() && t.is_contiguous() && t.data() != nullptr);
        CHECK(t.stride(3) == 1 && t.stride(2) == 768 && t.stride(1) == 32 * 768 && t.stride(0) == 32 * 768);
    }
    {  // HostRoundtrip
        const std::vector<float> src = iota(1000);
        Tensor t = Tensor::from_host(src.data(), {10, 100});
        std::vector<float> dst(1000, -1.0f);
        t.copy_to_host(dst.data(), t.size_bytes());
        CHECK(dst == src);
        CHECK(throws<std::invalid_argument>([&] { t.copy_to_host(dst.data(), t.size_bytes() + 4); }));
        CHECK(throws<std::invalid_argument>([&] { t.copy_from_host(src.data(), t.size_bytes() + 4); }));
    }
    {  // Zeros
        Tensor t = Tensor::zeros({3, 5, 7});
        std::vector<float> h(3 * 5 * 7, 1.0f);
        t.copy_to_host(h.data(), t.size_bytes());
        for (float v : h) CHECK(v == 0.0f);
    }
    {  // Clone: a deep copy
        const std::vector<float> src = iota(64);
        Tensor a = Tensor::from_host(src.data(), {8, 8});
        Tensor b = a.clone();
        CHECK(b.is_owning() && b.data() != a.data() && b.numel() == a.numel() && b.dtype() == a.dtype());
        std::vector<float> zero(64, 0.0f), hb(64), ha(64);
        a.copy_from_host(zero.data(), a.size_bytes());  // the clone keeps its own values
        b.copy_to_host(hb.data(), b.size_bytes());
        a.copy_to_host(ha.data(), a.size_bytes());
        CHECK(hb == src && ha == zero);
    }
    {  // MoveSemantics (ref:tests/test_tensor.cu:105-124)
        Tensor original({4, 16});
        void* p = original.data();
        const int64_t n = original.numel();
        Tensor moved(std::move(original));
        CHECK(moved.data() == p && moved.numel() == n && moved.is_owning());
        CHECK(original.data() == nullptr && !original.is_owning() && original.numel() == 1);
        Tensor assigned;
        assigned = std::move(moved);
        CHECK(assigned.data() == p && assigned.numel() == n && assigned.is_owning());
        CHECK(moved.data() == nullptr && !moved.is_owning() && moved.numel() == 1);
    }
    {  // View (ref:tests/test_tensor.cu:128-161)
        const std::vector<float> src = iota(32);
        Tensor t = Tensor::from_host(src.data(), {4, 8});
        Tensor v = t.view(2, 1, 3);
        CHECK(!v.is_owning() && v.shape(2) == 2 && v.shape(3) == 8 && v.numel() == 16);
        CHECK(static_cast<const char*>(v.data()) - static_cast<const char*>(t.data()) == 8 * 4);
        CHECK(v.is_contiguous());
        std::vector<float> h(16);
        v.copy_to_host(h.data(), v.size_bytes());
        for (int i = 0; i < 16; ++i) CHECK(h[i] == src[8 + i]);
        // a slice of the innermost dimension is a strided view: not contiguous, no reshape
        Tensor c = t.view(3, 2, 6);
        CHECK(!c.is_contiguous() && c.numel() == 16);
        CHECK(throws<std::runtime_error>([&] { (void)c.reshape({16}); }));
        CHECK(throws<std::runtime_error>([&] { (void)c.clone(); }));
    }
    {  // Quantized views: whole blocks; row slices stay contiguous, column slices do not
        Tensor q({4, 256}, DType::Q4_K);
        CHECK(q.size_bytes() == 4 * 144);
        Tensor rows = q.view(2, 1, 3);
        CHECK(rows.is_contiguous() && rows.size_bytes() == 2 * 144);
        CHECK(static_cast<const char*>(rows.data()) - static_cast<const char*>(q.data()) == 144);
        Tensor q8({4, 64}, DType::Q8_0);
        CHECK(throws<std::invalid_argument>([&] { (void)q8.view(3, 0, 16); }));
        Tensor half = q8.view(3, 32, 64);
        CHECK(!half.is_contiguous());
        CHECK(static_cast<const char*>(half.data()) - static_cast<const char*>(q8.data()) == 34);
        // the matmul reads whole contiguous rows: a column slice or a short tensor is refused
        float* dummy = nullptr;
        CHECK(throws<std::invalid_argument>([&] {
            cuinfer::matmul_dispatch(dummy, half, dummy, 1, 4, 32, cuinfer::WeightFormat::Q8_0);
        }));
        CHECK(throws<std::invalid_argument>([&] {
            cuinfer::matmul_dispatch(dummy, q8, dummy, 1, 8, 64, cuinfer::WeightFormat::Q8_0);
        }));
    }
    {  // Reshape (ref:tests/test_tensor.cu:165-198)
        const std::vector<float> src = iota(32);
        Tensor t = Tensor::from_host(src.data(), {4, 8});
        Tensor flat = t.reshape({32});
        CHECK(flat.numel() == 32 && flat.shape(3) == 32 && !flat.is_owning() && flat.data() == t.data());
        std::vector<float> h(32);
        flat.copy_to_host(h.data(), flat.size_bytes());
        CHECK(h == src);
        Tensor r3 = t.reshape({2, 2, 8});
        CHECK(r3.numel() == 32 && r3.shape(1) == 2 && r3.shape(2) == 2 && r3.shape(3) == 8);
        CHECK(throws<std::invalid_argument>([&] { (void)t.reshape({5, 8}); }));
        CHECK(throws<std::invalid_argument>([&] { (void)t.reshape({1, 1, 1, 4, 8}); }));
    }
    {  // DTypes (ref:tests/test_tensor.cu:200-230)
        const int N = 1024;
        Tensor fp16({N}, DType::FP16);
        CHECK(fp16.dtype() == DType::FP16 && fp16.size_bytes() == N * 2 && fp16.numel() == N && fp16.is_owning());
        Tensor i8({N}, DType::INT8);
        CHECK(i8.dtype() == DType::INT8 && i8.size_bytes() == N && i8.numel() == N && i8.is_owning());
        Tensor q6({3, 512}, DType::Q6_K);
        CHECK(q6.size_bytes() == 3 * 2 * 210 && q6.numel() == 3 * 512);
    }
}

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "cpu";
    try {
        cpu_checks();
        if (mode == "gpu") gpu_checks();
    } catch (const std::exception& e) {
        std::fprintf(stderr, "unexpected exception: %s\n", e.what());
        return 1;
    }
    if (g_failures) return 1;
    std::printf("ok\n");
    return 0;
}

// C++ host check of the reference-shaped API (cuinfer::GGUFParser,
// load_weight_quantized, load_lm_head, matmul_dispatch, embedding_lookup),
// built and run by tests/test_gguf_cpp.py.  Test infrastructure only.
//
//   gguf_api_check FILE                 parser checks (no GPU); prints "ok"
//   gguf_api_check FILE --gpu OUT X IDS   also: lm_head(x) and the embedding rows
//                                       of IDS, written to OUT as raw fp32
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "cuinfer/dispatch.h"
#include "cuinfer/gguf_parser.h"
#include "cuinfer/hip_utils.h"
#include "cuinfer/weights.h"

#define CHECK(c)                                                           \
    do {                                                                   \
        if (!(c)) {                                                        \
            std::fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
            return 1;                                                      \
        }                                                                  \
    } while (0)

template <class F>
static bool throws(F&& f) {
    try {
        f();
    } catch (const std::runtime_error&) {
        return true;
    }
    return false;
}

int main(int argc, char** argv) {
    if (argc < 2) return 2;
    cuinfer::GGUFParser p0(argv[1]);
    CHECK(p0.version() == 3);
    CHECK(p0.architecture() == "llama");
    CHECK(p0.embedding_length() == 512);
    CHECK(p0.rms_norm_eps() == 1e-5f);
    CHECK(p0.tie_word_embeddings());
    CHECK(throws([&] { (void)p0.get_string("nonexistent.key"); }));
    CHECK(throws([&] { (void)p0.get_string("llama.embedding_length"); }));  // a UINT32
    CHECK(throws([&] { (void)p0.tensor_data("nonexistent"); }));
    CHECK(p0.find_tensor("nonexistent") == nullptr);
    const cuinfer::GGUFTensorInfo* emb = p0.find_tensor("token_embd.weight");
    CHECK(emb && emb->type == cuinfer::GGMLType::Q6_K && emb->dimensions.size() == 2);
    cuinfer::GGUFParser p1(std::move(p0));  // move construction keeps the mapping
    CHECK(p1.find_tensor("token_embd.weight") != nullptr);
    cuinfer::GGUFParser p2(argv[1]);
    p2 = std::move(p1);  // move assignment
    CHECK(p2.version() == 3);
    CHECK(cuinfer::ggml_type_size(cuinfer::GGMLType::Q4_K) == 144 && cuinfer::ggml_block_size(cuinfer::GGMLType::Q4_K) == 256);
    CHECK(throws([] { (void)cuinfer::ggml_type_size(static_cast<cuinfer::GGMLType>(99)); }));
    if (argc < 6 || std::strcmp(argv[2], "--gpu") != 0) {
        std::printf("ok\n");
        return 0;
    }
    // GPU: the tied LM head straight from the quantized table, and embedding rows from it
    cuinfer::WeightFormat fmt;
    bool tied = false;
    cuinfer::Tensor head = cuinfer::load_lm_head(p2, fmt, &tied);
    CHECK(tied && fmt == cuinfer::WeightFormat::Q6_K);
    const int K = static_cast<int>(head.shape(3)), V = static_cast<int>(head.shape(2));
    cuinfer::WeightFormat ffmt;
    cuinfer::Tensor up = cuinfer::load_weight_quantized(p2, "blk.0.ffn_up.weight", ffmt);
    CHECK(ffmt == cuinfer::WeightFormat::Q4_K);
    CHECK(throws([&] { cuinfer::WeightFormat f2; (void)cuinfer::load_weight_quantized(p2, "missing.weight", f2); }));
    std::vector<float> x(K);
    FILE* fx = std::fopen(argv[4], "rb");
    CHECK(fx && std::fread(x.data(), 4, K, fx) == static_cast<size_t>(K));
    std::fclose(fx);
    std::vector<int32_t> ids;
    for (char* s = std::strtok(argv[5], ","); s; s = std::strtok(nullptr, ",")) ids.push_back(std::atoi(s));
    float *dx, *dy, *dup, *drows;
    int32_t* dids;
    CUINFER_CHECK_HIP(hipMalloc(&dx, K * 4));
    CUINFER_CHECK_HIP(hipMalloc(&dy, V * 4));
    CUINFER_CHECK_HIP(hipMalloc(&dup, up.shape(2) * 4));
    CUINFER_CHECK_HIP(hipMalloc(&drows, ids.size() * K * 4));
    CUINFER_CHECK_HIP(hipMalloc(&dids, ids.size() * 4));
    CUINFER_CHECK_HIP(hipMemcpy(dx, x.data(), K * 4, hipMemcpyHostToDevice));
    CUINFER_CHECK_HIP(hipMemcpy(dids, ids.data(), ids.size() * 4, hipMemcpyHostToDevice));
    cuinfer::matmul_dispatch(dx, head, dy, 1, V, K, fmt);
    cuinfer::matmul_dispatch(dx, up, dup, 1, static_cast<int>(up.shape(2)), K, ffmt);
    cuinfer::embedding_lookup(head, fmt, dids, drows, static_cast<int>(ids.size()));
    std::vector<float> y(V), u(up.shape(2)), rows(ids.size() * K);
    CUINFER_CHECK_HIP(hipMemcpy(y.data(), dy, V * 4, hipMemcpyDeviceToHost));
    CUINFER_CHECK_HIP(hipMemcpy(u.data(), dup, u.size() * 4, hipMemcpyDeviceToHost));
    CUINFER_CHECK_HIP(hipMemcpy(rows.data(), drows, rows.size() * 4, hipMemcpyDeviceToHost));
    FILE* fo = std::fopen(argv[3], "wb");
    CHECK(fo);
    std::fwrite(y.data(), 4, y.size(), fo);
    std::fwrite(u.data(), 4, u.size(), fo);
    std::fwrite(rows.data(), 4, rows.size(), fo);
    std::fclose(fo);
    std::printf("ok gpu\n");
    return 0;
}

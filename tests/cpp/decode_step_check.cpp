// C++ host check of cuinfer::DecodeStep loaded from a GGUF file the way the
// reference's TransformerModel constructor reads one (ref:src/model.cu:530-700:
// the configuration from the {arch}.* metadata, head_dim = dim / n_heads, the
// blk.N.* tensors in their file formats, output.weight or the tied token
// table), built and run by tests/test_decode_step_cpp.py.  Test infrastructure
// only.
//
//   decode_step_check FILE OUT IDS
//
// Step 1 runs the tokens IDS (comma-separated) eagerly at position 0; step 2
// captures a one-token step fed with step 1's greedy id of the last row and
// replays it once.  OUT receives, as raw little-endian words: step 1's logits
// [M, vocab] and ids [M], step 2's logits [vocab] and id, then layer 0's and
// the last layer's K and V cache rows 0 .. M (fp32 [M + 1, n_kv_heads, head_dim]
// each).
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "cuinfer/decode_step.h"
#include "cuinfer/gguf_parser.h"
#include "cuinfer/hip_utils.h"
#include "cuinfer/weights.h"

#define CHECK(c)                                                                \
    do {                                                                        \
        if (!(c)) {                                                             \
            std::fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
            return 1;                                                           \
        }                                                                       \
    } while (0)

namespace {

cuinfer::WeightRef weight(const cuinfer::GGUFParser& p, const std::string& name) {
    const cuinfer::GGUFTensorInfo* t = p.find_tensor(name);
    if (!t) throw std::runtime_error("missing tensor " + name);
    return {cuinfer::ggml_type_to_weight_format(t->type), p.tensor_data(*t)};
}

const float* norm(const cuinfer::GGUFParser& p, const std::string& name) {
    const cuinfer::GGUFTensorInfo* t = p.find_tensor(name);
    if (!t || t->type != cuinfer::GGMLType::F32) throw std::runtime_error("missing fp32 tensor " + name);
    return static_cast<const float*>(p.tensor_data(*t));
}

int run(int argc, char** argv) {
    CHECK(argc == 4);
    cuinfer::GGUFParser p(argv[1]);
    cuinfer::DecodeStepConfig cfg;
    cfg.n_layers = static_cast<int>(p.block_count());
    cfg.dim = static_cast<int>(p.embedding_length());
    cfg.n_heads = static_cast<int>(p.head_count());
    cfg.n_kv_heads = static_cast<int>(p.head_count_kv());
    cfg.head_dim = cfg.dim / cfg.n_heads;
    cfg.intermediate_size = static_cast<int>(p.feed_forward_length());
    cfg.vocab_size = static_cast<int>(p.vocab_size());
    cfg.max_seq_len = static_cast<int>(p.context_length());
    cfg.rms_norm_eps = p.rms_norm_eps();
    cfg.rope_theta = p.rope_freq_base();

    std::vector<int32_t> ids;
    for (char* s = std::strtok(argv[3], ","); s; s = std::strtok(nullptr, ",")) ids.push_back(std::atoi(s));
    const int M = static_cast<int>(ids.size());
    cfg.max_batch = M;
    CHECK(M >= 1 && M + 1 <= cfg.max_seq_len);

    cuinfer::DecodeStep step(cfg);
    for (int i = 0; i < cfg.n_layers; ++i) {
        const std::string b = "blk." + std::to_string(i) + ".";
        cuinfer::LayerWeightsRef L;
        L.attn_norm = norm(p, b + "attn_norm.weight");
        L.ffn_norm = norm(p, b + "ffn_norm.weight");
        L.q = weight(p, b + "attn_q.weight");
        L.k = weight(p, b + "attn_k.weight");
        L.v = weight(p, b + "attn_v.weight");
        L.o = weight(p, b + "attn_output.weight");
        L.gate = weight(p, b + "ffn_gate.weight");
        L.up = weight(p, b + "ffn_up.weight");
        L.down = weight(p, b + "ffn_down.weight");
        step.set_layer(i, L);
    }
    step.set_token_embedding(weight(p, "token_embd.weight"));
    if (p.tie_word_embeddings()) {
        step.set_output(norm(p, "output_norm.weight"), nullptr);
    } else {
        const cuinfer::WeightRef head = weight(p, "output.weight");
        step.set_output(norm(p, "output_norm.weight"), &head);
    }

    const size_t V = static_cast<size_t>(cfg.vocab_size);
    float* logits;
    int32_t *dids, *dnext;
    CUINFER_CHECK_HIP(hipMalloc(&logits, M * V * 4));
    CUINFER_CHECK_HIP(hipMalloc(&dids, M * 4));
    CUINFER_CHECK_HIP(hipMalloc(&dnext, M * 4));
    CUINFER_CHECK_HIP(hipMemcpy(dids, ids.data(), M * 4, hipMemcpyHostToDevice));
    hipStream_t s;
    CUINFER_CHECK_HIP(hipStreamCreate(&s));

    // step 1: M tokens at position 0, eager
    step.forward(dids, M, logits, dnext, s);
    CUINFER_CHECK_HIP(hipStreamSynchronize(s));
    CHECK(step.position() == M);
    std::vector<float> l1(M * V);
    std::vector<int32_t> n1(M);
    CUINFER_CHECK_HIP(hipMemcpy(l1.data(), logits, l1.size() * 4, hipMemcpyDeviceToHost));
    CUINFER_CHECK_HIP(hipMemcpy(n1.data(), dnext, M * 4, hipMemcpyDeviceToHost));

    // step 2: one token, the greedy id of step 1's last row, as a captured graph replayed once
    int32_t* feed = dnext + (M - 1);
    step.capture(feed, 1, logits, feed, s);
    CHECK(step.position() == M && step.captured_batch() == 1);
    step.replay(s);
    CUINFER_CHECK_HIP(hipStreamSynchronize(s));
    std::vector<float> l2(V);
    int32_t n2 = -1;
    CUINFER_CHECK_HIP(hipMemcpy(l2.data(), logits, V * 4, hipMemcpyDeviceToHost));
    CUINFER_CHECK_HIP(hipMemcpy(&n2, feed, 4, hipMemcpyDeviceToHost));

    FILE* fo = std::fopen(argv[2], "wb");
    CHECK(fo);
    std::fwrite(l1.data(), 4, l1.size(), fo);
    std::fwrite(n1.data(), 4, n1.size(), fo);
    std::fwrite(l2.data(), 4, l2.size(), fo);
    std::fwrite(&n2, 4, 1, fo);
    const size_t rows = static_cast<size_t>(M + 1) * cfg.n_kv_heads * cfg.head_dim;
    std::vector<float> c(rows);
    for (int li : {0, cfg.n_layers - 1}) {
        for (float* src : {step.k_cache(li), step.v_cache(li)}) {
            CUINFER_CHECK_HIP(hipMemcpy(c.data(), src, rows * 4, hipMemcpyDeviceToHost));
            std::fwrite(c.data(), 4, rows, fo);
        }
    }
    std::fclose(fo);
    CUINFER_CHECK_HIP(hipStreamDestroy(s));
    CUINFER_CHECK_HIP(hipFree(logits));
    CUINFER_CHECK_HIP(hipFree(dids));
    CUINFER_CHECK_HIP(hipFree(dnext));
    std::printf("ok gpu\n");
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        return run(argc, argv);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
}

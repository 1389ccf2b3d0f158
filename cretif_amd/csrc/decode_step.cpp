// decode_step.cpp -- cuinfer::DecodeStep and its C ABI (cri_decoder_*).
//
// The layer loop of TransformerModel::forward's quantized path
// (ref:src/model.cu:831-1039) over buffers allocated once, with every
// projection going through matmul_dispatch (its fused-prologue forms for
// batches of up to 16 tokens; for a prompt, K splits through the step's
// workspace and a SiLU * up epilogue on the gate/up GEMM) and the position kept
// in device memory so that one captured graph serves every following token.
#include "../../include/cuinfer/decode_step.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <string>

#include "../../include/cri.h"
#include "../../include/cuinfer/embedding.h"
#include "../../include/cuinfer/hip_utils.h"
#include "../../include/cuinfer/kernels/elementwise.h"
#include "internal.hpp"

namespace cuinfer {

namespace {

// Batches up to this many tokens take the fused RMSNorm / SwiGLU prologues.
constexpr int kFusedMaxBatch = 16;
// Larger batches (a prompt) run attention on the multi-row split kernel at head_dim 64, otherwise
// through batched_matmul_gqa in row blocks of cri::detail::kPromptRows rows (the scores workspace
// holds n_heads x that x max_seq_len floats).
using cri::detail::kPromptRows;

int round4(int n) { return (n + 3) / 4 * 4; }
// K parts of the one-token down projection (its partial sums go to the next RMSNorm prologue)
constexpr int kDownSplits = 4;
static_assert(kDownSplits <= cri::kResMaxSplits, "the RMSNorm prologue adds up at most kResMaxSplits parts");

DType dtype_of(WeightFormat f) {
    switch (f) {
        case WeightFormat::FP32: return DType::FP32;
        case WeightFormat::FP16: return DType::FP16;
        case WeightFormat::Q8_0: return DType::Q8_0;
        case WeightFormat::Q4_0: return DType::Q4_0;
        case WeightFormat::Q5_0: return DType::Q5_0;
        case WeightFormat::Q4_K: return DType::Q4_K;
        case WeightFormat::Q6_K: return DType::Q6_K;
    }
    return DType::FP32;
}

size_t row_bytes(WeightFormat f, int64_t K) {
    const DType d = dtype_of(f);
    return static_cast<size_t>(K / dtype_block_elements(d)) * dtype_block_bytes(d);
}

void check_k(WeightFormat f, int64_t K, const char* what) {
    if (f == WeightFormat::FP32)
        throw std::invalid_argument(std::string("DecodeStep: ") + what +
                                    " is FP32; projections take FP16 or a block format ([N, K] rows)");
    const int be = dtype_block_elements(dtype_of(f));
    if (K % be != 0)
        throw std::invalid_argument(std::string("DecodeStep: ") + what + " has K = " + std::to_string(K) +
                                    ", not a multiple of its " + weight_format_name(f) + " block size " +
                                    std::to_string(be));
}

void copy_in(void* dst, const void* src, size_t bytes, const char* what) {
    if (!src) throw std::invalid_argument(std::string("DecodeStep: null ") + what);
    CUINFER_CHECK_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDefault));
}

void check_status(int rc, const char* what) {
    if (rc == cri::detail::kFailed || rc == CRI_ERR_LAUNCH)
        throw std::runtime_error(std::string("DecodeStep: ") + what + " launch failed");
    if (rc != 0) throw std::runtime_error(std::string("DecodeStep: ") + what + " declined the shape");
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        throw std::runtime_error(std::string("DecodeStep: ") + what + " launch failed: " + hipGetErrorString(e));
}

bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

// a cri_status from the C ABI's dispatch
void check_cri(int rc, const char* what) {
    if (rc != CRI_OK) throw std::runtime_error(std::string("DecodeStep: ") + what + ": " + cri_last_error_string());
}

int cri_id(WeightFormat f) {
    switch (f) {
        case WeightFormat::FP32: return CRI_FP32;
        case WeightFormat::FP16: return CRI_FP16;
        case WeightFormat::Q8_0: return CRI_Q8_0;
        case WeightFormat::Q4_0: return CRI_Q4_0;
        case WeightFormat::Q5_0: return CRI_Q5_0;
        case WeightFormat::Q4_K: return CRI_Q4_K;
        case WeightFormat::Q6_K: return CRI_Q6_K;
    }
    return -1;
}

// RMSNorm(h + res) times W on the decode-batch kernels, with a split workspace (the first call
// of a layer writes h + res to h_out); with defer, a K split into defer_S partial sums (any
// count for 0) is left in ws for the consumer (defer->S = 0: C was written)
// the residual for launch_split_norm: `count` partial sums `stride` floats apart, or the plain
// residual (one part), or none
cri::SplitSums residual_sums(const float* part, long stride, int count, const float* res, int dim) {
    cri::SplitSums r;
    r.N = dim;
    if (count > 0) {
        r.part = part;
        r.stride = stride;
        r.S = count;
    } else if (res) {
        r.part = res;
        r.S = 1;
    }
    return r;
}

void norm_matmul(const float* h, const float* res, const float* norm_w, float* h_out, const Tensor& W, WeightFormat f,
                 float* C, int M, int N, int K, float eps, Tensor& ws, hipStream_t s, const char* what,
                 cri::SplitSums* defer = nullptr, int defer_S = 0) {
    check_cri(cri::detail::matmul_rmsnorm_split_ws(cri_id(f), h, res, norm_w, h_out, W.data(), C, M, N, K, eps,
                                                    ws.data_as<float>(), ws.numel(), s, defer, defer_S),
              what);
}

}  // namespace

struct DecodeStep::Layer {
    bool set = false;
    Tensor attn_norm, ffn_norm;
    // q/k/v: one [q_dim + 2 kv_dim, dim] matrix when the three share a format, else three
    bool qkv_fused = false;
    Tensor qkv, q, k, v;
    WeightFormat qkv_fmt = WeightFormat::Q4_K, q_fmt = WeightFormat::Q4_K, k_fmt = WeightFormat::Q4_K,
                 v_fmt = WeightFormat::Q4_K;
    Tensor o;
    WeightFormat o_fmt = WeightFormat::Q4_K;
    // gate/up: one [2 ffn, dim] matrix when they share a format (rows [0, ffn) gate, [ffn, 2 ffn) up)
    bool gu_fused = false;
    Tensor gu, gate, up;
    WeightFormat gu_fmt = WeightFormat::Q4_K, gate_fmt = WeightFormat::Q4_K, up_fmt = WeightFormat::Q4_K;
    Tensor down;
    WeightFormat down_fmt = WeightFormat::Q4_K;
};

DecodeStep::DecodeStep(const DecodeStepConfig& c) : cfg_(c) {
    auto bad = [](const std::string& m) { throw std::invalid_argument("DecodeStep: " + m); };
    if (c.n_layers < 1 || c.dim < 1 || c.n_heads < 1 || c.n_kv_heads < 1 || c.head_dim < 1 ||
        c.intermediate_size < 1 || c.vocab_size < 1 || c.max_seq_len < 1)
        bad("every dimension of the configuration must be positive");
    if (c.max_batch < 1 || c.max_batch > 65535) bad("max_batch must be in [1, 65535]");
    if (c.n_heads % c.n_kv_heads != 0) bad("n_heads is not a multiple of n_kv_heads");
    if (c.head_dim % 4 != 0 || c.head_dim > cri::detail::kDecodeAttnSplitMaxHeadDim)
        bad("head_dim must be a multiple of 4 and at most " +
            std::to_string(cri::detail::kDecodeAttnSplitMaxHeadDim) + " (the attention kernel's layout)");
    if (c.dim % 4 != 0 || c.intermediate_size % 4 != 0) bad("dim and intermediate_size must be multiples of 4");
    q_dim_ = c.n_heads * c.head_dim;
    kv_dim_ = c.n_kv_heads * c.head_dim;
    const int64_t MB = c.max_batch;
    layers_.resize(c.n_layers);
    for (auto& L : layers_) L = std::make_unique<Layer>();
    const int64_t cache = static_cast<int64_t>(c.n_layers) * c.max_seq_len * kv_dim_;
    k_cache_ = Tensor::zeros({cache});
    v_cache_ = Tensor::zeros({cache});
    pos_dev_ = Tensor::zeros({4}, DType::INT8);
    for (auto& h : hid_) h = Tensor::empty({MB, static_cast<int64_t>(c.dim)});
    normed_ = Tensor::empty({MB, static_cast<int64_t>(c.dim)});
    qkv_ = Tensor::empty({MB, static_cast<int64_t>(q_dim_ + 2 * kv_dim_)});
    ctx_ = Tensor::empty({MB, static_cast<int64_t>(q_dim_)});
    attn_out_ = Tensor::empty({MB, static_cast<int64_t>(c.dim)});
    ff_ = Tensor::empty({MB, 2 * static_cast<int64_t>(c.intermediate_size)});
    act_ = Tensor::empty({MB, static_cast<int64_t>(c.intermediate_size)});
    ffn_out_ = Tensor::empty({MB, static_cast<int64_t>(c.dim)});
    // records for the larger of the one-row and the multi-row chunk counts (the split attention
    // serves batches of up to kFusedMaxBatch rows, and prompts too where the multi-row kernel
    // takes them: head_dim 64)
    prompt_mrow_ = MB > kFusedMaxBatch && cri::detail::decode_attention_rows_mrow(static_cast<int>(MB), c.head_dim);
    const int64_t arows = prompt_mrow_ ? MB : std::min<int64_t>(MB, kFusedMaxBatch);
    // the most records any batch size up to arows writes (its rows x heads x chunks; the chunk count
    // falls as the rows grow)
    int64_t recs = 0;
    for (int64_t r = 1; r <= arows; ++r)
        recs = std::max<int64_t>(recs, r * c.n_heads *
                                           cri::detail::decode_attention_rows_chunks(c.n_heads, c.n_kv_heads, c.head_dim,
                                                                                     c.max_seq_len, static_cast<int>(r)));
    attn_ws_ = Tensor::empty({recs * (c.head_dim + 4)});
    // partial sums of the decode-batch matmuls (up to kFusedMaxBatch rows) and of a prompt's
    // prefill GEMMs whose K is split over workgroups
    const int64_t brows = std::min<int64_t>(MB, kFusedMaxBatch);
    split_ws_ = Tensor::empty({std::max<int64_t>(cri::detail::skinny_workspace_floats(static_cast<int>(brows), c.dim),
                                                 MB > kFusedMaxBatch ? cri::detail::kPrefillSplitFloats : 0)});
    // the decode batch's q/k/v and gate/up partial sums, left for RoPE and the down projection's
    // prologue to add up (a second workspace: the down projection splits into split_ws_ while
    // it reads these)
    defer_ws_ = Tensor::empty({cri::detail::skinny_workspace_floats(static_cast<int>(brows), c.dim)});
    // zeroed once; the argmax kernel that counts in them leaves them zero again
    argmax_part_ = Tensor::empty({MB * cri::detail::argmax_slices(c.vocab_size) * 2});
    argmax_count_ = Tensor::zeros({MB});
    res_parts_ = Tensor::empty({static_cast<int64_t>(cri::kResMaxSplits) * c.dim});
    norm_ss_ = Tensor::zeros({256});
    if (MB > kFusedMaxBatch && !prompt_mrow_) {
        const int64_t rows = std::min<int64_t>(MB, kPromptRows), T4 = round4(c.max_seq_len);
        gqa_q_ = Tensor::empty({c.n_heads * rows * c.head_dim});
        gqa_o_ = Tensor::empty({c.n_heads * rows * c.head_dim});
        gqa_k_ = Tensor::empty({c.n_kv_heads * T4 * c.head_dim});
        gqa_v_ = Tensor::empty({c.n_kv_heads * T4 * c.head_dim});
        gqa_s_ = Tensor::empty({c.n_heads * rows * T4});
    }
    // RoPE (cos, sin) per (position, pair), ref:src/kernels/elementwise.cu:241-248: the frequency
    // 1 / theta^(2i / head_dim) and the angle pos * freq with the reference's fp32 operations,
    // theta^e, cos and sin in double rounded once to fp32
    const int half = c.head_dim / 2;
    std::vector<float> rot(static_cast<size_t>(c.max_seq_len) * half * 2);
    for (int i = 0; i < half; ++i) {
        const float e = (2.0f * static_cast<float>(i)) / static_cast<float>(c.head_dim);
        const float freq = 1.0f / static_cast<float>(std::pow(static_cast<double>(c.rope_theta), static_cast<double>(e)));
        for (int p = 0; p < c.max_seq_len; ++p) {
            const float ang = static_cast<float>(p) * freq;
            rot[(static_cast<size_t>(p) * half + i) * 2] = static_cast<float>(std::cos(static_cast<double>(ang)));
            rot[(static_cast<size_t>(p) * half + i) * 2 + 1] = static_cast<float>(std::sin(static_cast<double>(ang)));
        }
    }
    rope_ = Tensor::from_host(rot.data(), {static_cast<int64_t>(rot.size())});
}

DecodeStep::~DecodeStep() { drop_graph(); }

void DecodeStep::drop_graph() {
    if (graph_exec_) {
        (void)hipDeviceSynchronize();  // a replay still running keeps its launch; the buffers may go after it
        (void)hipGraphExecDestroy(graph_exec_);
        graph_exec_ = nullptr;
    }
    if (graph_) {
        (void)hipGraphDestroy(graph_);
        graph_ = nullptr;
    }
    graph_m_ = 0;
}

void DecodeStep::set_layer(int li, const LayerWeightsRef& w) {
    if (li < 0 || li >= cfg_.n_layers) throw std::out_of_range("DecodeStep::set_layer: layer out of range");
    const int64_t D = cfg_.dim, F = cfg_.intermediate_size, QD = q_dim_, KVD = kv_dim_;
    check_k(w.q.format, D, "q");
    check_k(w.k.format, D, "k");
    check_k(w.v.format, D, "v");
    check_k(w.o.format, QD, "o");
    check_k(w.gate.format, D, "gate");
    check_k(w.up.format, D, "up");
    check_k(w.down.format, F, "down");
    drop_graph();
    // filled in a new layer; the old one (and its buffers) is replaced only once every copy succeeded
    auto fresh = std::make_unique<Layer>();
    Layer& L = *fresh;
    L.attn_norm = Tensor::empty({D});
    L.ffn_norm = Tensor::empty({D});
    copy_in(L.attn_norm.data(), w.attn_norm, D * 4, "attn_norm");
    copy_in(L.ffn_norm.data(), w.ffn_norm, D * 4, "ffn_norm");

    L.qkv_fused = w.q.format == w.k.format && w.q.format == w.v.format;
    L.q = Tensor();
    L.k = Tensor();
    L.v = Tensor();
    L.qkv = Tensor();
    if (L.qkv_fused) {
        L.qkv_fmt = w.q.format;
        const size_t rb = row_bytes(L.qkv_fmt, D);
        L.qkv = Tensor::empty({QD + 2 * KVD, D}, dtype_of(L.qkv_fmt));
        char* base = static_cast<char*>(L.qkv.data());
        copy_in(base, w.q.data, QD * rb, "q");
        copy_in(base + QD * rb, w.k.data, KVD * rb, "k");
        copy_in(base + (QD + KVD) * rb, w.v.data, KVD * rb, "v");
    } else {
        L.q_fmt = w.q.format;
        L.k_fmt = w.k.format;
        L.v_fmt = w.v.format;
        L.q = Tensor::empty({QD, D}, dtype_of(L.q_fmt));
        L.k = Tensor::empty({KVD, D}, dtype_of(L.k_fmt));
        L.v = Tensor::empty({KVD, D}, dtype_of(L.v_fmt));
        copy_in(L.q.data(), w.q.data, L.q.size_bytes(), "q");
        copy_in(L.k.data(), w.k.data, L.k.size_bytes(), "k");
        copy_in(L.v.data(), w.v.data, L.v.size_bytes(), "v");
    }
    L.o_fmt = w.o.format;
    L.o = Tensor::empty({D, QD}, dtype_of(L.o_fmt));
    copy_in(L.o.data(), w.o.data, L.o.size_bytes(), "o");

    L.gu_fused = w.gate.format == w.up.format;
    L.gu = Tensor();
    L.gate = Tensor();
    L.up = Tensor();
    if (L.gu_fused) {
        L.gu_fmt = w.gate.format;
        const size_t rb = row_bytes(L.gu_fmt, D);
        L.gu = Tensor::empty({2 * F, D}, dtype_of(L.gu_fmt));
        char* base = static_cast<char*>(L.gu.data());
        copy_in(base, w.gate.data, F * rb, "gate");
        copy_in(base + F * rb, w.up.data, F * rb, "up");
    } else {
        L.gate_fmt = w.gate.format;
        L.up_fmt = w.up.format;
        L.gate = Tensor::empty({F, D}, dtype_of(L.gate_fmt));
        L.up = Tensor::empty({F, D}, dtype_of(L.up_fmt));
        copy_in(L.gate.data(), w.gate.data, L.gate.size_bytes(), "gate");
        copy_in(L.up.data(), w.up.data, L.up.size_bytes(), "up");
    }
    L.down_fmt = w.down.format;
    L.down = Tensor::empty({D, F}, dtype_of(L.down_fmt));
    copy_in(L.down.data(), w.down.data, L.down.size_bytes(), "down");
    L.set = true;
    layers_[li] = std::move(fresh);
}

void DecodeStep::set_token_embedding(const WeightRef& table) {
    if (table.format != WeightFormat::FP32) check_k(table.format, cfg_.dim, "token embedding");
    drop_graph();
    Tensor t = Tensor::empty({static_cast<int64_t>(cfg_.vocab_size), static_cast<int64_t>(cfg_.dim)},
                             dtype_of(table.format));
    copy_in(t.data(), table.data, t.size_bytes(), "token embedding");
    tok_table_ = std::move(t);
    tok_fmt_ = table.format;
    tok_set_ = true;
}

void DecodeStep::set_output(const float* output_norm, const WeightRef* lm_head) {
    if (lm_head && lm_head->format != WeightFormat::FP32) check_k(lm_head->format, cfg_.dim, "lm_head");
    drop_graph();
    Tensor norm = Tensor::empty({static_cast<int64_t>(cfg_.dim)});
    copy_in(norm.data(), output_norm, static_cast<size_t>(cfg_.dim) * 4, "output_norm");
    Tensor head;
    if (lm_head) {
        head = Tensor::empty({static_cast<int64_t>(cfg_.vocab_size), static_cast<int64_t>(cfg_.dim)},
                             dtype_of(lm_head->format));
        copy_in(head.data(), lm_head->data, head.size_bytes(), "lm_head");
        lm_fmt_ = lm_head->format;
    }
    out_norm_ = std::move(norm);
    lm_head_ = std::move(head);
    lm_tied_ = lm_head == nullptr;
    out_set_ = true;
}

void DecodeStep::check_ready() const {
    for (size_t i = 0; i < layers_.size(); ++i)
        if (!layers_[i]->set) throw std::logic_error("DecodeStep: layer " + std::to_string(i) + " has no weights");
    if (!tok_set_) throw std::logic_error("DecodeStep: no token embedding table");
    if (!out_set_) throw std::logic_error("DecodeStep: no output norm / LM head");
    if (lm_tied_ && !tok_set_) throw std::logic_error("DecodeStep: tied LM head without a token table");
}

float* DecodeStep::k_cache(int layer) {
    if (layer < 0 || layer >= cfg_.n_layers) throw std::out_of_range("DecodeStep::k_cache: layer out of range");
    return k_cache_.data_as<float>() + static_cast<int64_t>(layer) * cfg_.max_seq_len * kv_dim_;
}
float* DecodeStep::v_cache(int layer) {
    if (layer < 0 || layer >= cfg_.n_layers) throw std::out_of_range("DecodeStep::v_cache: layer out of range");
    return v_cache_.data_as<float>() + static_cast<int64_t>(layer) * cfg_.max_seq_len * kv_dim_;
}

namespace {
// device bytes a tensor holds (an unset Tensor reports a one-element shape but holds nothing)
size_t held_bytes(const Tensor& t) { return t.data() ? t.size_bytes() : 0; }
}  // namespace

size_t DecodeStep::step_weight_bytes(int M) const {
    size_t n = held_bytes(out_norm_);
    if (lm_tied_) {
        n += held_bytes(tok_table_);  // the LM head reads the whole table, the token rows among it
    } else {
        n += held_bytes(lm_head_);
        const int rows = std::max(0, std::min(M, cfg_.vocab_size));
        n += static_cast<size_t>(rows) * (tok_fmt_ == WeightFormat::FP32 ? static_cast<size_t>(cfg_.dim) * 4
                                                                          : row_bytes(tok_fmt_, cfg_.dim));
    }
    for (const auto& L : layers_)
        for (const Tensor* t : {&L->attn_norm, &L->ffn_norm, &L->qkv, &L->q, &L->k, &L->v, &L->o, &L->gu, &L->gate,
                                &L->up, &L->down})
            n += held_bytes(*t);
    return n;
}

size_t DecodeStep::weight_bytes() const {
    size_t n = held_bytes(tok_table_) + held_bytes(out_norm_) + held_bytes(lm_head_);
    for (const auto& L : layers_)
        for (const Tensor* t : {&L->attn_norm, &L->ffn_norm, &L->qkv, &L->q, &L->k, &L->v, &L->o, &L->gu, &L->gate,
                                &L->up, &L->down})
            n += held_bytes(*t);
    return n;
}

void DecodeStep::set_position(int pos, hipStream_t s) {
    if (pos < 0 || pos > cfg_.max_seq_len)
        throw std::out_of_range("DecodeStep::set_position: " + std::to_string(pos) + " outside [0, max_seq_len]");
    check_status(cri::detail::launch_pos_set(static_cast<int*>(pos_dev_.data()), pos, s), "position update");
    pos_host_ = pos;
}

// hidden[cur] (+ res) -> RMSNorm -> q/k/v -> RoPE + cache append -> attention -> o: attn_out
void DecodeStep::attn_block(Layer& L, int li, int M, int& cur, const float*& res, hipStream_t s) {
    const int D = cfg_.dim, QD = q_dim_, KVD = kv_dim_, MB = cfg_.max_batch;
    const float eps = cfg_.rms_norm_eps;
    float* h = hid_[cur].data_as<float>();
    float* h_next = hid_[1 - cur].data_as<float>();
    float* base = qkv_.data_as<float>();
    float *q, *k, *v;
    long ldq, ldk, ldv;
    if (L.qkv_fused) {
        q = base;
        k = base + QD;
        v = base + QD + KVD;
        ldq = ldk = ldv = QD + 2 * KVD;
    } else {
        q = base;
        k = base + static_cast<long>(MB) * QD;
        v = k + static_cast<long>(MB) * KVD;
        ldq = QD;
        ldk = ldv = KVD;
    }
    cri::SplitSums qkv_sums;  // S > 0: the fused projection's partial sums, added up by RoPE
    const int* pos = static_cast<const int*>(pos_dev_.data());
    // one token, fused q/k/v: the GEMV rotates q and k and appends k and v to the caches in its
    // epilogue (false: its layout declined, the RoPE kernel runs after the projection)
    auto rope_gemv = [&]() {
        cri::RopeOut R;
        R.pos = pos;
        R.rot = rope_.data_as<float>();
        R.kc = k_cache(li);
        R.vc = v_cache(li);
        R.qd = QD;
        R.kvd = KVD;
        R.half = cfg_.head_dim / 2;
        cri::ActIn act{h, res, L.attn_norm.data_as<float>(), h_next, D, eps};
        act.split = D;
        act.kn = res_splits_;
        const int rc = cri::detail::launch_gemv_rope(cri_id(L.qkv_fmt), act, L.qkv.data(), q, QD + 2 * KVD, D, R, s,
                                                     res_splits_ > 0);
        if (rc == cri::detail::kDeclined) return false;
        check_status(rc, "q/k/v projection with RoPE");
        return true;
    };
    bool roped = false;
    if (M == 1 && L.qkv_fused && rope_gemv()) {
        roped = true;
        cur = 1 - cur;
    } else if (res_splits_) {  // one token, the residual as partial sums (q/k/v GEMVs add them up)
        const float* an = L.attn_norm.data_as<float>();
        if (L.qkv_fused) {
            norm_matmul_splitres(h, an, h_next, L.qkv, L.qkv_fmt, q, QD + 2 * KVD, s, "q/k/v projection");
        } else {
            norm_matmul_splitres(h, an, h_next, L.q, L.q_fmt, q, QD, s, "q projection");
            norm_matmul_splitres(h, an, nullptr, L.k, L.k_fmt, k, KVD, s, "k projection");
            norm_matmul_splitres(h, an, nullptr, L.v, L.v_fmt, v, KVD, s, "v projection");
        }
        cur = 1 - cur;
    } else if (M <= kFusedMaxBatch) {
        // h_next = h + res; projections of RMSNorm(h_next) (the first writes h_next)
        if (L.qkv_fused) {
            norm_matmul(h, res, L.attn_norm.data_as<float>(), h_next, L.qkv, L.qkv_fmt, q, M, QD + 2 * KVD, D, eps,
                        defer_ws_, s, "q/k/v projection", &qkv_sums);
        } else {
            const float* an = L.attn_norm.data_as<float>();
            norm_matmul(h, res, an, h_next, L.q, L.q_fmt, q, M, QD, D, eps, split_ws_, s, "q projection");
            norm_matmul(h, res, an, nullptr, L.k, L.k_fmt, k, M, KVD, D, eps, split_ws_, s, "k projection");
            norm_matmul(h, res, an, nullptr, L.v, L.v_fmt, v, M, KVD, D, eps, split_ws_, s, "v projection");
        }
        cur = 1 - cur;
    } else {
        // hidden += res; normed = RMSNorm(hidden)  (ref:src/model.cu:963-967 for the residual form)
        prompt_norm(h, res, L.attn_norm.data_as<float>(), M, s, "attention RMSNorm");
        const float* n = normed_.data_as<float>();
        float* w = split_ws_.data_as<float>();
        const long wn = split_ws_.numel();
        // K splits of the prompt GEMMs store their partial sums in split_ws_ instead of adding them
        // with atomics: the fused projection's are added by RoPE, the others' by a reduction launch
        if (L.qkv_fused) {
            check_cri(cri::detail::matmul_split_ws(cri_id(L.qkv_fmt), n, L.qkv.data(), q, M, QD + 2 * KVD, D, w, wn, s,
                                                   &qkv_sums),
                      "q/k/v projection");
        } else {
            check_cri(cri::detail::matmul_split_ws(cri_id(L.q_fmt), n, L.q.data(), q, M, QD, D, w, wn, s), "q projection");
            check_cri(cri::detail::matmul_split_ws(cri_id(L.k_fmt), n, L.k.data(), k, M, KVD, D, w, wn, s),
                      "k projection");
            check_cri(cri::detail::matmul_split_ws(cri_id(L.v_fmt), n, L.v.data(), v, M, KVD, D, w, wn, s),
                      "v projection");
        }
    }
    if (!roped)
        check_status(cri::detail::launch_rope_append(q, ldq, k, ldk, v, ldv, M, cfg_.n_heads, cfg_.n_kv_heads,
                                                     cfg_.head_dim, rope_.data_as<float>(), pos, k_cache(li),
                                                     v_cache(li), s, &qkv_sums, QD, QD + KVD),
                     "rope/append");
    // row m attends to positions [0, pos + m] (ref:src/attention.cu:60-75; one token: :410-511)
    const float scale = 1.0f / std::sqrt(static_cast<float>(cfg_.head_dim));
    if (M > kFusedMaxBatch && !prompt_mrow_) {
        // a prompt: Q K^T and P V through batched_matmul_gqa around a causal softmax, in row blocks
        // (ref:src/attention.cu:809-871); the products span the cache positions the block can see,
        // rounded up to a multiple of 4 -- the whole cache when recording a graph, which is then
        // correct at any position it is replayed at
        for (int m0 = 0; m0 < M; m0 += kPromptRows) {
            const int mb = std::min(kPromptRows, M - m0);
            const int T4 = capturing_ ? round4(cfg_.max_seq_len)
                                      : std::min(round4(pos_host_ + m0 + mb), round4(cfg_.max_seq_len));
            check_status(cri::detail::launch_prefill_attention(
                             q + static_cast<long>(m0) * ldq, ldq, k_cache(li), v_cache(li),
                             ctx_.data_as<float>() + static_cast<long>(m0) * QD, m0, mb, cfg_.n_heads,
                             cfg_.n_kv_heads, cfg_.head_dim, T4, pos, scale, gqa_q_.data_as<float>(),
                             gqa_k_.data_as<float>(), gqa_v_.data_as<float>(), gqa_s_.data_as<float>(),
                             gqa_o_.data_as<float>(), s),
                         "prompt attention");
        }
    } else {
        // chunks for the whole cache (the chunk length follows the position in the kernel, so a
        // graph is valid at any position and computes what the eager step does)
        const int nchunks = cri::detail::decode_attention_rows_chunks(cfg_.n_heads, cfg_.n_kv_heads, cfg_.head_dim,
                                                                      cfg_.max_seq_len, M);
        check_status(cri::detail::launch_decode_attention_rows(q, ldq, k_cache(li), v_cache(li), ctx_.data_as<float>(),
                                                               QD, M, cfg_.n_heads, cfg_.n_kv_heads, cfg_.head_dim,
                                                               pos, 1, nchunks, scale, attn_ws_.data_as<float>(), s),
                     "attention");
    }
    // (2..16 tokens, and a prompt's K split: its partial sums are left for the FFN's RMSNorm row kernel)
    cri::SplitSums o_sums;
    check_cri(cri::detail::matmul_split_ws(cri_id(L.o_fmt), ctx_.data_as<float>(), L.o.data(),
                                           attn_out_.data_as<float>(), M, D, QD, split_ws_.data_as<float>(),
                                           split_ws_.numel(), s,
                                           split_flow(M) || prompt_defers(M) ? &o_sums : nullptr),
              "o projection");
    res = attn_out_.data_as<float>();
    res_splits_ = 0;
    res_part_ = o_sums.part;
    res_part_stride_ = o_sums.stride;
    res_part_count_ = o_sums.S;
}

bool DecodeStep::prompt_defers(int M) const {
    return M > kFusedMaxBatch && cfg_.dim % 4 == 0 && cfg_.dim <= 4096;
}

// a prompt's RMSNorm(hidden + residual) into normed_, hidden updated in place; the residual is the
// pending partial sums of a K-split projection when there are any (the row kernel adds them in
// split order), else res
void DecodeStep::prompt_norm(float* h, const float* res, const float* w, int M, hipStream_t s, const char* what) {
    const int D = cfg_.dim;
    if (res_part_count_ > 0) {
        check_status(cri::detail::launch_split_norm(h, residual_sums(res_part_, res_part_stride_, res_part_count_,
                                                                     nullptr, D),
                                                    w, h, normed_.data_as<float>(), M, D, cfg_.rms_norm_eps, s),
                     what);
        res_part_count_ = 0;
    } else {
        rmsnorm_residual(h, res, w, h, normed_.data_as<float>(), M, D, cfg_.rms_norm_eps, s);
    }
}

bool DecodeStep::split_flow(int M) const {
    return M > 1 && M <= kFusedMaxBatch && cfg_.dim % (4 * cri::detail::kNormParts) == 0 && cfg_.dim <= 4096;
}

bool DecodeStep::next_takes_split(int li) const {
    const int D = cfg_.dim;
    if (li + 1 < cfg_.n_layers) {
        const Layer& N = *layers_[li + 1];
        if (N.qkv_fused) return cri::detail::gemv_supported(cri_id(N.qkv_fmt), D, N.qkv.data());
        return cri::detail::gemv_supported(cri_id(N.q_fmt), D, N.q.data()) &&
               cri::detail::gemv_supported(cri_id(N.k_fmt), D, N.k.data()) &&
               cri::detail::gemv_supported(cri_id(N.v_fmt), D, N.v.data());
    }
    const Tensor& W = lm_tied_ ? tok_table_ : lm_head_;
    const WeightFormat wf = lm_tied_ ? tok_fmt_ : lm_fmt_;
    return wf != WeightFormat::FP32 && cri::detail::gemv_supported(cri_id(wf), D, W.data());
}

void DecodeStep::norm_matmul_splitres(const float* h, const float* norm_w, float* h_out, const Tensor& W,
                                      WeightFormat f, float* C, int N, hipStream_t s, const char* what) {
    const int D = cfg_.dim;
    check_cri(cri::detail::matmul_rmsnorm_splitres(cri_id(f), h, res_parts_.data_as<float>(), res_splits_, D, norm_w,
                                                   h_out, W.data(), C, N, D, cfg_.rms_norm_eps, s),
              what);
}

// hidden[cur] (+ attn_out) -> RMSNorm -> gate/up -> SiLU(gate) * up -> down: ffn_out
void DecodeStep::ffn_block(Layer& L, int li, int M, int& cur, const float*& res, hipStream_t s) {
    const int D = cfg_.dim, F = cfg_.intermediate_size, MB = cfg_.max_batch;
    const float eps = cfg_.rms_norm_eps;
    float* h = hid_[cur].data_as<float>();
    float* h_next = hid_[1 - cur].data_as<float>();
    float* ff = ff_.data_as<float>();
    float* ffn_out = ffn_out_.data_as<float>();
    // One token: the down GEMV splits K into kDownSplits parts (each workgroup stages that share
    // of the SwiGLU activations instead of all of them) and leaves the partial sums for the next
    // RMSNorm prologue to add up (false: not taken, C is computed whole).
    bool split_down = false;
    cri::SplitSums down_sums;  // a prompt's down projection: its K split's partial sums (S = 0: ffn_out written)
    auto down_split = [&](const float* gate, const float* up, int ld) {
        if (M != 1 || !next_takes_split(li)) return false;
        const cri::ActIn act{gate, up, nullptr, nullptr, ld, 0.0f};
        const int rc = cri::detail::launch_gemv_ksplit(cri::kActSwiGLU, cri_id(L.down_fmt), act, L.down.data(),
                                                       res_parts_.data_as<float>(), D, F, kDownSplits, s);
        if (rc == cri::detail::kDeclined) return false;
        check_status(rc, "down projection (K split)");
        return true;
    };
    if (split_flow(M)) {
        // for the fused gate/up the row factor is left out of normed and applied by the down
        // projection's prologue to gate/up's sums, which also adds up a two-way split of them
        float* ss = L.gu_fused ? norm_ss_.data_as<float>() : nullptr;
        check_status(cri::detail::launch_split_norm(h, residual_sums(res_part_, res_part_stride_, res_part_count_, res, D),
                                                    L.ffn_norm.data_as<float>(), h_next, normed_.data_as<float>(), M,
                                                    D, eps, s, ss),
                     "FFN RMSNorm");
        const float* n = normed_.data_as<float>();
        float* w = split_ws_.data_as<float>();
        const long wn = split_ws_.numel();
        if (L.gu_fused) {
            cri::SplitSums gu;
            check_cri(cri::detail::matmul_split_ws(cri_id(L.gu_fmt), n, L.gu.data(), ff, M, 2 * F, D,
                                                   defer_ws_.data_as<float>(), defer_ws_.numel(), s, &gu, 2),
                      "gate/up projection");
            if (!gu.S) {  // reduced (or never split) into ff: one partial sum
                gu.part = ff;
                gu.stride = 0;
                gu.S = 1;
            }
            gu.ssq = ss;
            gu.nss = cri::detail::kNormParts;
            gu.K = D;
            gu.eps = eps;
            check_cri(cri::detail::matmul_swiglu2_split_ws(cri_id(L.down_fmt), gu, F, 2 * F, L.down.data(), ffn_out, M,
                                                           D, F, w, wn, s),
                      "down projection");
        } else {
            float* up = ff + static_cast<long>(MB) * F;
            float* dw = defer_ws_.data_as<float>();
            const long dwn = defer_ws_.numel();
            check_cri(cri::detail::matmul_split_ws(cri_id(L.gate_fmt), n, L.gate.data(), ff, M, F, D, dw, dwn, s),
                      "gate projection");
            check_cri(cri::detail::matmul_split_ws(cri_id(L.up_fmt), n, L.up.data(), up, M, F, D, dw, dwn, s),
                      "up projection");
            check_cri(cri::detail::matmul_swiglu_split_ws(cri_id(L.down_fmt), ff, up, F, L.down.data(), ffn_out, M, D,
                                                          F, w, wn, s),
                      "down projection");
        }
        cur = 1 - cur;
    } else if (M <= kFusedMaxBatch) {
        if (L.gu_fused) {
            // ff rows: [gate (F) | up (F)]
            // a two-way K split of gate/up is added up inside the down projection's prologue
            cri::SplitSums gu;
            norm_matmul(h, res, L.ffn_norm.data_as<float>(), h_next, L.gu, L.gu_fmt, ff, M, 2 * F, D, eps, defer_ws_,
                        s, "gate/up projection", &gu, 2);
            if (gu.S)
                check_cri(cri::detail::matmul_swiglu2_split_ws(cri_id(L.down_fmt), gu, F, 2 * F, L.down.data(), ffn_out,
                                                               M, D, F, split_ws_.data_as<float>(), split_ws_.numel(), s),
                          "down projection");
            else if (!(split_down = down_split(ff, ff + F, 2 * F)))
                check_cri(cri::detail::matmul_swiglu_split_ws(cri_id(L.down_fmt), ff, ff + F, 2 * F, L.down.data(),
                                                              ffn_out, M, D, F, split_ws_.data_as<float>(),
                                                              split_ws_.numel(), s),
                          "down projection");
        } else {
            float* up = ff + static_cast<long>(MB) * F;
            norm_matmul(h, res, L.ffn_norm.data_as<float>(), h_next, L.gate, L.gate_fmt, ff, M, F, D, eps, split_ws_, s,
                        "gate projection");
            norm_matmul(h, res, L.ffn_norm.data_as<float>(), nullptr, L.up, L.up_fmt, up, M, F, D, eps, split_ws_, s,
                        "up projection");
            if (!(split_down = down_split(ff, up, F)))
                check_cri(cri::detail::matmul_swiglu_split_ws(cri_id(L.down_fmt), ff, up, F, L.down.data(), ffn_out, M,
                                                              D, F, split_ws_.data_as<float>(), split_ws_.numel(), s),
                          "down projection");
        }
        cur = 1 - cur;
    } else {
        prompt_norm(h, res, L.ffn_norm.data_as<float>(), M, s, "FFN RMSNorm");
        const float* n = normed_.data_as<float>();
        float* gate = ff;
        float* up = ff + static_cast<long>(MB) * F;
        // (a K split, at short prompts, goes through split_ws_ and a reduction launch: the same bits
        // on every call)
        float* w = split_ws_.data_as<float>();
        const long wn = split_ws_.numel();
        // the stacked gate/up matrix: both products and SiLU(gate) * up in one launch where the
        // tiles fill the GPU unsplit (ref:src/model.cu:986-997 computes the same in three steps)
        const int fused_rc = L.gu_fused ? cri::detail::launch_prefill_swiglu(cri_id(L.gu_fmt), n, L.gu.data(),
                                                                             act_.data_as<float>(), M, F, D, s)
                                        : cri::detail::kDeclined;
        if (fused_rc != cri::detail::kDeclined) {
            check_status(fused_rc, "gate/up projection with SiLU * up");
        } else if (L.gu_fused) {
            // the stacked matrix read as its two halves ([0, F) gate, [F, 2F) up)
            const Tensor g = L.gu.view(2, 0, F), u = L.gu.view(2, F, 2 * F);
            check_cri(cri::detail::matmul_split_ws(cri_id(L.gu_fmt), n, g.data(), gate, M, F, D, w, wn, s),
                      "gate projection");
            check_cri(cri::detail::matmul_split_ws(cri_id(L.gu_fmt), n, u.data(), up, M, F, D, w, wn, s),
                      "up projection");
        } else {
            check_cri(cri::detail::matmul_split_ws(cri_id(L.gate_fmt), n, L.gate.data(), gate, M, F, D, w, wn, s),
                      "gate projection");
            check_cri(cri::detail::matmul_split_ws(cri_id(L.up_fmt), n, L.up.data(), up, M, F, D, w, wn, s),
                      "up projection");
        }
        if (fused_rc == cri::detail::kDeclined)
            silu_mul(gate, up, act_.data_as<float>(), static_cast<long long>(M) * F, s);  // ref:src/model.cu:996-997
        // a K split's partial sums are left for the next RMSNorm row kernel (the next layer's or the final one)
        check_cri(cri::detail::matmul_split_ws(cri_id(L.down_fmt), act_.data_as<float>(), L.down.data(), ffn_out, M, D,
                                               F, split_ws_.data_as<float>(), split_ws_.numel(), s,
                                               prompt_defers(M) ? &down_sums : nullptr),
                  "down projection");
    }
    if (split_down) {
        res = res_parts_.data_as<float>();
        res_splits_ = kDownSplits;
    } else {
        res = ffn_out;
    }
    res_part_ = down_sums.part;
    res_part_stride_ = down_sums.stride;
    res_part_count_ = down_sums.S;
}

void DecodeStep::enqueue(const int32_t* ids, int M, float* logits, int32_t* next_ids, hipStream_t s, float* taps,
                         bool last_only) {
    const int D = cfg_.dim, V = cfg_.vocab_size;
    const float eps = cfg_.rms_norm_eps;
    // token rows straight from the table in its own format (the reference's Embedding::forward
    // reads an FP32 table, ref:src/embedding.cu:237-263)
    CUINFER_CHECK_CRI(
        cri_embedding_rows(cri_id(tok_fmt_), tok_table_.data(), ids, hid_[0].data_as<float>(), M, D, V, s));
    int cur = 0;
    const float* res = nullptr;  // residual still to be added to hidden[cur]
    res_splits_ = 0;
    res_part_count_ = 0;
    // the residual stream entering layer i (i = n_layers: the final norm): hidden + the pending residual
    auto tap = [&](int i) {
        if (!taps) return;
        const cri::SplitSums r = res_splits_ ? residual_sums(res_parts_.data_as<float>(), D, res_splits_, nullptr, D)
                                             : residual_sums(res_part_, res_part_stride_, res_part_count_, res, D);
        check_status(cri::detail::launch_hidden_tap(hid_[cur].data_as<float>(), r,
                                                    taps + static_cast<long>(i) * M * D, M, D, s),
                     "layer tap");
    };
    for (int li = 0; li < cfg_.n_layers; ++li) {
        Layer& L = *layers_[li];
        tap(li);
        attn_block(L, li, M, cur, res, s);
        ffn_block(L, li, M, cur, res, s);
    }
    tap(cfg_.n_layers);
    // final RMSNorm(hidden + ffn_out) and the LM head
    const Tensor& W = lm_tied_ ? tok_table_ : lm_head_;
    const WeightFormat wf = lm_tied_ ? tok_fmt_ : lm_fmt_;
    float* h = hid_[cur].data_as<float>();
    int* pos = static_cast<int*>(pos_dev_.data());
    if (last_only && M > 1) {
        // the final RMSNorm, the LM head and the argmax of row M - 1 alone (prefill())
        const long last = static_cast<long>(M - 1) * D;
        if (split_flow(M)) {  // the pending residual as partial sums: the row kernel adds them for every row
            check_status(cri::detail::launch_split_norm(h, residual_sums(res_part_, res_part_stride_, res_part_count_,
                                                                         res, D),
                                                        out_norm_.data_as<float>(), hid_[1 - cur].data_as<float>(),
                                                        normed_.data_as<float>(), M, D, eps, s),
                         "final RMSNorm");
            res_part_count_ = 0;
            const float* n = normed_.data_as<float>() + last;
            if (wf == WeightFormat::FP32)
                matmul_transposed_b(n, W.data_as<float>(), logits, 1, V, D, s);
            else
                matmul_dispatch(n, W, logits, 1, V, D, wf, s);
        } else if (res_part_count_ > 0) {  // a prompt's pending partial sums: the row kernel on the last row
            check_status(cri::detail::launch_split_norm(h + last, residual_sums(res_part_ + last, res_part_stride_,
                                                                                res_part_count_, nullptr, D),
                                                        out_norm_.data_as<float>(), hid_[1 - cur].data_as<float>() + last,
                                                        normed_.data_as<float>(), 1, D, eps, s),
                         "final RMSNorm");
            res_part_count_ = 0;
            if (wf == WeightFormat::FP32)
                matmul_transposed_b(normed_.data_as<float>(), W.data_as<float>(), logits, 1, V, D, s);
            else
                matmul_dispatch(normed_.data_as<float>(), W, logits, 1, V, D, wf, s);
        } else if (wf != WeightFormat::FP32) {  // a plain residual: RMSNorm inside the LM head's prologue
            matmul_dispatch_rmsnorm(h + last, res ? res + last : nullptr, out_norm_.data_as<float>(),
                                    hid_[1 - cur].data_as<float>() + last, W, logits, 1, V, D, wf, eps, s);
        } else {
            rmsnorm_residual(h + last, res ? res + last : nullptr, out_norm_.data_as<float>(), h + last,
                             normed_.data_as<float>(), 1, D, eps, s);
            matmul_transposed_b(normed_.data_as<float>(), W.data_as<float>(), logits, 1, V, D, s);
        }
        if (next_ids)
            check_status(cri::detail::launch_argmax_rows(logits, V, 1, V, next_ids, argmax_part_.data_as<float>(),
                                                         static_cast<unsigned*>(argmax_count_.data()), pos, M, s),
                         "argmax");
        else
            check_status(cri::detail::launch_pos_add(pos, M, s), "position update");
        return;
    }
    if (split_flow(M)) {  // the final RMSNorm as a row kernel, the LM head on plain activations
        check_status(cri::detail::launch_split_norm(h, residual_sums(res_part_, res_part_stride_, res_part_count_, res, D),
                                                    out_norm_.data_as<float>(), hid_[1 - cur].data_as<float>(),
                                                    normed_.data_as<float>(), M, D, eps, s),
                     "final RMSNorm");
        res_part_count_ = 0;
        if (wf == WeightFormat::FP32)
            matmul_transposed_b(normed_.data_as<float>(), W.data_as<float>(), logits, M, V, D, s);
        else
            check_cri(cri::detail::matmul_split_ws(cri_id(wf), normed_.data_as<float>(), W.data(), logits, M, V, D,
                                                   split_ws_.data_as<float>(), split_ws_.numel(), s),
                      "LM head");
    } else if (res_splits_) {  // one token, the last down projection's partial sums
        norm_matmul_splitres(h, out_norm_.data_as<float>(), hid_[1 - cur].data_as<float>(), W, wf, logits, V, s,
                             "LM head");
        res_splits_ = 0;
    } else if (wf != WeightFormat::FP32 && M <= kFusedMaxBatch) {
        matmul_dispatch_rmsnorm(h, res, out_norm_.data_as<float>(), hid_[1 - cur].data_as<float>(), W, logits, M, V,
                                D, wf, eps, s);
    } else {
        prompt_norm(h, res, out_norm_.data_as<float>(), M, s, "final RMSNorm");
        if (wf == WeightFormat::FP32)  // tied FP32 table (ref:src/model.cu:1027-1029)
            matmul_transposed_b(normed_.data_as<float>(), W.data_as<float>(), logits, M, V, D, s);
        else
            matmul_dispatch(normed_.data_as<float>(), W, logits, M, V, D, wf, s);
    }
    if (next_ids)  // the argmax's last workgroup also advances the position
        check_status(cri::detail::launch_argmax_rows(logits, V, M, V, next_ids, argmax_part_.data_as<float>(),
                                                     static_cast<unsigned*>(argmax_count_.data()), pos, M, s),
                     "argmax");
    else
        check_status(cri::detail::launch_pos_add(pos, M, s), "position update");
}

void DecodeStep::check_call(const int32_t* ids, int M, float* logits, int32_t* next_ids, const char* what) const {
    check_ready();
    const std::string fn = std::string("DecodeStep::") + what + ": ";
    if (M < 1 || M > cfg_.max_batch)
        throw std::invalid_argument(fn + "M = " + std::to_string(M) + " outside [1, max_batch = " +
                                    std::to_string(cfg_.max_batch) + "]");
    if (!ids || !logits) throw std::invalid_argument(fn + "null token_ids or logits");
    if (!aligned4(ids) || !aligned4(logits) || !aligned4(next_ids))
        throw std::invalid_argument(fn + "token_ids, logits and next_ids must be 4-byte aligned");
    if (pos_host_ + M > cfg_.max_seq_len)  // ref:src/model.cu:845-851
        throw std::overflow_error(fn + "would exceed max sequence length (" + std::to_string(pos_host_ + M) + " > " +
                                  std::to_string(cfg_.max_seq_len) + ")");
}

void DecodeStep::forward(const int32_t* ids, int M, float* logits, int32_t* next_ids, hipStream_t s) {
    check_call(ids, M, logits, next_ids, "forward");
    enqueue(ids, M, logits, next_ids, s);
    pos_host_ += M;
}

void DecodeStep::prefill(const int32_t* ids, int M, float* logits, int32_t* next_id, hipStream_t s) {
    check_call(ids, M, logits, next_id, "prefill");
    enqueue(ids, M, logits, next_id, s, nullptr, true);
    pos_host_ += M;
}

void DecodeStep::forward_taps(const int32_t* ids, int M, float* logits, int32_t* next_ids, float* taps,
                              hipStream_t s) {
    check_call(ids, M, logits, next_ids, "forward_taps");
    if (!taps || !aligned4(taps)) throw std::invalid_argument("DecodeStep::forward_taps: null or unaligned hidden_taps");
    enqueue(ids, M, logits, next_ids, s, taps);
    pos_host_ += M;
}

void DecodeStep::capture(const int32_t* ids, int M, float* logits, int32_t* next_ids, hipStream_t s) {
    check_ready();
    if (!s) throw std::invalid_argument("DecodeStep::capture: the null stream cannot be captured");
    if (M < 1 || M > cfg_.max_batch) throw std::invalid_argument("DecodeStep::capture: M outside [1, max_batch]");
    if (!ids || !logits) throw std::invalid_argument("DecodeStep::capture: null token_ids or logits");
    if (!aligned4(ids) || !aligned4(logits) || !aligned4(next_ids))
        throw std::invalid_argument("DecodeStep::capture: token_ids, logits and next_ids must be 4-byte aligned");
    drop_graph();
    CUINFER_CHECK_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    capturing_ = true;
    try {
        enqueue(ids, M, logits, next_ids, s);
    } catch (...) {
        capturing_ = false;
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(s, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
    }
    capturing_ = false;
    CUINFER_CHECK_HIP(hipStreamEndCapture(s, &graph_));
    CUINFER_CHECK_HIP(hipGraphInstantiate(&graph_exec_, graph_, nullptr, nullptr, 0));
    graph_m_ = M;
}

void DecodeStep::replay(hipStream_t s) {
    if (!graph_exec_) throw std::logic_error("DecodeStep::replay: nothing captured");
    if (pos_host_ + graph_m_ > cfg_.max_seq_len)
        throw std::overflow_error("DecodeStep::replay: would exceed max sequence length (" +
                                  std::to_string(pos_host_ + graph_m_) + " > " + std::to_string(cfg_.max_seq_len) +
                                  ")");
    CUINFER_CHECK_HIP(hipGraphLaunch(graph_exec_, s));
    pos_host_ += graph_m_;
}

}  // namespace cuinfer

// ---------------------------------------------------------------- C ABI
void cri_internal_set_error(const char* msg);  // abi.cpp

struct cri_decoder {
    cuinfer::DecodeStep step;
    explicit cri_decoder(const cuinfer::DecodeStepConfig& c) : step(c) {}
};

namespace {

int dec_fail(int status, const char* fn, const std::string& what) {
    cri_internal_set_error((std::string(fn) + ": " + what).c_str());
    return status;
}

// exceptions of the C++ layer -> status codes
template <class F>
int guarded(const char* fn, F&& f) {
    try {
        f();
        return CRI_OK;
    } catch (const std::overflow_error& e) {
        return dec_fail(CRI_ERR_SHAPE, fn, e.what());
    } catch (const std::out_of_range& e) {
        return dec_fail(CRI_ERR_INVALID_ARGUMENT, fn, e.what());
    } catch (const std::invalid_argument& e) {
        return dec_fail(CRI_ERR_INVALID_ARGUMENT, fn, e.what());
    } catch (const std::logic_error& e) {
        return dec_fail(CRI_ERR_INVALID_ARGUMENT, fn, e.what());
    } catch (const std::exception& e) {
        return dec_fail(CRI_ERR_LAUNCH, fn, e.what());
    }
}

bool weight_format(int f, cuinfer::WeightFormat* out, bool allow_fp32) {
    using cuinfer::WeightFormat;
    switch (f) {
        case CRI_Q8_0: *out = WeightFormat::Q8_0; return true;
        case CRI_Q4_0: *out = WeightFormat::Q4_0; return true;
        case CRI_Q5_0: *out = WeightFormat::Q5_0; return true;
        case CRI_Q4_K: *out = WeightFormat::Q4_K; return true;
        case CRI_Q6_K: *out = WeightFormat::Q6_K; return true;
        case CRI_FP16: *out = WeightFormat::FP16; return true;
        case CRI_FP32: *out = WeightFormat::FP32; return allow_fp32;
    }
    return false;
}

}  // namespace

extern "C" {

int cri_decoder_create(const cri_decoder_config* c, cri_decoder** out) {
    const char* fn = "cri_decoder_create";
    if (!c || !out) return dec_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null argument");
    *out = nullptr;
    cuinfer::DecodeStepConfig cfg;
    cfg.n_layers = c->n_layers;
    cfg.dim = c->dim;
    cfg.n_heads = c->n_heads;
    cfg.n_kv_heads = c->n_kv_heads;
    cfg.head_dim = c->head_dim;
    cfg.intermediate_size = c->ffn_dim;
    cfg.vocab_size = c->vocab_size;
    cfg.max_seq_len = c->max_seq_len;
    cfg.rms_norm_eps = c->rms_norm_eps;
    cfg.rope_theta = c->rope_theta;
    cfg.max_batch = c->max_batch;
    return guarded(fn, [&] { *out = new cri_decoder(cfg); });
}

void cri_decoder_destroy(cri_decoder* d) { delete d; }

int cri_decoder_set_layer(cri_decoder* d, int layer, const cri_decoder_layer* w) {
    const char* fn = "cri_decoder_set_layer";
    if (!d || !w) return dec_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null argument");
    cuinfer::LayerWeightsRef r;
    r.attn_norm = w->attn_norm;
    r.ffn_norm = w->ffn_norm;
    const struct {
        int f;
        const void* p;
        cuinfer::WeightRef* dst;
        const char* name;
    } ws[] = {{w->q_format, w->q, &r.q, "q"},          {w->k_format, w->k, &r.k, "k"},
              {w->v_format, w->v, &r.v, "v"},          {w->o_format, w->o, &r.o, "o"},
              {w->gate_format, w->gate, &r.gate, "gate"}, {w->up_format, w->up, &r.up, "up"},
              {w->down_format, w->down, &r.down, "down"}};
    for (const auto& x : ws) {
        if (!weight_format(x.f, &x.dst->format, false))
            return dec_fail(CRI_ERR_UNSUPPORTED, fn, std::string("unsupported format id for ") + x.name);
        x.dst->data = x.p;
    }
    return guarded(fn, [&] { d->step.set_layer(layer, r); });
}

int cri_decoder_set_embedding(cri_decoder* d, int format, const void* table) {
    const char* fn = "cri_decoder_set_embedding";
    if (!d) return dec_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null decoder");
    cuinfer::WeightRef r;
    if (!weight_format(format, &r.format, true)) return dec_fail(CRI_ERR_UNSUPPORTED, fn, "unsupported format id");
    r.data = table;
    return guarded(fn, [&] { d->step.set_token_embedding(r); });
}

int cri_decoder_set_output(cri_decoder* d, const float* output_norm, int format, const void* lm_head) {
    const char* fn = "cri_decoder_set_output";
    if (!d) return dec_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null decoder");
    cuinfer::WeightRef r;
    if (format >= 0 && !weight_format(format, &r.format, true))
        return dec_fail(CRI_ERR_UNSUPPORTED, fn, "unsupported format id");
    r.data = lm_head;
    return guarded(fn, [&] { d->step.set_output(output_norm, format < 0 ? nullptr : &r); });
}

int cri_decoder_forward(cri_decoder* d, const int* token_ids, int M, float* logits, int* next_ids, hipStream_t s) {
    const char* fn = "cri_decoder_forward";
    if (!d) return dec_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null decoder");
    return guarded(fn, [&] { d->step.forward(token_ids, M, logits, next_ids, s); });
}

int cri_decoder_prefill(cri_decoder* d, const int* token_ids, int M, float* logits, int* next_id, hipStream_t s) {
    const char* fn = "cri_decoder_prefill";
    if (!d) return dec_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null decoder");
    return guarded(fn, [&] { d->step.prefill(token_ids, M, logits, next_id, s); });
}

int cri_decoder_forward_taps(cri_decoder* d, const int* token_ids, int M, float* logits, int* next_ids,
                             float* hidden_taps, hipStream_t s) {
    const char* fn = "cri_decoder_forward_taps";
    if (!d) return dec_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null decoder");
    return guarded(fn, [&] { d->step.forward_taps(token_ids, M, logits, next_ids, hidden_taps, s); });
}

int cri_decoder_capture(cri_decoder* d, const int* token_ids, int M, float* logits, int* next_ids, hipStream_t s) {
    const char* fn = "cri_decoder_capture";
    if (!d) return dec_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null decoder");
    return guarded(fn, [&] { d->step.capture(token_ids, M, logits, next_ids, s); });
}

int cri_decoder_replay(cri_decoder* d, hipStream_t s) {
    const char* fn = "cri_decoder_replay";
    if (!d) return dec_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null decoder");
    return guarded(fn, [&] { d->step.replay(s); });
}

int cri_decoder_set_position(cri_decoder* d, int pos, hipStream_t s) {
    const char* fn = "cri_decoder_set_position";
    if (!d) return dec_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null decoder");
    return guarded(fn, [&] { d->step.set_position(pos, s); });
}

int cri_decoder_position(const cri_decoder* d) { return d ? d->step.position() : CRI_ERR_INVALID_ARGUMENT; }

int cri_decoder_kv_cache(cri_decoder* d, int layer, float** k, float** v) {
    const char* fn = "cri_decoder_kv_cache";
    if (!d || !k || !v) return dec_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null argument");
    return guarded(fn, [&] {
        *k = d->step.k_cache(layer);
        *v = d->step.v_cache(layer);
    });
}

long long cri_decoder_weight_bytes(const cri_decoder* d) {
    return d ? static_cast<long long>(d->step.weight_bytes()) : CRI_ERR_INVALID_ARGUMENT;
}

long long cri_decoder_step_weight_bytes(const cri_decoder* d, int M) {
    if (!d || M < 1) return CRI_ERR_INVALID_ARGUMENT;
    return static_cast<long long>(d->step.step_weight_bytes(M));
}

}  // extern "C"

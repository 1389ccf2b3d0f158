// weights.cpp -- GGUF -> device weights (include/cuinfer/weights.h) and the C
// ABI of the GGUF reader (include/cri.h, cri_gguf_*).
#include "../../include/cuinfer/weights.h"

#include <hip/hip_runtime_api.h>

#include <cstring>
#include <stdexcept>
#include <string>

#include "../../include/cri.h"
#include "../../include/cuinfer/hip_utils.h"
#include "internal.hpp"

namespace cuinfer {

WeightFormat ggml_type_to_weight_format(GGMLType type) {
    switch (type) {
        case GGMLType::F32: return WeightFormat::FP32;
        case GGMLType::F16: return WeightFormat::FP16;
        case GGMLType::Q8_0: return WeightFormat::Q8_0;
        case GGMLType::Q4_0: return WeightFormat::Q4_0;
        case GGMLType::Q5_0: return WeightFormat::Q5_0;
        case GGMLType::Q4_K: return WeightFormat::Q4_K;
        case GGMLType::Q6_K: return WeightFormat::Q6_K;
        default: break;
    }
    throw std::runtime_error(std::string("GGML type ") + ggml_type_name(type) + " is not a weight format of this library");
}

static DType dtype_of(WeightFormat f) {
    switch (f) {
        case WeightFormat::FP16: return DType::FP16;
        case WeightFormat::Q8_0: return DType::Q8_0;
        case WeightFormat::Q4_0: return DType::Q4_0;
        case WeightFormat::Q5_0: return DType::Q5_0;
        case WeightFormat::Q4_K: return DType::Q4_K;
        case WeightFormat::Q6_K: return DType::Q6_K;
        default: return DType::FP32;
    }
}

static Tensor upload_2d(const GGUFParser& parser, const GGUFTensorInfo& info, WeightFormat& out_format) {
    if (info.dimensions.size() != 2)
        throw std::runtime_error("load_weight_quantized: expected a 2-D tensor for '" + info.name + "', got " +
                                 std::to_string(info.dimensions.size()) + "-D");
    out_format = ggml_type_to_weight_format(info.type);
    // the matmuls take N and K as int: larger dimensions cannot be multiplied, only misread
    constexpr uint64_t kMaxDim = 0x7fffffffu;
    if (info.dimensions[0] == 0 || info.dimensions[1] == 0 || info.dimensions[0] > kMaxDim ||
        info.dimensions[1] > kMaxDim)
        throw std::runtime_error("load_weight_quantized: '" + info.name + "' has dimensions {" +
                                 std::to_string(info.dimensions[0]) + ", " + std::to_string(info.dimensions[1]) +
                                 "}, outside [1, 2^31 - 1]");
    const int64_t K = static_cast<int64_t>(info.dimensions[0]), N = static_cast<int64_t>(info.dimensions[1]);
    Tensor t({N, K}, dtype_of(out_format));
    const size_t bytes = info.byte_size();
    if (t.size_bytes() != bytes)
        throw std::runtime_error("load_weight_quantized: size mismatch for '" + info.name + "'");
    t.copy_from_host(parser.tensor_data(info), bytes);
    return t;
}

Tensor load_weight_quantized(const GGUFParser& parser, const std::string& name, WeightFormat& out_format) {
    const GGUFTensorInfo* info = parser.find_tensor(name);
    if (!info) throw std::runtime_error("load_weight_quantized: tensor '" + name + "' not found in GGUF file");
    return upload_2d(parser, *info, out_format);
}

Tensor load_lm_head(const GGUFParser& parser, WeightFormat& out_format, bool* tied) {
    const GGUFTensorInfo* info = parser.find_tensor("output.weight");
    const bool is_tied = info == nullptr;
    if (is_tied) info = parser.find_tensor("token_embd.weight");
    if (!info) throw std::runtime_error("load_lm_head: neither output.weight nor token_embd.weight is in the file");
    if (tied) *tied = is_tied;
    return upload_2d(parser, *info, out_format);
}

void embedding_lookup(const Tensor& table, WeightFormat format, const int32_t* ids, float* out, int n_ids,
                      hipStream_t stream) {
    int id;
    switch (format) {
        case WeightFormat::FP32: id = CRI_FP32; break;
        case WeightFormat::FP16: id = CRI_FP16; break;
        case WeightFormat::Q8_0: id = CRI_Q8_0; break;
        case WeightFormat::Q4_0: id = CRI_Q4_0; break;
        case WeightFormat::Q5_0: id = CRI_Q5_0; break;
        case WeightFormat::Q4_K: id = CRI_Q4_K; break;
        case WeightFormat::Q6_K: id = CRI_Q6_K; break;
        default: throw std::invalid_argument("embedding_lookup: unknown format");
    }
    const int vocab = static_cast<int>(table.shape(2)), dim = static_cast<int>(table.shape(3));
    CUINFER_CHECK_CRI(cri_embedding_rows(id, table.data(), ids, out, n_ids, dim, vocab, stream));
}

}  // namespace cuinfer

// ---------------------------------------------------------------- C ABI
struct cri_gguf {
    cuinfer::GGUFParser parser;
    explicit cri_gguf(const char* path) : parser(path) {}
};

// abi.cpp: sets the thread's message returned by cri_last_error_string()
void cri_internal_set_error(const char* msg);

namespace {
int gguf_fail(int status, const char* fn, const std::string& what) {
    cri_internal_set_error((std::string(fn) + ": " + what).c_str());
    return status;
}

int ggml_to_format(cuinfer::GGMLType t) {
    switch (t) {
        case cuinfer::GGMLType::Q8_0: return CRI_Q8_0;
        case cuinfer::GGMLType::Q4_0: return CRI_Q4_0;
        case cuinfer::GGMLType::Q5_0: return CRI_Q5_0;
        case cuinfer::GGMLType::Q4_K: return CRI_Q4_K;
        case cuinfer::GGMLType::Q6_K: return CRI_Q6_K;
        case cuinfer::GGMLType::F16: return CRI_FP16;
        case cuinfer::GGMLType::F32: return CRI_FP32;
        default: return -1;
    }
}

template <class F>
int metadata_get(const cri_gguf* g, const char* key, const char* fn, F&& f) {
    if (!g || !key) return gguf_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null argument");
    try {
        f();
        return CRI_OK;
    } catch (const std::exception& e) {
        return gguf_fail(CRI_ERR_SHAPE, fn, e.what());
    }
}
}  // namespace

extern "C" {

int cri_gguf_open(const char* path, cri_gguf** out) {
    const char* fn = "cri_gguf_open";
    if (!path || !out) return gguf_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null argument");
    *out = nullptr;
    try {
        *out = new cri_gguf(path);
        return CRI_OK;
    } catch (const std::exception& e) {
        return gguf_fail(CRI_ERR_FILE, fn, e.what());
    }
}

void cri_gguf_close(cri_gguf* file) { delete file; }

int cri_gguf_version(const cri_gguf* g) { return g ? static_cast<int>(g->parser.version()) : CRI_ERR_INVALID_ARGUMENT; }
long long cri_gguf_tensor_count(const cri_gguf* g) {
    return g ? static_cast<long long>(g->parser.tensor_count()) : CRI_ERR_INVALID_ARGUMENT;
}
long long cri_gguf_metadata_count(const cri_gguf* g) {
    return g ? static_cast<long long>(g->parser.metadata_count()) : CRI_ERR_INVALID_ARGUMENT;
}

int cri_gguf_find_tensor(const cri_gguf* g, const char* name) {
    if (!g || !name) return -1;
    const cuinfer::GGUFTensorInfo* t = g->parser.find_tensor(name);
    return t ? static_cast<int>(t - g->parser.tensors().data()) : -1;
}

int cri_gguf_tensor_info(const cri_gguf* g, int index, cri_gguf_tensor* out) {
    const char* fn = "cri_gguf_tensor_info";
    if (!g || !out) return gguf_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null argument");
    const auto& ts = g->parser.tensors();
    if (index < 0 || static_cast<size_t>(index) >= ts.size())
        return gguf_fail(CRI_ERR_INVALID_ARGUMENT, fn, "index " + std::to_string(index) + " out of range");
    const auto& t = ts[index];
    std::memset(out, 0, sizeof *out);
    out->name = t.name.c_str();
    out->ggml_type = static_cast<int>(t.type);
    out->format = ggml_to_format(t.type);
    out->n_dims = static_cast<int>(t.dimensions.size());
    for (size_t d = 0; d < t.dimensions.size() && d < 8; ++d) out->dims[d] = static_cast<long long>(t.dimensions[d]);
    try {
        out->n_elements = static_cast<long long>(t.element_count());
    } catch (const std::exception&) {
        out->n_elements = -1;  // the dimensions' product overflows (a tensor of a type not checked at open)
    }
    try {
        out->byte_size = static_cast<long long>(t.byte_size());
    } catch (const std::exception&) {
        out->byte_size = -1;  // a type this reader does not know
    }
    out->data_offset = static_cast<long long>(t.data_offset);
    return CRI_OK;
}

const void* cri_gguf_tensor_data(const cri_gguf* g, int index) {
    if (!g || index < 0 || static_cast<size_t>(index) >= g->parser.tensors().size()) return nullptr;
    return g->parser.tensor_data(g->parser.tensors()[index]);
}

int cri_gguf_metadata_type(const cri_gguf* g, const char* key) {
    if (!g || !key) return -1;
    auto it = g->parser.metadata().find(key);
    return it == g->parser.metadata().end() ? -1 : static_cast<int>(it->second.type);
}

int cri_gguf_get_u32(const cri_gguf* g, const char* key, unsigned* out) {
    return metadata_get(g, key, "cri_gguf_get_u32", [&] { *out = g->parser.get_uint32(key); });
}
int cri_gguf_get_i32(const cri_gguf* g, const char* key, int* out) {
    return metadata_get(g, key, "cri_gguf_get_i32", [&] { *out = g->parser.get_int32(key); });
}
int cri_gguf_get_u64(const cri_gguf* g, const char* key, unsigned long long* out) {
    return metadata_get(g, key, "cri_gguf_get_u64", [&] { *out = g->parser.get_uint64(key); });
}
int cri_gguf_get_f32(const cri_gguf* g, const char* key, float* out) {
    return metadata_get(g, key, "cri_gguf_get_f32", [&] { *out = g->parser.get_float32(key); });
}
int cri_gguf_get_string(const cri_gguf* g, const char* key, const char** out) {
    return metadata_get(g, key, "cri_gguf_get_string", [&] {
        auto it = g->parser.metadata().find(key);
        if (it == g->parser.metadata().end()) throw std::runtime_error(std::string("GGUF metadata key not found: ") + key);
        *out = it->second.as_string().c_str();
    });
}
long long cri_gguf_get_array_length(const cri_gguf* g, const char* key) {
    long long n = 0;
    const int rc = metadata_get(g, key, "cri_gguf_get_array_length", [&] {
        auto it = g->parser.metadata().find(key);
        if (it == g->parser.metadata().end()) throw std::runtime_error(std::string("GGUF metadata key not found: ") + key);
        n = static_cast<long long>(it->second.as_array().size());
    });
    return rc == CRI_OK ? n : rc;
}

int cri_gguf_model_params(const cri_gguf* g, cri_gguf_model* out) {
    const char* fn = "cri_gguf_model_params";
    if (!g || !out) return gguf_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null argument");
    std::memset(out, 0, sizeof *out);
    const auto& P = g->parser;
    try {
        const std::string arch = P.architecture();
        std::strncpy(out->architecture, arch.c_str(), sizeof out->architecture - 1);
    } catch (const std::exception& e) {
        return gguf_fail(CRI_ERR_SHAPE, fn, e.what());
    }
    unsigned* fields[] = {&out->context_length, &out->embedding_length, &out->block_count,
                          &out->head_count, &out->head_count_kv, &out->feed_forward_length,
                          &out->rope_dimension_count, &out->vocab_size};
    uint32_t (cuinfer::GGUFParser::*getters[])() const = {
        &cuinfer::GGUFParser::context_length, &cuinfer::GGUFParser::embedding_length,
        &cuinfer::GGUFParser::block_count, &cuinfer::GGUFParser::head_count,
        &cuinfer::GGUFParser::head_count_kv, &cuinfer::GGUFParser::feed_forward_length,
        &cuinfer::GGUFParser::rope_dimension_count, &cuinfer::GGUFParser::vocab_size};
    for (int i = 0; i < 8; ++i) {
        try {
            *fields[i] = (P.*getters[i])();
        } catch (const std::exception&) {
            out->missing |= 1u << i;
        }
    }
    out->rope_freq_base = P.rope_freq_base();
    out->rms_norm_eps = P.rms_norm_eps();
    out->tie_word_embeddings = P.tie_word_embeddings() ? 1 : 0;
    return CRI_OK;
}

int cri_gguf_upload(const cri_gguf* g, int index, void* device_dst, long long dst_bytes, hipStream_t stream) {
    const char* fn = "cri_gguf_upload";
    cri_gguf_tensor info;
    const int rc = cri_gguf_tensor_info(g, index, &info);
    if (rc != CRI_OK) return rc;
    if (!device_dst) return gguf_fail(CRI_ERR_INVALID_ARGUMENT, fn, "null destination");
    if (info.byte_size < 0) return gguf_fail(CRI_ERR_UNSUPPORTED, fn, "tensor of an unknown GGML type");
    if (dst_bytes < info.byte_size)
        return gguf_fail(CRI_ERR_SHAPE, fn,
                         "destination holds " + std::to_string(dst_bytes) + " bytes, tensor '" + info.name +
                             "' has " + std::to_string(info.byte_size));
    const hipError_t e = hipMemcpyAsync(device_dst, cri_gguf_tensor_data(g, index), static_cast<size_t>(info.byte_size),
                                        hipMemcpyHostToDevice, stream);
    if (e != hipSuccess) return gguf_fail(CRI_ERR_LAUNCH, fn, std::string("hipMemcpyAsync: ") + hipGetErrorString(e));
    // the source is the file mapping: finish before returning so the caller may close the file
    const hipError_t s = hipStreamSynchronize(stream);
    if (s != hipSuccess) return gguf_fail(CRI_ERR_LAUNCH, fn, std::string("hipStreamSynchronize: ") + hipGetErrorString(s));
    return CRI_OK;
}

}  // extern "C"

// gguf_parser.h -- GGUF files (the on-disk format of the weights this library
// multiplies): header, metadata, tensor directory, memory-mapped tensor data.
//
// Same interface and semantics as the reference's parser
// (ref:include/cuinfer/gguf_parser.h:1-253, ref:src/gguf_parser.cpp): versions 2
// and 3, the 13 metadata value types (arrays nest), typed getters that throw
// std::runtime_error on a missing key or a type mismatch, the model helpers
// with their defaults, tensor data 32-byte aligned unless `general.alignment`
// says otherwise.  One deliberate difference: a tensor whose data would lie
// past the end of the file, or whose element count is not a multiple of its
// block size, is rejected when the file is opened (the reference returns a
// pointer past its mapping).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <unordered_map>
#include <variant>
#include <vector>

namespace cuinfer {

constexpr uint32_t GGUF_MAGIC = 0x46554747;  // "GGUF", little-endian
constexpr uint32_t GGUF_VERSION_3 = 3;
constexpr size_t GGUF_DEFAULT_ALIGNMENT = 32;

// Metadata value type tags (GGUF specification).
enum class GGUFValueType : uint32_t {
    UINT8 = 0,
    INT8 = 1,
    UINT16 = 2,
    INT16 = 3,
    UINT32 = 4,
    INT32 = 5,
    FLOAT32 = 6,
    BOOL = 7,
    STRING = 8,
    ARRAY = 9,
    UINT64 = 10,
    INT64 = 11,
    FLOAT64 = 12,
};
const char* gguf_value_type_name(GGUFValueType type);

// Tensor data type tags (GGML).
enum class GGMLType : uint32_t {
    F32 = 0,
    F16 = 1,
    Q4_0 = 2,
    Q4_1 = 3,
    Q5_0 = 6,
    Q5_1 = 7,
    Q8_0 = 8,
    Q8_1 = 9,
    Q2_K = 10,
    Q3_K = 11,
    Q4_K = 12,
    Q5_K = 13,
    Q6_K = 14,
};
const char* ggml_type_name(GGMLType type);
// Bytes per block and elements per block (1 for F32/F16); std::runtime_error for an
// unknown type.  Q2_K and Q3_K are 84 and 110 bytes per 256 elements (the GGML block
// layouts; the reference's table lists 256 for both, ref:src/gguf_parser.cpp:87-88).
size_t ggml_type_size(GGMLType type);
size_t ggml_block_size(GGMLType type);

struct GGUFValue {
    GGUFValueType type;
    using ValueVariant = std::variant<uint8_t, int8_t, uint16_t, int16_t, uint32_t, int32_t, float, bool, std::string,
                                      std::vector<GGUFValue>, uint64_t, int64_t, double>;
    ValueVariant value;

    // Each throws std::runtime_error unless the value has exactly that type.
    uint8_t as_uint8() const;
    int8_t as_int8() const;
    uint16_t as_uint16() const;
    int16_t as_int16() const;
    uint32_t as_uint32() const;
    int32_t as_int32() const;
    float as_float32() const;
    bool as_bool() const;
    const std::string& as_string() const;
    const std::vector<GGUFValue>& as_array() const;
    uint64_t as_uint64() const;
    int64_t as_int64() const;
    double as_float64() const;
};

struct GGUFTensorInfo {
    std::string name;
    std::vector<uint64_t> dimensions;  // dimensions[0] is the innermost (K of an [N, K] weight)
    GGMLType type;
    uint64_t offset;       // within the data section, as stored
    uint64_t data_offset;  // from the start of the file

    size_t byte_size() const;  // throws if the element count is not a multiple of the block size
    uint64_t element_count() const;
};

class GGUFParser {
public:
    explicit GGUFParser(const std::string& file_path);
    ~GGUFParser();
    GGUFParser(const GGUFParser&) = delete;
    GGUFParser& operator=(const GGUFParser&) = delete;
    GGUFParser(GGUFParser&&) noexcept;
    GGUFParser& operator=(GGUFParser&&) noexcept;

    uint32_t version() const;
    uint64_t tensor_count() const;
    uint64_t metadata_count() const;

    const std::unordered_map<std::string, GGUFValue>& metadata() const;
    bool has_metadata(const std::string& key) const;
    std::string get_string(const std::string& key) const;
    uint32_t get_uint32(const std::string& key) const;
    int32_t get_int32(const std::string& key) const;
    uint64_t get_uint64(const std::string& key) const;
    float get_float32(const std::string& key) const;

    std::string architecture() const;       // general.architecture
    uint32_t context_length() const;        // {arch}.context_length
    uint32_t embedding_length() const;      // {arch}.embedding_length
    uint32_t block_count() const;           // {arch}.block_count
    uint32_t head_count() const;            // {arch}.attention.head_count
    uint32_t head_count_kv() const;         // {arch}.attention.head_count_kv
    uint32_t feed_forward_length() const;   // {arch}.feed_forward_length
    float rope_freq_base() const;           // {arch}.rope.freq_base, default 10000
    float rms_norm_eps() const;             // {arch}.attention.layer_norm_rms_epsilon, default 1e-5
    uint32_t rope_dimension_count() const;  // {arch}.rope.dimension_count
    uint32_t vocab_size() const;            // {arch}.vocab_size, else the tokenizer.ggml.tokens length
    bool tie_word_embeddings() const;       // no output.weight tensor

    const std::vector<GGUFTensorInfo>& tensors() const;
    const GGUFTensorInfo* find_tensor(const std::string& name) const;  // nullptr if absent
    // Host pointer into the mapped file, valid while the parser lives.
    const void* tensor_data(const GGUFTensorInfo& info) const;
    const void* tensor_data(const std::string& name) const;  // throws if absent

    void print_info() const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace cuinfer

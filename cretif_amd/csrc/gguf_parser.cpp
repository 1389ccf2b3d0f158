// gguf_parser.cpp -- GGUF reader (include/cuinfer/gguf_parser.h).
//
// The file is memory-mapped read-only; every read goes through a cursor that
// checks it against the mapping, so a malformed or truncated file raises
// std::runtime_error instead of reading past the end.  Counts that cannot fit
// in the bytes left (an array of 2^60 elements in a 1 KB file) are rejected
// before anything is allocated.
#include "../../include/cuinfer/gguf_parser.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <stdexcept>

namespace cuinfer {

const char* gguf_value_type_name(GGUFValueType type) {
    static const char* const names[] = {"UINT8", "INT8",  "UINT16", "INT16", "UINT32", "INT32", "FLOAT32",
                                        "BOOL",  "STRING", "ARRAY", "UINT64", "INT64", "FLOAT64"};
    const uint32_t t = static_cast<uint32_t>(type);
    return t < 13 ? names[t] : "UNKNOWN";
}

namespace {

struct TypeInfo {
    GGMLType type;
    const char* name;
    size_t bytes, elems;
};
// GGML block layouts
constexpr TypeInfo kTypes[] = {
    {GGMLType::F32, "F32", 4, 1},        {GGMLType::F16, "F16", 2, 1},       {GGMLType::Q4_0, "Q4_0", 18, 32},
    {GGMLType::Q4_1, "Q4_1", 20, 32},    {GGMLType::Q5_0, "Q5_0", 22, 32},   {GGMLType::Q5_1, "Q5_1", 24, 32},
    {GGMLType::Q8_0, "Q8_0", 34, 32},    {GGMLType::Q8_1, "Q8_1", 36, 32},   {GGMLType::Q2_K, "Q2_K", 84, 256},
    {GGMLType::Q3_K, "Q3_K", 110, 256},  {GGMLType::Q4_K, "Q4_K", 144, 256}, {GGMLType::Q5_K, "Q5_K", 176, 256},
    {GGMLType::Q6_K, "Q6_K", 210, 256},
};

const TypeInfo* type_info(GGMLType type) {
    for (const auto& t : kTypes)
        if (t.type == type) return &t;
    return nullptr;
}

[[noreturn]] void bad_type(const char* fn, GGMLType type) {
    throw std::runtime_error(std::string(fn) + ": unsupported GGML type " + std::to_string(static_cast<uint32_t>(type)));
}

}  // namespace

const char* ggml_type_name(GGMLType type) {
    const TypeInfo* t = type_info(type);
    return t ? t->name : "UNKNOWN";
}
size_t ggml_type_size(GGMLType type) {
    const TypeInfo* t = type_info(type);
    if (!t) bad_type("ggml_type_size", type);
    return t->bytes;
}
size_t ggml_block_size(GGMLType type) {
    const TypeInfo* t = type_info(type);
    if (!t) bad_type("ggml_block_size", type);
    return t->elems;
}

// ---------------------------------------------------------------- GGUFValue
namespace {
template <class T>
const T& value_as(const GGUFValue& v, GGUFValueType want) {
    if (v.type != want)
        throw std::runtime_error(std::string("GGUFValue type mismatch: expected ") + gguf_value_type_name(want) +
                                 ", got " + gguf_value_type_name(v.type));
    return std::get<T>(v.value);
}
}  // namespace

uint8_t GGUFValue::as_uint8() const { return value_as<uint8_t>(*this, GGUFValueType::UINT8); }
int8_t GGUFValue::as_int8() const { return value_as<int8_t>(*this, GGUFValueType::INT8); }
uint16_t GGUFValue::as_uint16() const { return value_as<uint16_t>(*this, GGUFValueType::UINT16); }
int16_t GGUFValue::as_int16() const { return value_as<int16_t>(*this, GGUFValueType::INT16); }
uint32_t GGUFValue::as_uint32() const { return value_as<uint32_t>(*this, GGUFValueType::UINT32); }
int32_t GGUFValue::as_int32() const { return value_as<int32_t>(*this, GGUFValueType::INT32); }
float GGUFValue::as_float32() const { return value_as<float>(*this, GGUFValueType::FLOAT32); }
bool GGUFValue::as_bool() const { return value_as<bool>(*this, GGUFValueType::BOOL); }
const std::string& GGUFValue::as_string() const { return value_as<std::string>(*this, GGUFValueType::STRING); }
const std::vector<GGUFValue>& GGUFValue::as_array() const {
    return value_as<std::vector<GGUFValue>>(*this, GGUFValueType::ARRAY);
}
uint64_t GGUFValue::as_uint64() const { return value_as<uint64_t>(*this, GGUFValueType::UINT64); }
int64_t GGUFValue::as_int64() const { return value_as<int64_t>(*this, GGUFValueType::INT64); }
double GGUFValue::as_float64() const { return value_as<double>(*this, GGUFValueType::FLOAT64); }

// ---------------------------------------------------------------- tensor info
uint64_t GGUFTensorInfo::element_count() const {
    if (dimensions.empty()) return 0;
    uint64_t n = 1;
    for (uint64_t d : dimensions)
        if (__builtin_mul_overflow(n, d, &n))
            throw std::runtime_error("Tensor '" + name + "': the product of its dimensions overflows 64 bits");
    return n;
}

size_t GGUFTensorInfo::byte_size() const {
    const uint64_t n = element_count();
    const size_t be = ggml_block_size(type), bb = ggml_type_size(type);
    if (n % be != 0)
        throw std::runtime_error("Tensor '" + name + "' has " + std::to_string(n) +
                                 " elements, not a multiple of its block size " + std::to_string(be));
    uint64_t bytes;
    if (__builtin_mul_overflow(n / be, static_cast<uint64_t>(bb), &bytes))
        throw std::runtime_error("Tensor '" + name + "': its byte size overflows 64 bits");
    return static_cast<size_t>(bytes);
}

// ---------------------------------------------------------------- reader
namespace {

class Cursor {
public:
    Cursor(const uint8_t* p, size_t n) : p_(p), n_(n) {}
    size_t pos() const { return pos_; }
    size_t left() const { return n_ - pos_; }
    void need(size_t k, const char* what) const {
        if (k > left())
            throw std::runtime_error(std::string("GGUF: truncated file (") + what + " at byte " +
                                     std::to_string(pos_) + " needs " + std::to_string(k) + " bytes, " +
                                     std::to_string(left()) + " left)");
    }
    template <class T>
    T get(const char* what) {
        need(sizeof(T), what);
        T v;
        std::memcpy(&v, p_ + pos_, sizeof(T));
        pos_ += sizeof(T);
        return v;
    }
    std::string str(const char* what) {
        const uint64_t len = get<uint64_t>(what);
        need(static_cast<size_t>(len > left() ? left() + 1 : len), what);
        std::string s(reinterpret_cast<const char*>(p_ + pos_), static_cast<size_t>(len));
        pos_ += static_cast<size_t>(len);
        return s;
    }

private:
    const uint8_t* p_;
    size_t n_;
    size_t pos_ = 0;
};

constexpr int kMaxArrayDepth = 16;

GGUFValue read_value(Cursor& c, GGUFValueType type, int depth) {
    GGUFValue v;
    v.type = type;
    switch (type) {
        case GGUFValueType::UINT8: v.value = c.get<uint8_t>("uint8"); break;
        case GGUFValueType::INT8: v.value = c.get<int8_t>("int8"); break;
        case GGUFValueType::UINT16: v.value = c.get<uint16_t>("uint16"); break;
        case GGUFValueType::INT16: v.value = c.get<int16_t>("int16"); break;
        case GGUFValueType::UINT32: v.value = c.get<uint32_t>("uint32"); break;
        case GGUFValueType::INT32: v.value = c.get<int32_t>("int32"); break;
        case GGUFValueType::FLOAT32: v.value = c.get<float>("float32"); break;
        case GGUFValueType::BOOL: v.value = c.get<uint8_t>("bool") != 0; break;
        case GGUFValueType::STRING: v.value = c.str("string"); break;
        case GGUFValueType::UINT64: v.value = c.get<uint64_t>("uint64"); break;
        case GGUFValueType::INT64: v.value = c.get<int64_t>("int64"); break;
        case GGUFValueType::FLOAT64: v.value = c.get<double>("float64"); break;
        case GGUFValueType::ARRAY: {
            if (depth >= kMaxArrayDepth) throw std::runtime_error("GGUF: arrays nested too deeply");
            const auto et = static_cast<GGUFValueType>(c.get<uint32_t>("array type"));
            const uint64_t count = c.get<uint64_t>("array length");
            if (count > c.left())  // every element takes at least one byte
                throw std::runtime_error("GGUF: array of " + std::to_string(count) + " elements in " +
                                         std::to_string(c.left()) + " remaining bytes");
            std::vector<GGUFValue> items;
            items.reserve(static_cast<size_t>(count));
            for (uint64_t i = 0; i < count; ++i) items.push_back(read_value(c, et, depth + 1));
            v.value = std::move(items);
            break;
        }
        default:
            throw std::runtime_error("GGUF: unknown metadata value type " +
                                     std::to_string(static_cast<uint32_t>(type)));
    }
    return v;
}

}  // namespace

struct GGUFParser::Impl {
    std::string path;
    const uint8_t* map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t tensor_count = 0, kv_count = 0;
    std::unordered_map<std::string, GGUFValue> metadata;
    std::vector<GGUFTensorInfo> tensors;
    std::unordered_map<std::string, size_t> by_name;
    size_t data_start = 0;

    ~Impl() {
        if (map) munmap(const_cast<uint8_t*>(map), size);
    }
};

GGUFParser::GGUFParser(const std::string& file_path) : impl_(new Impl) {
    Impl& I = *impl_;
    I.path = file_path;
    const int fd = open(file_path.c_str(), O_RDONLY);
    if (fd < 0) throw std::runtime_error("GGUF: cannot open '" + file_path + "': " + std::strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        throw std::runtime_error("GGUF: cannot stat '" + file_path + "'");
    }
    I.size = static_cast<size_t>(st.st_size);
    constexpr size_t kHeader = 4 + 4 + 8 + 8;
    if (I.size < kHeader) {
        close(fd);
        throw std::runtime_error("GGUF: file too small for the header (" + std::to_string(I.size) + " bytes, need " +
                                 std::to_string(kHeader) + ")");
    }
    void* m = mmap(nullptr, I.size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) throw std::runtime_error("GGUF: cannot map '" + file_path + "'");
    I.map = static_cast<const uint8_t*>(m);

    Cursor c(I.map, I.size);
    const uint32_t magic = c.get<uint32_t>("magic");
    if (magic != GGUF_MAGIC) {
        char buf[96];
        std::snprintf(buf, sizeof buf, "Invalid GGUF magic: expected 0x%08x, got 0x%08x", GGUF_MAGIC, magic);
        throw std::runtime_error(buf);
    }
    I.version = c.get<uint32_t>("version");
    if (I.version < 2 || I.version > 3)
        throw std::runtime_error("Unsupported GGUF version: " + std::to_string(I.version) + " (supported: 2, 3)");
    I.tensor_count = c.get<uint64_t>("tensor count");
    I.kv_count = c.get<uint64_t>("metadata count");
    if (I.kv_count > c.left() || I.tensor_count > c.left())
        throw std::runtime_error("GGUF: counts exceed the file size");
    for (uint64_t i = 0; i < I.kv_count; ++i) {
        std::string key = c.str("metadata key");
        const auto t = static_cast<GGUFValueType>(c.get<uint32_t>("metadata type"));
        I.metadata[std::move(key)] = read_value(c, t, 0);
    }
    I.tensors.reserve(static_cast<size_t>(I.tensor_count));
    for (uint64_t i = 0; i < I.tensor_count; ++i) {
        GGUFTensorInfo info;
        info.name = c.str("tensor name");
        const uint32_t nd = c.get<uint32_t>("tensor rank");
        if (nd > 8) throw std::runtime_error("GGUF: tensor '" + info.name + "' has " + std::to_string(nd) + " dims");
        info.dimensions.resize(nd);
        for (uint32_t d = 0; d < nd; ++d) info.dimensions[d] = c.get<uint64_t>("tensor dim");
        info.type = static_cast<GGMLType>(c.get<uint32_t>("tensor type"));
        info.offset = c.get<uint64_t>("tensor offset");
        info.data_offset = 0;
        I.tensors.push_back(std::move(info));
    }
    size_t align = GGUF_DEFAULT_ALIGNMENT;
    auto it = I.metadata.find("general.alignment");
    if (it != I.metadata.end() && it->second.type == GGUFValueType::UINT32 && it->second.as_uint32() != 0)
        align = it->second.as_uint32();
    I.data_start = (c.pos() + align - 1) / align * align;
    for (size_t i = 0; i < I.tensors.size(); ++i) {
        GGUFTensorInfo& t = I.tensors[i];
        t.data_offset = I.data_start + t.offset;
        if (type_info(t.type)) {  // tensors of unknown types are listed; their data is not checked
            const size_t bytes = t.byte_size();
            if (t.offset > I.size || t.data_offset > I.size || bytes > I.size - t.data_offset)
                throw std::runtime_error("GGUF: tensor '" + t.name + "' (" + std::to_string(bytes) + " bytes at " +
                                         std::to_string(t.data_offset) + ") lies past the end of the file (" +
                                         std::to_string(I.size) + " bytes)");
        }
        I.by_name.emplace(t.name, i);
    }
}

GGUFParser::~GGUFParser() = default;
GGUFParser::GGUFParser(GGUFParser&&) noexcept = default;
GGUFParser& GGUFParser::operator=(GGUFParser&&) noexcept = default;

uint32_t GGUFParser::version() const { return impl_->version; }
uint64_t GGUFParser::tensor_count() const { return impl_->tensor_count; }
uint64_t GGUFParser::metadata_count() const { return impl_->kv_count; }
const std::unordered_map<std::string, GGUFValue>& GGUFParser::metadata() const { return impl_->metadata; }
bool GGUFParser::has_metadata(const std::string& key) const { return impl_->metadata.count(key) != 0; }

namespace {
const GGUFValue& lookup(const std::unordered_map<std::string, GGUFValue>& md, const std::string& key) {
    auto it = md.find(key);
    if (it == md.end()) throw std::runtime_error("GGUF metadata key not found: " + key);
    return it->second;
}
}  // namespace

std::string GGUFParser::get_string(const std::string& key) const { return lookup(impl_->metadata, key).as_string(); }
uint32_t GGUFParser::get_uint32(const std::string& key) const { return lookup(impl_->metadata, key).as_uint32(); }
int32_t GGUFParser::get_int32(const std::string& key) const { return lookup(impl_->metadata, key).as_int32(); }
uint64_t GGUFParser::get_uint64(const std::string& key) const { return lookup(impl_->metadata, key).as_uint64(); }
float GGUFParser::get_float32(const std::string& key) const { return lookup(impl_->metadata, key).as_float32(); }

std::string GGUFParser::architecture() const { return get_string("general.architecture"); }
uint32_t GGUFParser::context_length() const { return get_uint32(architecture() + ".context_length"); }
uint32_t GGUFParser::embedding_length() const { return get_uint32(architecture() + ".embedding_length"); }
uint32_t GGUFParser::block_count() const { return get_uint32(architecture() + ".block_count"); }
uint32_t GGUFParser::head_count() const { return get_uint32(architecture() + ".attention.head_count"); }
uint32_t GGUFParser::head_count_kv() const { return get_uint32(architecture() + ".attention.head_count_kv"); }
uint32_t GGUFParser::feed_forward_length() const { return get_uint32(architecture() + ".feed_forward_length"); }
float GGUFParser::rope_freq_base() const {
    const std::string key = architecture() + ".rope.freq_base";
    return has_metadata(key) ? get_float32(key) : 10000.0f;
}
float GGUFParser::rms_norm_eps() const {
    const std::string key = architecture() + ".attention.layer_norm_rms_epsilon";
    return has_metadata(key) ? get_float32(key) : 1e-5f;
}
uint32_t GGUFParser::rope_dimension_count() const { return get_uint32(architecture() + ".rope.dimension_count"); }
uint32_t GGUFParser::vocab_size() const {
    const std::string key = architecture() + ".vocab_size";
    if (has_metadata(key)) return get_uint32(key);
    auto it = impl_->metadata.find("tokenizer.ggml.tokens");
    if (it != impl_->metadata.end()) return static_cast<uint32_t>(it->second.as_array().size());
    throw std::runtime_error("Cannot determine vocab_size: neither '" + key +
                             "' nor 'tokenizer.ggml.tokens' is in the metadata");
}
bool GGUFParser::tie_word_embeddings() const { return find_tensor("output.weight") == nullptr; }

const std::vector<GGUFTensorInfo>& GGUFParser::tensors() const { return impl_->tensors; }
const GGUFTensorInfo* GGUFParser::find_tensor(const std::string& name) const {
    auto it = impl_->by_name.find(name);
    return it == impl_->by_name.end() ? nullptr : &impl_->tensors[it->second];
}
const void* GGUFParser::tensor_data(const GGUFTensorInfo& info) const { return impl_->map + info.data_offset; }
const void* GGUFParser::tensor_data(const std::string& name) const {
    const GGUFTensorInfo* t = find_tensor(name);
    if (!t) throw std::runtime_error("GGUF: tensor not found: " + name);
    return tensor_data(*t);
}

void GGUFParser::print_info() const {
    const Impl& I = *impl_;
    std::printf("GGUF file:      %s\n", I.path.c_str());
    std::printf("Version:        %u\n", I.version);
    std::printf("Tensors:        %llu\n", static_cast<unsigned long long>(I.tensor_count));
    std::printf("Metadata keys:  %llu\n", static_cast<unsigned long long>(I.kv_count));
    std::printf("Data section:   byte %zu\n", I.data_start);
    for (const auto& kv : I.metadata) std::printf("  %-48s %s\n", kv.first.c_str(), gguf_value_type_name(kv.second.type));
    for (const auto& t : I.tensors) {
        std::printf("  %-40s %-5s [", t.name.c_str(), ggml_type_name(t.type));
        for (size_t d = 0; d < t.dimensions.size(); ++d)
            std::printf("%s%llu", d ? ", " : "", static_cast<unsigned long long>(t.dimensions[d]));
        std::printf("] @%llu\n", static_cast<unsigned long long>(t.data_offset));
    }
}

}  // namespace cuinfer

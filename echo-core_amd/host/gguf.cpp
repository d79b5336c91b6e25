// gguf.cpp — GGUF v3 reader (include/gguf_reader.h, include/echo_gguf.h) and
// the GGUF -> device loader of the hybrid decoder.
//
// File format (GGUF v3, little endian): magic "GGUF", u32 version, u64 tensor
// count, u64 metadata count, metadata (string key, u32 value type, value),
// tensor infos (string name, u32 n_dims, u64 ne[n_dims], u32 ggml type, u64
// offset), then the tensor data section at the next multiple of
// general.alignment.  The reference parses the same layout in
// src/gguf_reader.cpp:275-433 and echo-core-zig/src/gguf/reader.zig:128-190.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "echo_engine.h"
#include "echo_gguf.h"
#include "echo_hip.h"
#include "gguf_reader.h"
#include "types.h"

extern "C" int ec_set_error(int code, const char* msg);

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF"

enum : uint32_t {
    V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
    V_STRING = 8, V_ARRAY = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12,
};

// Elements per block and bytes per block of each ggml type (ggml's type
// traits; 0 = not a storage type this reader sizes).
struct TypeSize {
    uint32_t elems, bytes;
};
TypeSize type_size(GGMLType t) {
    switch (t) {
        case GGMLType::F32: return {1, 4};
        case GGMLType::F16: return {1, 2};
        case GGMLType::BF16: return {1, 2};
        case GGMLType::F64: return {1, 8};
        case GGMLType::I8: return {1, 1};
        case GGMLType::I16: return {1, 2};
        case GGMLType::I32: return {1, 4};
        case GGMLType::Q4_0: return {32, 18};
        case GGMLType::Q4_1: return {32, 20};
        case GGMLType::Q5_0: return {32, 22};
        case GGMLType::Q5_1: return {32, 24};
        case GGMLType::Q8_0: return {32, 34};
        case GGMLType::Q8_1: return {32, 36};
        case GGMLType::Q2_K: return {256, 84};
        case GGMLType::Q3_K: return {256, 110};
        case GGMLType::Q4_K: return {256, 144};
        case GGMLType::Q5_K: return {256, 176};
        case GGMLType::Q6_K: return {256, 210};
        case GGMLType::IQ2_XXS: return {256, 66};
        case GGMLType::IQ2_XS: return {256, 74};
        case GGMLType::IQ2_S: return {256, 82};
        case GGMLType::IQ3_XXS: return {256, 98};
        case GGMLType::IQ1_S: return {256, 50};
        case GGMLType::IQ4_NL: return {32, 18};
        case GGMLType::IQ4_XS: return {256, 136};
        case GGMLType::Q4_0_4_4:
        case GGMLType::Q4_0_4_8:
        case GGMLType::Q4_0_8_8: return {32, 18};
        default: return {0, 0};
    }
}

// Bounds-checked little-endian cursor over the mapped file.
struct Cursor {
    const uint8_t* p;
    size_t n, at = 0;
    void need(size_t k) const {
        if (k > n - at) throw std::runtime_error("GGUF: truncated file (read past end at byte " + std::to_string(at) + ")");
    }
    template <class T>
    T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p + at, sizeof(T));
        at += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t len = get<uint64_t>();
        need(len);
        std::string s((const char*)p + at, (size_t)len);
        at += len;
        return s;
    }
};

// An array of n elements of at least `min_bytes` each must fit in the rest of
// the file (absurd counts fail before anything is allocated).
void check_count(const Cursor& c, uint64_t n, size_t min_bytes) {
    if (n > (c.n - c.at) / min_bytes) throw std::runtime_error("GGUF: array length exceeds the file");
}

template <class T, class W>
std::vector<W> read_array(Cursor& c, uint64_t n) {
    check_count(c, n, sizeof(T));
    std::vector<W> v;
    v.reserve((size_t)n);
    for (uint64_t i = 0; i < n; ++i) v.push_back((W)c.get<T>());
    return v;
}

GGUFValue read_value(Cursor& c, uint32_t type) {
    switch (type) {
        case V_U8: return (uint64_t)c.get<uint8_t>();
        case V_I8: return (int64_t)c.get<int8_t>();
        case V_U16: return (uint64_t)c.get<uint16_t>();
        case V_I16: return (int64_t)c.get<int16_t>();
        case V_U32: return (uint64_t)c.get<uint32_t>();
        case V_I32: return (int64_t)c.get<int32_t>();
        case V_F32: return (double)c.get<float>();
        case V_BOOL: return c.get<uint8_t>() != 0;
        case V_STRING: return c.str();
        case V_U64: return c.get<uint64_t>();
        case V_I64: return c.get<int64_t>();
        case V_F64: return c.get<double>();
        case V_ARRAY: {
            const uint32_t et = c.get<uint32_t>();
            const uint64_t n = c.get<uint64_t>();
            switch (et) {
                case V_U8: return read_array<uint8_t, uint64_t>(c, n);
                case V_I8: return read_array<int8_t, int64_t>(c, n);
                case V_U16: return read_array<uint16_t, uint64_t>(c, n);
                case V_I16: return read_array<int16_t, int64_t>(c, n);
                case V_U32: return read_array<uint32_t, uint64_t>(c, n);
                case V_I32: return read_array<int32_t, int64_t>(c, n);
                case V_U64: return read_array<uint64_t, uint64_t>(c, n);
                case V_I64: return read_array<int64_t, int64_t>(c, n);
                case V_F32: return read_array<float, double>(c, n);
                case V_F64: return read_array<double, double>(c, n);
                case V_BOOL: {
                    check_count(c, n, 1);
                    std::vector<bool> v;
                    for (uint64_t i = 0; i < n; ++i) v.push_back(c.get<uint8_t>() != 0);
                    return v;
                }
                case V_STRING: {
                    check_count(c, n, 8);
                    std::vector<std::string> v;
                    for (uint64_t i = 0; i < n; ++i) v.push_back(c.str());
                    return v;
                }
                default: throw std::runtime_error("GGUF: unsupported array element type " + std::to_string(et));
            }
        }
        default: throw std::runtime_error("GGUF: unknown metadata value type " + std::to_string(type));
    }
}

bool as_u64(const GGUFValue& v, uint64_t& out) {
    if (auto p = std::get_if<uint64_t>(&v)) return out = *p, true;
    if (auto p = std::get_if<int64_t>(&v)) return *p >= 0 ? (out = (uint64_t)*p, true) : false;
    return false;
}

bool ends_with(const std::string& s, const std::string& suf) {
    return s.size() >= suf.size() && s.compare(s.size() - suf.size(), suf.size(), suf) == 0;
}

}  // namespace

GGMLType ggml_type_from_uint32(uint32_t v) {
    if (v < (uint32_t)GGMLType::COUNT) return (GGMLType)v;
    throw std::runtime_error("GGUF: unknown GGML type id " + std::to_string(v));
}

struct ec_gguf {
    std::unique_ptr<GGUFReader> r;
};

GGUFReader::GGUFReader(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) throw std::runtime_error("GGUF: cannot open '" + path + "'");
    struct stat st;
    if (::fstat(fd, &st) != 0 || st.st_size < 24) {
        ::close(fd);
        throw std::runtime_error("GGUF: '" + path + "' is too small to be a GGUF file");
    }
    size_ = (size_t)st.st_size;
    void* m = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) throw std::runtime_error("GGUF: mmap of '" + path + "' failed");
    map_ = (const uint8_t*)m;
    try {
        Cursor c{map_, size_};
        const uint32_t magic = c.get<uint32_t>();
        if (magic != kMagic) throw std::runtime_error("GGUF: bad magic (expected \"GGUF\")");
        const uint32_t version = c.get<uint32_t>();
        if (version != 3) throw std::runtime_error("GGUF: unsupported version " + std::to_string(version) + " (expected 3)");
        const uint64_t n_tensors = c.get<uint64_t>();
        const uint64_t n_kv = c.get<uint64_t>();
        for (uint64_t i = 0; i < n_kv; ++i) {
            std::string key = c.str();
            const uint32_t type = c.get<uint32_t>();
            metadata_[key] = read_value(c, type);
        }
        // architecture prefix: the key in front of one of these suffixes
        static const char* kSuffixes[] = {".context_length", ".embedding_length", ".block_count",
                                          ".feed_forward_length", ".attention.head_count",
                                          ".attention.head_count_kv"};
        for (const auto& kv : metadata_) {
            for (const char* s : kSuffixes)
                if (kv.first.size() > strlen(s) && ends_with(kv.first, s)) {
                    model_prefix_ = kv.first.substr(0, kv.first.size() - strlen(s) + 1);
                    break;
                }
            if (!model_prefix_.empty()) break;
        }
        for (uint64_t i = 0; i < n_tensors; ++i) {
            std::string name = c.str();
            const uint32_t nd = c.get<uint32_t>();
            if (nd == 0 || nd > 4) throw std::runtime_error("GGUF: tensor '" + name + "' has " + std::to_string(nd) + " dims");
            std::vector<uint64_t> shape(nd);
            uint64_t n = 1;
            for (uint32_t d = 0; d < nd; ++d) {
                shape[d] = c.get<uint64_t>();
                if (shape[d] != 0 && n > UINT64_MAX / shape[d])
                    throw std::runtime_error("GGUF: tensor '" + name + "' has an element count that overflows");
                n *= shape[d];
            }
            const GGMLType t = ggml_type_from_uint32(c.get<uint32_t>());
            const uint64_t off = c.get<uint64_t>();
            const TypeSize ts = type_size(t);
            if (ts.elems == 0) throw std::runtime_error("GGUF: tensor '" + name + "' has an unsized type");
            if (n % ts.elems) throw std::runtime_error("GGUF: tensor '" + name + "' is not a whole number of blocks");
            if (tensors_.count(name)) throw std::runtime_error("GGUF: duplicate tensor '" + name + "'");
            order_.push_back(name);
            tensors_[name] = TensorInfo{off, n / ts.elems * ts.bytes, std::move(shape), t};
        }
        const uint64_t align = (uint64_t)alignment();
        if (align == 0) throw std::runtime_error("GGUF: general.alignment is 0");
        data_offset_ = (off_t)((c.at + align - 1) / align * align);
        if ((uint64_t)data_offset_ > (uint64_t)size_) throw std::runtime_error("GGUF: data section past the end of the file");
        const uint64_t data_bytes = (uint64_t)size_ - (uint64_t)data_offset_;
        for (const auto& kv : tensors_)  // two comparisons: offset + size could wrap
            if (kv.second.offset > data_bytes || kv.second.size > data_bytes - kv.second.offset)
                throw std::runtime_error("GGUF: tensor '" + kv.first + "' extends past the end of the file");
        // model config (reference field semantics; head_dim from key_length when present)
        auto u = [&](const char* suffix) -> uint64_t {
            auto it = metadata_.find(model_prefix_ + suffix);
            uint64_t v = 0;
            return (it != metadata_.end() && as_u64(it->second, v)) ? v : 0;
        };
        config_.max_seq_len = (uint32_t)u("context_length");
        config_.hidden_dim = (uint32_t)u("embedding_length");
        config_.num_layers = (uint32_t)u("block_count");
        config_.ffn_hidden_dim = (uint32_t)u("feed_forward_length");
        config_.num_heads = (uint32_t)u("attention.head_count");
        const uint64_t kvh = u("attention.head_count_kv");
        config_.num_kv_heads = kvh ? (uint32_t)kvh : config_.num_heads;
        config_.head_dim = config_.num_heads ? config_.hidden_dim / config_.num_heads : 0;
        if (const uint64_t kl = u("attention.key_length")) config_.head_dim = (uint32_t)kl;
        uint64_t vocab = u("vocab_size");
        if (!vocab) {
            auto it = metadata_.find("vocab_size");
            if (it != metadata_.end()) as_u64(it->second, vocab);
        }
        auto tok = metadata_.find("tokenizer.ggml.tokens");
        if (tok != metadata_.end())
            if (auto p = std::get_if<std::vector<std::string>>(&tok->second)) tokens_ = *p;
        if (!vocab) vocab = tokens_.size();
        if (!vocab) {  // the embedding's row count when the metadata names none
            auto emb = tensors_.find("token_embd.weight");
            if (emb != tensors_.end() && emb->second.shape.size() >= 2) vocab = emb->second.shape[1];
        }
        config_.vocab_size = (uint32_t)vocab;
        config_.ffn_type = config_.ffn_hidden_dim ? ModelConfig::FFNType::GatedSwiGLU : ModelConfig::FFNType::Dense;
        config_.norm_type = ModelConfig::NormType::RMSNorm;
        config_.pos_encoding = ModelConfig::PosEncoding::RoPE;
        config_.use_kv_quantization = false;
        config_.ssm_inner_size = (uint32_t)u("ssm.inner_size");
        config_.ssm_num_heads = (uint32_t)u("ssm.time_step_rank");
        config_.ssm_conv_kernel = (uint32_t)u("ssm.conv_kernel");
        config_.full_attention_interval = (uint32_t)u("full_attention_interval");
        auto rb = metadata_.find(model_prefix_ + "rope.freq_base");
        if (rb != metadata_.end())
            if (auto p = std::get_if<double>(&rb->second)) config_.rope_base = (float)*p;
    } catch (...) {
        ::munmap((void*)map_, size_);
        map_ = nullptr;
        throw;
    }
}

GGUFReader::~GGUFReader() {
    if (map_) ::munmap((void*)map_, size_);
}

int GGUFReader::alignment() const {
    auto it = metadata_.find("general.alignment");
    uint64_t v = 0;
    if (it != metadata_.end() && as_u64(it->second, v)) return (int)v;
    return 32;
}

const uint8_t* GGUFReader::tensor_data(const std::string& name) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end()) throw std::runtime_error("GGUF: tensor '" + name + "' not found");
    return map_ + data_offset_ + it->second.offset;
}

std::vector<uint8_t> GGUFReader::load_tensor(const std::string& name) const {
    const uint8_t* p = tensor_data(name);
    return std::vector<uint8_t>(p, p + tensors_.at(name).size);
}

const TensorInfo* GGUFReader::find_tensor_by_suffix(const std::string& suffix) const {
    for (const auto& kv : tensors_)
        if (ends_with(kv.first, suffix)) return &kv.second;
    return nullptr;
}

void GGUFReader::assert_alignment(int align) const {
    if (align <= 0) throw std::runtime_error("GGUF: alignment must be positive");
    for (const auto& kv : tensors_)
        if (kv.second.offset % (uint64_t)align)
            throw std::runtime_error("GGUF: tensor '" + kv.first + "' offset " + std::to_string(kv.second.offset) +
                                     " is not aligned to " + std::to_string(align) + " bytes");
}

// ------------------------------------------------------------------- C ABI
namespace {
int fail(const std::exception& ex) { return ec_set_error(EC_ERR_ARG, ex.what()); }

void fill(const GGUFReader& r, const std::string& name, const TensorInfo& t, ec_gguf_tensor* out) {
    out->name = r.tensors().find(name)->first.c_str();
    out->type = (uint32_t)t.dtype;
    out->n_dims = (uint32_t)t.shape.size();
    for (int d = 0; d < 4; ++d) out->shape[d] = d < (int)t.shape.size() ? t.shape[d] : 1;
    out->offset = t.offset;
    out->bytes = t.size;
    out->data = r.tensor_data(name);
}
}  // namespace

extern "C" int ec_gguf_open(const char* path, ec_gguf** out) {
    if (!path || !out) return ec_set_error(EC_ERR_ARG, "ec_gguf_open: null argument");
    *out = nullptr;
    auto g = std::make_unique<ec_gguf>();
    try {
        g->r = std::make_unique<GGUFReader>(path);
    } catch (const std::exception& ex) {
        return fail(ex);
    }
    *out = g.release();
    return EC_OK;
}

extern "C" void ec_gguf_close(ec_gguf* g) { delete g; }

extern "C" uint64_t ec_gguf_tensor_count(const ec_gguf* g) { return g ? g->r->tensor_names().size() : 0; }

extern "C" int ec_gguf_tensor_at(const ec_gguf* g, uint64_t i, ec_gguf_tensor* out) {
    if (!g || !out || i >= g->r->tensor_names().size()) return ec_set_error(EC_ERR_ARG, "ec_gguf_tensor_at: bad argument");
    const std::string& n = g->r->tensor_names()[i];
    fill(*g->r, n, g->r->tensors().at(n), out);
    return EC_OK;
}

extern "C" int ec_gguf_find_tensor(const ec_gguf* g, const char* name, ec_gguf_tensor* out) {
    if (!g || !name || !out) return ec_set_error(EC_ERR_ARG, "ec_gguf_find_tensor: null argument");
    auto it = g->r->tensors().find(name);
    if (it == g->r->tensors().end())
        return ec_set_error(EC_ERR_ARG, (std::string("GGUF: tensor '") + name + "' not found").c_str());
    fill(*g->r, it->first, it->second, out);
    return EC_OK;
}

extern "C" int ec_gguf_get_uint(const ec_gguf* g, const char* key, uint64_t* out) {
    if (!g || !key || !out) return ec_set_error(EC_ERR_ARG, "ec_gguf_get_uint: null argument");
    auto it = g->r->metadata().find(key);
    if (it == g->r->metadata().end() || !as_u64(it->second, *out))
        return ec_set_error(EC_ERR_ARG, (std::string("GGUF: no unsigned integer '") + key + "'").c_str());
    return EC_OK;
}

extern "C" int ec_gguf_get_float(const ec_gguf* g, const char* key, double* out) {
    if (!g || !key || !out) return ec_set_error(EC_ERR_ARG, "ec_gguf_get_float: null argument");
    auto it = g->r->metadata().find(key);
    if (it != g->r->metadata().end()) {
        if (auto p = std::get_if<double>(&it->second)) return *out = *p, EC_OK;
        if (auto p = std::get_if<uint64_t>(&it->second)) return *out = (double)*p, EC_OK;
        if (auto p = std::get_if<int64_t>(&it->second)) return *out = (double)*p, EC_OK;
    }
    return ec_set_error(EC_ERR_ARG, (std::string("GGUF: no number '") + key + "'").c_str());
}

extern "C" int ec_gguf_get_string(const ec_gguf* g, const char* key, const char** out) {
    if (!g || !key || !out) return ec_set_error(EC_ERR_ARG, "ec_gguf_get_string: null argument");
    auto it = g->r->metadata().find(key);
    if (it != g->r->metadata().end())
        if (auto p = std::get_if<std::string>(&it->second)) return *out = p->c_str(), EC_OK;
    return ec_set_error(EC_ERR_ARG, (std::string("GGUF: no string '") + key + "'").c_str());
}

extern "C" uint64_t ec_gguf_token_count(const ec_gguf* g) { return g ? g->r->tokens().size() : 0; }

extern "C" const char* ec_gguf_token(const ec_gguf* g, uint64_t i) {
    return (g && i < g->r->tokens().size()) ? g->r->tokens()[i].c_str() : nullptr;
}

extern "C" uint32_t ec_gguf_alignment(const ec_gguf* g) { return g ? (uint32_t)g->r->alignment() : 0; }

extern "C" uint64_t ec_gguf_data_offset(const ec_gguf* g) { return g ? (uint64_t)g->r->data_offset() : 0; }

extern "C" const char* ec_gguf_arch_prefix(const ec_gguf* g) { return g ? g->r->model_prefix().c_str() : nullptr; }

// ------------------------------------------------------ GGUF -> engine loader
namespace {
bool has(const GGUFReader& r, const std::string& n) { return r.tensors().count(n) != 0; }

std::string blk(uint32_t l, const char* s) { return "blk." + std::to_string(l) + "." + s; }

// The engine's storage format of a ggml type (-1: not one it stores).
int engine_fmt(GGMLType t) {
    switch (t) {
        case GGMLType::Q8_0: return EC_Q8_0;
        case GGMLType::Q4_K: return EC_Q4_K;
        case GGMLType::F16: return EC_F16;
        case GGMLType::F32: return EC_F32;
        default: return -1;
    }
}

const char* type_name(GGMLType t) {
    switch (t) {
        case GGMLType::Q8_0: return "Q8_0";
        case GGMLType::Q4_K: return "Q4_K";
        case GGMLType::F16: return "F16";
        case GGMLType::F32: return "F32";
        default: return "another type";
    }
}

// Tensors by kind, each in the formats the reference reads it in
// (src/inference.cpp:526-545 dispatches matrices per dtype; norms and the
// embedding are fp16 there, :233-237): matrices Q8_0 or Q4_K, vectors F32 or
// F16 (widened to fp32 here, exactly), the embedding Q8_0, F16 or F32.
struct Loader {
    const GGUFReader& r;
    ec_engine* e;
    const TensorInfo& need(const std::string& n, std::initializer_list<GGMLType> ok_types, uint64_t ne0,
                           uint64_t ne1) {
        auto it = r.tensors().find(n);
        if (it == r.tensors().end()) throw std::runtime_error("GGUF: tensor '" + n + "' not found");
        const TensorInfo& ti = it->second;
        const uint64_t s1 = ti.shape.size() > 1 ? ti.shape[1] : 1;
        bool ok = ti.shape[0] == ne0 && s1 == ne1;
        for (size_t d = 2; d < ti.shape.size(); ++d) ok = ok && ti.shape[d] == 1;
        if (!ok)
            throw std::runtime_error("GGUF: tensor '" + n + "' must be [" + std::to_string(ne0) + ", " +
                                     std::to_string(ne1) + "]");
        bool type_ok = false;
        std::string names;
        for (GGMLType t : ok_types) {
            type_ok = type_ok || ti.dtype == t;
            names += std::string(names.empty() ? "" : " or ") + type_name(t);
        }
        if (!type_ok)
            throw std::runtime_error("GGUF: tensor '" + n + "' is " + type_name(ti.dtype) + ", must be " + names);
        return ti;
    }
    void set(uint32_t layer, int id, const void* p, size_t bytes) {
        if (ec_engine_set_tensor(e, (int)layer, id, p, bytes) != EC_OK)
            throw std::runtime_error(std::string("GGUF load: ") + ec_last_error());
    }
    void format(uint32_t layer, int id, GGMLType t, const std::string& n) {
        if (ec_engine_set_format(e, (int)layer, id, engine_fmt(t)) != EC_OK)
            throw std::runtime_error("GGUF load: '" + n + "': " + ec_last_error());
    }
    // fp32 vector from an F32 or F16 tensor
    void vec(uint32_t layer, int id, const std::string& n, uint64_t ne0, uint64_t ne1) {
        const TensorInfo& ti = need(n, {GGMLType::F32, GGMLType::F16}, ne0, ne1);
        if (ti.dtype == GGMLType::F32) return set(layer, id, r.tensor_data(n), ti.size);
        const uint8_t* src = r.tensor_data(n);
        std::vector<float> v(ne0 * ne1);
        for (size_t i = 0; i < v.size(); ++i) {
            fp16_t h;
            memcpy(&h, src + 2 * i, 2);
            v[i] = fp16_to_fp32(h);
        }
        set(layer, id, v.data(), v.size() * sizeof(float));
    }
    // one matrix, stored in its own format
    void mat(uint32_t layer, int id, const std::string& n, uint64_t ne0, uint64_t ne1) {
        const TensorInfo& ti = need(n, {GGMLType::Q8_0, GGMLType::Q4_K}, ne0, ne1);
        format(layer, id, ti.dtype, n);
        set(layer, id, r.tensor_data(n), ti.size);
    }
    // rows of several matrices (same K, one format) stacked in order into one
    // engine matrix
    void stack(uint32_t layer, int id, const std::vector<std::pair<std::string, uint64_t>>& parts, uint64_t K) {
        std::vector<uint8_t> buf;
        GGMLType t0 = GGMLType::Q8_0;
        for (size_t i = 0; i < parts.size(); ++i) {
            const auto& p = parts[i];
            const TensorInfo& ti = need(p.first, {GGMLType::Q8_0, GGMLType::Q4_K}, K, p.second);
            if (i == 0) t0 = ti.dtype;
            if (ti.dtype != t0)
                throw std::runtime_error("GGUF: '" + p.first + "' is " + type_name(ti.dtype) + " but '" +
                                         parts[0].first + "' is " + type_name(t0) +
                                         ": the fused projection needs one format");
            const uint8_t* d = r.tensor_data(p.first);
            buf.insert(buf.end(), d, d + ti.size);
        }
        format(layer, id, t0, parts[0].first);
        set(layer, id, buf.data(), buf.size());
    }
};
}  // namespace

extern "C" int ec_gguf_engine_config(const ec_gguf* g, uint32_t max_batch, uint32_t max_ctx, ec_engine_cfg* out) {
    if (!g || !out || max_batch == 0 || max_ctx == 0) return ec_set_error(EC_ERR_ARG, "ec_gguf_engine_config: bad argument");
    try {
        const GGUFReader& r = *g->r;
        const std::string& p = r.model_prefix();
        auto u = [&](const char* s, uint64_t dflt) -> uint64_t {
            auto it = r.metadata().find(p + s);
            uint64_t v = 0;
            return (it != r.metadata().end() && as_u64(it->second, v)) ? v : dflt;
        };
        ec_engine_cfg c{};
        const ModelConfig& m = r.config();
        c.hidden = m.hidden_dim;
        c.n_layers = m.num_layers;
        c.ffn = m.ffn_hidden_dim;
        c.n_heads = m.num_heads;
        c.n_kv = m.num_kv_heads;
        c.head_dim = m.head_dim;
        c.ssm_inner = (uint32_t)u("ssm.inner_size", 0);
        c.ssm_heads = (uint32_t)u("ssm.time_step_rank", 0);
        c.conv_kernel = (uint32_t)u("ssm.conv_kernel", 4);
        auto emb = r.tensors().find("token_embd.weight");
        if (emb == r.tensors().end() || emb->second.shape.size() < 2)
            throw std::runtime_error("GGUF: token_embd.weight [hidden, vocab] not found");
        c.vocab = (uint32_t)emb->second.shape[1];
        // attention interval: metadata, else the first block with attention weights
        uint64_t interval = u("full_attention_interval", 0);
        if (!interval) {
            for (uint32_t l = 0; l < c.n_layers && !interval; ++l)
                if (has(r, blk(l, "attn_q.weight"))) interval = l + 1;
            if (!interval) throw std::runtime_error("GGUF: no attention block and no full_attention_interval");
        }
        c.attn_interval = (uint32_t)interval;
        double base = 10000.0;
        ec_gguf_get_float(g, (p + "rope.freq_base").c_str(), &base);
        c.rope_base = (float)base;
        c.max_batch = max_batch;
        c.max_ctx = max_ctx;
        for (uint32_t l = 0; l < c.n_layers; ++l) {
            const bool attn = (l + 1) % c.attn_interval == 0;
            const bool delta = has(r, blk(l, "ssm_out.weight"));
            if (attn == delta)
                throw std::runtime_error("GGUF: block " + std::to_string(l) + (attn ? " should be attention" : " should be delta-net") +
                                         " with attention interval " + std::to_string(c.attn_interval));
        }
        if (c.hidden == 0 || c.n_layers == 0 || c.ffn == 0 || c.n_heads == 0 || c.vocab == 0)
            throw std::runtime_error("GGUF: incomplete model metadata");
        *out = c;
        return EC_OK;
    } catch (const std::exception& ex) {
        return fail(ex);
    }
}

// Upload the decoder's tensors from a parsed file (shared by the C ABI and the
// InferenceEngine facade); throws on a missing or mis-shaped tensor.
void ec_load_gguf_tensors(ec_engine* e, const GGUFReader& r) {
    ec_engine_cfg c;
    if (ec_engine_get_config(e, &c) != EC_OK) throw std::runtime_error(ec_last_error());
    {
        Loader L{r, e};
        const uint64_t H = c.hidden, F = c.ffn, V = c.vocab;
        const uint64_t q_dim = (uint64_t)c.n_heads * c.head_dim, kv_dim = (uint64_t)c.n_kv * c.head_dim;
        const uint64_t value_dim = c.ssm_inner, key_dim = c.ssm_inner / 2, conv_dim = 2 * key_dim + value_dim;
        const TensorInfo& emb = L.need("token_embd.weight", {GGMLType::Q8_0, GGMLType::F16, GGMLType::F32}, H, V);
        L.format(0, EC_T_EMBED, emb.dtype, "token_embd.weight");
        L.set(0, EC_T_EMBED, r.tensor_data("token_embd.weight"), emb.size);
        L.vec(0, EC_T_FINAL_NORM, "output_norm.weight", H, 1);
        L.mat(0, EC_T_LM_HEAD, has(r, "output.weight") ? "output.weight" : "token_embd.weight", H, V);
        for (uint32_t l = 0; l < c.n_layers; ++l) {
            const bool attn = (l + 1) % c.attn_interval == 0;
            L.vec(l, EC_T_ATTN_NORM, blk(l, "attn_norm.weight"), H, 1);
            const std::string fn = has(r, blk(l, "post_attention_norm.weight")) ? blk(l, "post_attention_norm.weight")
                                                                              : blk(l, "ffn_norm.weight");
            L.vec(l, EC_T_FFN_NORM, fn, H, 1);
            // gate and up are one engine matrix: one format for both
            const TensorInfo& gate = L.need(blk(l, "ffn_gate.weight"), {GGMLType::Q8_0, GGMLType::Q4_K}, H, F);
            const TensorInfo& up = L.need(blk(l, "ffn_up.weight"), {GGMLType::Q8_0, GGMLType::Q4_K}, H, F);
            if (gate.dtype != up.dtype)
                throw std::runtime_error("GGUF: block " + std::to_string(l) + " ffn_gate is " + type_name(gate.dtype) +
                                         ", ffn_up " + type_name(up.dtype) + ": gate and up need one format");
            L.format(l, EC_T_W_GATE, gate.dtype, blk(l, "ffn_gate.weight"));
            L.set(l, EC_T_W_GATE, r.tensor_data(blk(l, "ffn_gate.weight")), gate.size);
            L.set(l, EC_T_W_UP, r.tensor_data(blk(l, "ffn_up.weight")), up.size);
            L.mat(l, EC_T_W_DOWN, blk(l, "ffn_down.weight"), F, H);
            if (attn) {
                L.stack(l, EC_T_W_IN, {{blk(l, "attn_q.weight"), q_dim}, {blk(l, "attn_k.weight"), kv_dim},
                                       {blk(l, "attn_v.weight"), kv_dim}}, H);
                L.mat(l, EC_T_W_OUT, blk(l, "attn_output.weight"), q_dim, H);
                const std::vector<float> zero(c.head_dim, 0.0f);
                const char* norms[2] = {"attn_q_norm.weight", "attn_k_norm.weight"};
                const int ids[2] = {EC_T_Q_NORM, EC_T_K_NORM};
                for (int i = 0; i < 2; ++i) {
                    if (has(r, blk(l, norms[i])))
                        L.vec(l, ids[i], blk(l, norms[i]), c.head_dim, 1);
                    else
                        L.set(l, ids[i], zero.data(), zero.size() * 4);
                }
            } else {
                L.stack(l, EC_T_W_IN, {{blk(l, "attn_qkv.weight"), conv_dim}, {blk(l, "attn_gate.weight"), value_dim},
                                       {blk(l, "ssm_alpha.weight"), c.ssm_heads},
                                       {blk(l, "ssm_beta.weight"), c.ssm_heads}}, H);
                L.mat(l, EC_T_W_OUT, blk(l, "ssm_out.weight"), value_dim, H);
                L.vec(l, EC_T_CONV_W, blk(l, "ssm_conv1d.weight"), c.conv_kernel, conv_dim);
                L.vec(l, EC_T_A_LOG, blk(l, "ssm_a"), c.ssm_heads, 1);
                L.vec(l, EC_T_DT_BIAS, blk(l, "ssm_dt.bias"), c.ssm_heads, 1);
                L.vec(l, EC_T_SSM_NORM, blk(l, "ssm_norm.weight"), 128, 1);
            }
        }
    }
}

extern "C" int ec_engine_load_gguf(ec_engine* e, const ec_gguf* g) {
    if (!e || !g) return ec_set_error(EC_ERR_ARG, "ec_engine_load_gguf: null argument");
    try {
        ec_load_gguf_tensors(e, *g->r);
        return EC_OK;
    } catch (const std::exception& ex) {
        return fail(ex);
    }
}

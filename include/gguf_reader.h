// gguf_reader.h — GGUF v3 reader with the reference's interface
// (include/gguf_reader.h:1-120 of echo-core): same enum values, value variant,
// TensorInfo fields and public GGUFReader members, so code written against the
// reference's header compiles against this one and links libechohip.so.
//
// Implementation (echo-core_amd/host/gguf.cpp) maps the file read-only and
// parses it with bounds checks; errors throw std::runtime_error as the
// reference does.  Semantics that follow the GGUF v3 specification and the
// reference's Zig reader (echo-core-zig/src/gguf/reader.zig:186,491-506)
// rather than the C++ reader:
//   - tensor data starts at the end of the tensor infos rounded up to
//     alignment() ("general.alignment", default 32), and TensorInfo::offset is
//     relative to that start; load_tensor() reads data_offset() + offset;
//   - TensorInfo::size of a block-quantized tensor counts whole blocks of the
//     type's own block length (32 elements for Q4_0..Q8_1, 256 for the K and IQ
//     quants);
//   - config().head_dim is "<arch>.attention.key_length" when present.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <sys/types.h>
#include <unordered_map>
#include <variant>
#include <vector>

#include "config.h"

// GGML tensor types (ggml type ids as stored in GGUF tensor infos).
enum class GGMLType : uint32_t {
    F32 = 0,
    F16 = 1,
    Q4_0 = 2,
    Q4_1 = 3,
    Q5_0 = 4,
    Q5_1 = 5,
    Q8_0 = 6,
    Q8_1 = 7,
    Q2_K = 8,
    Q3_K = 9,
    Q4_K = 10,
    Q5_K = 11,
    Q6_K = 12,
    IQ2_XXS = 13,
    IQ2_XS = 14,
    I16 = 15,
    F64 = 16,
    IQ1_S = 17,
    IQ4_NL = 18,
    IQ4_XS = 19,
    I8 = 20,
    I32 = 21,
    IQ2_S = 22,
    IQ3_XXS = 23,
    BF16 = 24,
    Q4_0_4_4 = 25,
    Q4_0_4_8 = 26,
    Q4_0_8_8 = 27,
    COUNT,
};

// Throws std::runtime_error for ids >= COUNT.
GGMLType ggml_type_from_uint32(uint32_t v);

struct TensorInfo {
    uint64_t offset;             // relative to GGUFReader::data_offset()
    uint64_t size;               // bytes
    std::vector<uint64_t> shape; // ne0 (fastest) first
    GGMLType dtype;
};

// Metadata values: unsigned integers widen to uint64_t, signed to int64_t,
// floats to double; arrays become vectors of the same.
using GGUFValue = std::variant<uint64_t, int64_t, double, bool, std::string, std::vector<uint64_t>,
                               std::vector<int64_t>, std::vector<double>, std::vector<bool>,
                               std::vector<std::string>>;

class GGUFReader {
public:
    explicit GGUFReader(const std::string& path);
    ~GGUFReader();
    GGUFReader(const GGUFReader&) = delete;
    GGUFReader& operator=(const GGUFReader&) = delete;

    const ModelConfig& config() const { return config_; }
    const std::vector<std::string>& tokens() const { return tokens_; }
    const std::unordered_map<std::string, TensorInfo>& tensors() const { return tensors_; }

    // Copy of one tensor's bytes.
    std::vector<uint8_t> load_tensor(const std::string& name) const;

    const std::unordered_map<std::string, GGUFValue>& metadata() const { return metadata_; }

    // "general.alignment" (default 32).
    int alignment() const;

    // File offset of the tensor data section.
    off_t data_offset() const { return data_offset_; }

    // First tensor whose name ends with `suffix` (nullptr if none).
    const TensorInfo* find_tensor_by_suffix(const std::string& suffix) const;

    // Throws if a tensor offset is not a multiple of `align`.
    void assert_alignment(int align = 32) const;

    // Extensions (not in the reference header): the mapped bytes of a tensor
    // (valid while the reader lives), tensor names in file order, the metadata
    // key prefix of the model architecture ("qwen35." etc.) and the file size.
    const uint8_t* tensor_data(const std::string& name) const;
    const std::vector<std::string>& tensor_names() const { return order_; }
    const std::string& model_prefix() const { return model_prefix_; }
    size_t file_size() const { return size_; }

private:
    const uint8_t* map_ = nullptr;
    size_t size_ = 0;
    off_t data_offset_ = 0;
    std::string model_prefix_;
    std::unordered_map<std::string, GGUFValue> metadata_;
    std::vector<std::string> tokens_;
    std::unordered_map<std::string, TensorInfo> tensors_;
    std::vector<std::string> order_;
    ModelConfig config_{};
};

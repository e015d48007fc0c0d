// GGUF v3 index over a read-only memory mapping of the file (host code, no
// HIP).  Parsing follows GGUFReader::load (src/gguf.cpp:371-530): the same
// limits, the same order of checks and the same load_error messages, the
// metadata values rendered as that reader renders them, and the data section
// at the first multiple of general.alignment (default 32) after the header.
// Tensor bytes are not read: tensor_data() points into the mapping, which
// stays valid for as long as the index lives.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace mlq {

// GGML tensor types the format names (include/mini_llama/gguf.h:12-18).
constexpr uint32_t kGgmlF32 = 0;
constexpr uint32_t kGgmlF16 = 1;
constexpr uint32_t kGgmlQ4_0 = 2;
constexpr uint32_t kGgmlQ4_1 = 3;
constexpr uint32_t kGgmlQ8_0 = 8;

struct GgufMeta {
    std::string key;
    uint32_t type = 0;   // GGUF value type (include/mini_llama/gguf.h:27-41)
    std::string value;   // rendered as the reference renders it
    uint64_t value_pos = 0;  // file offset of the value
};

struct GgufTensor {
    std::string name;
    std::vector<uint64_t> dims;  // ne0 (fastest) first
    uint32_t type = 0;           // GGML type
    uint64_t offset = 0;         // from the start of the data section
    uint64_t nbytes = 0;         // 0 for types without a known size
};

class GgufIndex {
public:
    GgufIndex() = default;
    GgufIndex(const GgufIndex&) = delete;
    GgufIndex& operator=(const GgufIndex&) = delete;
    ~GgufIndex();

    // Maps and parses `path`.  Returns false with `error` set on failure.
    bool open(const std::string& path);

    // Start of a tensor's bytes in the mapping (nullptr when it has none).
    const uint8_t* tensor_data(const GgufTensor& t) const;
    // Index of the tensor called `name`, or -1.
    int64_t find(const std::string& name) const;

    // Typed metadata reads with the acceptance rules of gguf_get_metadata_int /
    // _float / _string / _string_array (src/gguf.cpp:674-820): integers of any
    // width and sign, float32 / float64, strings, and the element count of an
    // array of strings.  False when the key is absent or has another type.
    bool get_int(const std::string& key, int64_t& out) const;
    bool get_float(const std::string& key, double& out) const;
    bool get_string(const std::string& key, std::string& out) const;
    bool get_string_array_size(const std::string& key, uint64_t& out) const;

    uint32_t version = 0;
    uint64_t n_tensors = 0;
    uint64_t n_metadata = 0;
    uint64_t data_offset = 0;
    std::vector<GgufMeta> metadata;
    std::vector<GgufTensor> tensors;
    std::string error;

private:
    void unmap();
    const uint8_t* base_ = nullptr;
    uint64_t size_ = 0;
};

const char* ggml_type_label(uint32_t type);    // "F32", "Q4_0", ... "UNKNOWN"
const char* gguf_value_label(uint32_t type);   // "uint32", "string", ... "unknown"

}  // namespace mlq

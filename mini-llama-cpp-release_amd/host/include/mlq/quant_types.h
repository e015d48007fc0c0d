// Host-side types of the quantized-linear path: the f32 tensor and the
// ggml-compatible block formats, as the reference defines them
// (include/mini_llama/tensor.h:11-61, include/mini_llama/quantized_tensor.h:13-114).
// The block structs are the storage contract shared with the GGUF loader and
// the device kernels, so their byte layout is fixed by static_assert.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace mlq {

enum class QuantType { F32 = 0, Q8_0 = 1, Q4_0 = 2, Q4_1 = 3 };

constexpr int kBlockElems = 32;

#pragma pack(push, 1)
struct BlockQ8_0 {
    uint16_t d;     // fp16 scale
    int8_t qs[32];  // element i = d * qs[i]
};
struct BlockQ4_0 {
    uint16_t d;      // fp16 scale
    uint8_t qs[16];  // element j (low nibble) and j+16 (high nibble) = d * (n - 8)
};
struct BlockQ4_1 {
    uint16_t d;      // fp16 scale
    uint16_t m;      // fp16 offset
    uint8_t qs[16];  // element = d * n + m
};
#pragma pack(pop)
static_assert(sizeof(BlockQ8_0) == 34, "BlockQ8_0 is 34 bytes");
static_assert(sizeof(BlockQ4_0) == 18, "BlockQ4_0 is 18 bytes");
static_assert(sizeof(BlockQ4_1) == 20, "BlockQ4_1 is 20 bytes");

inline size_t block_bytes(QuantType t) {
    switch (t) {
        case QuantType::Q8_0: return sizeof(BlockQ8_0);
        case QuantType::Q4_0: return sizeof(BlockQ4_0);
        case QuantType::Q4_1: return sizeof(BlockQ4_1);
        default: return 0;
    }
}

inline std::string shape_string(const std::vector<int>& shape) {
    std::string s = "[";
    for (size_t i = 0; i < shape.size(); ++i) {
        if (i) s += ", ";
        s += std::to_string(shape[i]);
    }
    return s + "]";
}

// Dense f32 host tensor; rejects non-positive dimensions like the reference.
struct Tensor {
    std::vector<float> data;
    std::vector<int> shape;

    Tensor() = default;
    explicit Tensor(const std::vector<int>& s, float fill = 0.0f) : shape(s) {
        size_t n = 1;
        for (size_t a = 0; a < s.size(); ++a) {
            if (s[a] <= 0) {
                throw std::runtime_error("Tensor constructor: dimension at axis " + std::to_string(a) +
                                         " must be positive, got " + std::to_string(s[a]) + " in shape " +
                                         shape_string(s));
            }
            n *= static_cast<size_t>(s[a]);
        }
        data.assign(n, fill);
    }
    size_t size() const { return data.size(); }
    int ndim() const { return static_cast<int>(shape.size()); }
    std::string shape_str() const { return shape_string(shape); }
};

// Tagged quantized weight: exactly one of the vectors is used, per `type`.
struct QuantizedTensor {
    QuantType type = QuantType::F32;
    std::vector<int> shape;  // [out_features, in_features]
    std::vector<float> f32_data;
    std::vector<BlockQ8_0> q8_0_data;
    std::vector<BlockQ4_0> q4_0_data;
    std::vector<BlockQ4_1> q4_1_data;

    const void* blocks() const {
        switch (type) {
            case QuantType::Q8_0: return q8_0_data.data();
            case QuantType::Q4_0: return q4_0_data.data();
            case QuantType::Q4_1: return q4_1_data.data();
            default: return nullptr;
        }
    }
    size_t block_count() const {
        switch (type) {
            case QuantType::Q8_0: return q8_0_data.size();
            case QuantType::Q4_0: return q4_0_data.size();
            case QuantType::Q4_1: return q4_1_data.size();
            default: return 0;
        }
    }
};

}  // namespace mlq

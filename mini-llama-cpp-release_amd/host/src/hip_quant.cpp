// HIP quantized linear, host-side C++ layer over the C ABI (see mlq/hip_quant.h).
//
// The shape validation and the host bias add are mlq/linear_checks.h, shared
// with the drop-in of the reference's device interface (dropin/hip_quant.cpp):
// src/cuda_quant.cu:150-243 and 139-148, 283-285, with "hip" callers.
#include "mlq/hip_quant.h"
#include "mlq/linear_checks.h"

#include "mlq_hip.h"

#include <stdexcept>
#include <string>

namespace mlq {

namespace {

const char* caller_of(QuantType t) {
    switch (t) {
        case QuantType::Q8_0: return "hip_q8_0_linear";
        case QuantType::Q4_0: return "hip_q4_0_linear";
        case QuantType::Q4_1: return "hip_q4_1_linear";
        default: return "hip_linear";
    }
}

[[noreturn]] void throw_abi(const char* caller) {
    const std::string msg = mlq_hip_last_error();
    // The C ABI messages already carry the caller prefix; keep them verbatim.
    if (msg.rfind(caller, 0) == 0) throw std::runtime_error(msg);
    throw std::runtime_error(std::string(caller) + ": " + msg);
}

void validate_shape(const std::vector<int>& xs, const std::string& xstr, const std::vector<int>& ws,
                    size_t block_count, const char* caller) {
    checks::linear_shape(xs, xstr, ws, block_count, caller);
}

void add_bias(Tensor& y, const Tensor& bias, int rows, int cols, const char* caller) {
    checks::add_bias(y.data.data(), bias.shape, bias.data.data(), rows, cols, caller);
}

Tensor device_weight_linear(QuantType t, const Tensor& x, const void* w, size_t count,
                            const std::vector<int>& ws, const Tensor* bias, int device_id) {
    const char* caller = caller_of(t);
    if (w == nullptr) throw std::runtime_error(std::string(caller) + ": device weight pointer is null");
    validate_shape(x.shape, x.shape_str(), ws, count, caller);
    const bool is_1d = x.ndim() == 1;
    const int rows = is_1d ? 1 : x.shape[0];
    const int out = ws[0];
    Tensor y(is_1d ? std::vector<int>{out} : std::vector<int>{rows, out});
    mlq_weight_t h = nullptr;
    if (mlq_hip_wrap_weight(device_id, static_cast<int>(t), w, count, out, ws[1], &h) != MLQ_OK) {
        throw_abi(caller);
    }
    const int rc = mlq_hip_quant_linear(h, x.data.data(), rows, y.data.data(), 0, nullptr);
    mlq_hip_free_weight(h);
    if (rc != MLQ_OK) throw_abi(caller);
    if (bias != nullptr) add_bias(y, *bias, rows, out, caller);
    return y;
}

template <typename Block>
Tensor host_weight_linear(QuantType t, const Tensor& x, const std::vector<Block>& weight,
                          const std::vector<int>& ws, const Tensor* bias, int device_id) {
    validate_shape(x.shape, x.shape_str(), ws, weight.size(), caller_of(t));
    HipDeviceBuffer w(weight.size() * sizeof(Block), device_id);
    w.upload(weight.data(), weight.size() * sizeof(Block));
    return device_weight_linear(t, x, w.data(), weight.size(), ws, bias, device_id);
}

HipTensor device_input_linear(QuantType t, const HipTensor& x, const void* w, size_t count,
                              const std::vector<int>& ws, int device_id) {
    const char* caller = caller_of(t);
    if (w == nullptr) throw std::runtime_error(std::string(caller) + ": device weight pointer is null");
    if (x.device_id() != device_id) {
        throw std::runtime_error(std::string(caller) + ": input tensor is on a different HIP device");
    }
    validate_shape(x.shape(), x.shape_str(), ws, count, caller);
    const bool is_1d = x.ndim() == 1;
    const int rows = is_1d ? 1 : x.shape()[0];
    const int out = ws[0];
    HipTensor y(is_1d ? std::vector<int>{out} : std::vector<int>{rows, out}, device_id);
    if (mlq_hip_quant_linear_device(device_id, static_cast<int>(t), w, count, out, ws[1],
                                    static_cast<const float*>(x.data()), rows, static_cast<float*>(y.data()),
                                    nullptr) != MLQ_OK) {
        throw_abi(caller);
    }
    void* stream = nullptr;
    if (mlq_hip_stream(device_id, &stream) != MLQ_OK || mlq_hip_synchronize(stream) != MLQ_OK) {
        throw_abi(caller);
    }
    return y;
}

}  // namespace

bool hip_quant_built() { return mlq_hip_built() != 0; }

Tensor hip_q8_0_linear(const Tensor& x, const std::vector<BlockQ8_0>& weight, const std::vector<int>& ws,
                       const Tensor* bias, int device_id) {
    return host_weight_linear(QuantType::Q8_0, x, weight, ws, bias, device_id);
}
Tensor hip_q8_0_linear_device_weight(const Tensor& x, const void* w, size_t count, const std::vector<int>& ws,
                                     const Tensor* bias, int device_id) {
    return device_weight_linear(QuantType::Q8_0, x, w, count, ws, bias, device_id);
}
HipTensor hip_q8_0_linear_device_input(const HipTensor& x, const void* w, size_t count,
                                       const std::vector<int>& ws, int device_id) {
    return device_input_linear(QuantType::Q8_0, x, w, count, ws, device_id);
}

Tensor hip_q4_0_linear(const Tensor& x, const std::vector<BlockQ4_0>& weight, const std::vector<int>& ws,
                       const Tensor* bias, int device_id) {
    return host_weight_linear(QuantType::Q4_0, x, weight, ws, bias, device_id);
}
Tensor hip_q4_0_linear_device_weight(const Tensor& x, const void* w, size_t count, const std::vector<int>& ws,
                                     const Tensor* bias, int device_id) {
    return device_weight_linear(QuantType::Q4_0, x, w, count, ws, bias, device_id);
}
HipTensor hip_q4_0_linear_device_input(const HipTensor& x, const void* w, size_t count,
                                       const std::vector<int>& ws, int device_id) {
    return device_input_linear(QuantType::Q4_0, x, w, count, ws, device_id);
}

Tensor hip_q4_1_linear(const Tensor& x, const std::vector<BlockQ4_1>& weight, const std::vector<int>& ws,
                       const Tensor* bias, int device_id) {
    return host_weight_linear(QuantType::Q4_1, x, weight, ws, bias, device_id);
}
Tensor hip_q4_1_linear_device_weight(const Tensor& x, const void* w, size_t count, const std::vector<int>& ws,
                                     const Tensor* bias, int device_id) {
    return device_weight_linear(QuantType::Q4_1, x, w, count, ws, bias, device_id);
}
HipTensor hip_q4_1_linear_device_input(const HipTensor& x, const void* w, size_t count,
                                       const std::vector<int>& ws, int device_id) {
    return device_input_linear(QuantType::Q4_1, x, w, count, ws, device_id);
}

HipUploadedWeight hip_upload_linear_weight(const QuantizedTensor& weight, const std::string& name,
                                           int device_id) {
    const char* tn = weight.type == QuantType::Q8_0 ? "Q8_0" : weight.type == QuantType::Q4_0 ? "Q4_0"
                   : weight.type == QuantType::Q4_1 ? "Q4_1" : "F32";
    if (weight.type == QuantType::F32) {
        throw std::runtime_error("HIP weight upload: F32 weights are not on the quantized path: " + name);
    }
    if (weight.shape.size() != 2) {
        throw std::runtime_error(std::string("HIP weight upload: expected 2D ") + tn + " weight for " + name);
    }
    if (weight.block_count() == 0) {
        throw std::runtime_error(std::string("HIP weight upload: empty ") + tn + " data for " + name);
    }
    const int nb = (weight.shape[1] + kBlockElems - 1) / kBlockElems;
    const size_t expected = static_cast<size_t>(weight.shape[0]) * nb;
    if (weight.block_count() != expected) {
        throw std::runtime_error(std::string("HIP weight upload: ") + tn + " block count mismatch for " + name +
                                 ", expected " + std::to_string(expected) + ", got " +
                                 std::to_string(weight.block_count()));
    }
    HipUploadedWeight up;
    up.name = name;
    up.type = weight.type;
    up.shape = weight.shape;
    up.block_count = weight.block_count();
    const size_t bytes = up.block_count * block_bytes(weight.type);
    up.buffer.reset(bytes, device_id);
    up.buffer.upload(weight.blocks(), bytes);
    return up;
}

int hip_sample_greedy_device(const HipTensor& x, const HipUploadedWeight& w, int device_id) {
    if (w.type != QuantType::Q8_0 && w.type != QuantType::Q4_0 && w.type != QuantType::Q4_1) {
        throw std::runtime_error("HIP greedy sampling unsupported weight type: " + w.name);
    }
    const char* caller = caller_of(w.type);
    if (x.ndim() != 1) {
        throw std::runtime_error(std::string(caller) + ": greedy sampling expects x shape [in_features], got " +
                                 x.shape_str());
    }
    validate_shape(x.shape(), x.shape_str(), w.shape, w.block_count, caller);
    const int qtype = w.type == QuantType::Q8_0 ? MLQ_Q8_0 : w.type == QuantType::Q4_0 ? MLQ_Q4_0 : MLQ_Q4_1;
    mlq_weight_t h = nullptr;
    if (mlq_hip_wrap_weight(device_id, qtype, w.buffer.data(), w.block_count, w.shape[0], w.shape[1], &h) != MLQ_OK) {
        throw_abi(caller);
    }
    int token = -1;
    const int rc = mlq_hip_sample_greedy(h, static_cast<const float*>(x.data()), nullptr, &token, nullptr);
    const std::string msg = rc == MLQ_OK ? std::string() : std::string(mlq_hip_last_error());
    mlq_hip_free_weight(h);
    if (rc != MLQ_OK) throw std::runtime_error(msg);
    return token;
}

HipTensor hip_linear_device(const HipTensor& x, const HipUploadedWeight& w, int device_id) {
    switch (w.type) {
        case QuantType::Q8_0:
            return hip_q8_0_linear_device_input(x, w.buffer.data(), w.block_count, w.shape, device_id);
        case QuantType::Q4_0:
            return hip_q4_0_linear_device_input(x, w.buffer.data(), w.block_count, w.shape, device_id);
        case QuantType::Q4_1:
            return hip_q4_1_linear_device_input(x, w.buffer.data(), w.block_count, w.shape, device_id);
        default:
            throw std::runtime_error("HIP forward linear unsupported weight type: " + w.name);
    }
}

}  // namespace mlq

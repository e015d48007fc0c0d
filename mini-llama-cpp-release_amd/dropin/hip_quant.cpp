// The reference's quantized-linear device interface
// (include/mini_llama/cuda_quant.h: cuda_quant_built and the nine
// cuda_q8_0 / q4_0 / q4_1 _linear{,_device_weight,_device_input} functions on
// Tensor / CudaTensor) on the MI355X HIP kernels: a HIP build of the reference
// compiles this file in place of src/cuda_quant.cpp and src/cuda_quant.cu.
// Validation order and messages are the reference's (src/cuda_quant.cu:139-243,
// 253-255, 299-301; mlq/linear_checks.h, shared with the mlq:: host layer), so
// model.cpp's weight upload (src/model.cpp:145-316), forward.cpp's
// forward_linear / forward_linear_device (src/forward.cpp:172-291) and the
// reference's own tests/test_cuda_quant.cpp run unchanged on the HIP kernels.
#include "mini_llama/cuda_quant.h"
#include "mini_llama/cuda_runtime.h"
#include "mini_llama/cuda_tensor.h"

#include "hip_common.h"
#include "mlq/linear_checks.h"

#include <stdexcept>
#include <string>
#include <vector>

namespace mini_llama {

namespace {

using hipdrop::check;

void validate(const std::vector<int>& xs, const std::string& xstr, const std::vector<int>& ws, size_t blocks,
              const char* caller) {
    mlq::checks::linear_shape(xs, xstr, ws, blocks, caller);
}

void add_bias(Tensor& y, const Tensor& bias, int rows, int cols, const char* caller) {
    mlq::checks::add_bias(y.data.data(), bias.shape, bias.data.data(), rows, cols, caller);
}

// cuda_q*_linear_device_weight: host x and y, device weight blocks.
Tensor device_weight(int qtype, const char* caller, const Tensor& x, const void* w, size_t blocks,
                     const std::vector<int>& ws, const Tensor* bias, int device_id) {
    if (w == nullptr) throw std::runtime_error(std::string(caller) + ": device weight pointer is null");
    validate(x.shape, x.shape_str(), ws, blocks, caller);
    const bool is_1d = x.ndim() == 1;
    const int rows = is_1d ? 1 : x.shape[0];
    const int out = ws[0];
    Tensor y(is_1d ? std::vector<int>{out} : std::vector<int>{rows, out}, 0.0f);
    cuda_set_device(device_id);
    mlq_weight_t h = nullptr;
    check(mlq_hip_wrap_weight(device_id, qtype, w, blocks, out, ws[1], &h), caller);
    const int rc = mlq_hip_quant_linear(h, x.data.data(), rows, y.data.data(), 0, nullptr);
    (void)mlq_hip_free_weight(h);
    check(rc, caller);
    if (bias != nullptr) add_bias(y, *bias, rows, out, caller);
    return y;
}

// cuda_q*_linear: host weight blocks, uploaded for the call.
template <typename Block>
Tensor host_weight(int qtype, const char* caller, const Tensor& x, const std::vector<Block>& weight,
                   const std::vector<int>& ws, const Tensor* bias, int device_id) {
    validate(x.shape, x.shape_str(), ws, weight.size(), caller);
    CudaDeviceBuffer w(weight.size() * sizeof(Block), device_id);
    w.upload(weight.data(), weight.size() * sizeof(Block));
    return device_weight(qtype, caller, x, w.data(), weight.size(), ws, bias, device_id);
}

// cuda_q*_linear_device_input: device x and y (y allocated here).
CudaTensor device_input(int qtype, const char* caller, const CudaTensor& x, const void* w, size_t blocks,
                        const std::vector<int>& ws, int device_id) {
    if (w == nullptr) throw std::runtime_error(std::string(caller) + ": device weight pointer is null");
    if (x.device_id() != device_id) {
        throw std::runtime_error(std::string(caller) + ": input tensor is on a different CUDA device");
    }
    validate(x.shape(), x.shape_str(), ws, blocks, caller);
    const bool is_1d = x.ndim() == 1;
    const int rows = is_1d ? 1 : x.shape()[0];
    const int out = ws[0];
    CudaTensor y(is_1d ? std::vector<int>{out} : std::vector<int>{rows, out}, device_id);
    check(mlq_hip_quant_linear_device(device_id, qtype, w, blocks, out, ws[1], static_cast<const float*>(x.data()),
                                      rows, static_cast<float*>(y.data()), nullptr),
          caller);
    // Asynchronous on the library stream: every later drop-in call on this
    // device is issued there too, and host reads of y synchronize it.
    return y;
}

}  // namespace

bool cuda_quant_built() { return true; }

Tensor cuda_q8_0_linear(const Tensor& x, const std::vector<BlockQ8_0>& weight, const std::vector<int>& weight_shape,
                        const Tensor* bias, int device_id) {
    return host_weight(MLQ_Q8_0, "cuda_q8_0_linear", x, weight, weight_shape, bias, device_id);
}

Tensor cuda_q8_0_linear_device_weight(const Tensor& x, const void* q8_0_device, size_t q8_0_block_count,
                                      const std::vector<int>& weight_shape, const Tensor* bias, int device_id) {
    return device_weight(MLQ_Q8_0, "cuda_q8_0_linear", x, q8_0_device, q8_0_block_count, weight_shape, bias,
                         device_id);
}

CudaTensor cuda_q8_0_linear_device_input(const CudaTensor& x, const void* q8_0_device, size_t q8_0_block_count,
                                         const std::vector<int>& weight_shape, int device_id) {
    return device_input(MLQ_Q8_0, "cuda_q8_0_linear", x, q8_0_device, q8_0_block_count, weight_shape, device_id);
}

Tensor cuda_q4_0_linear(const Tensor& x, const std::vector<BlockQ4_0>& weight, const std::vector<int>& weight_shape,
                        const Tensor* bias, int device_id) {
    return host_weight(MLQ_Q4_0, "cuda_q4_0_linear", x, weight, weight_shape, bias, device_id);
}

Tensor cuda_q4_0_linear_device_weight(const Tensor& x, const void* q4_0_device, size_t q4_0_block_count,
                                      const std::vector<int>& weight_shape, const Tensor* bias, int device_id) {
    return device_weight(MLQ_Q4_0, "cuda_q4_0_linear", x, q4_0_device, q4_0_block_count, weight_shape, bias,
                         device_id);
}

CudaTensor cuda_q4_0_linear_device_input(const CudaTensor& x, const void* q4_0_device, size_t q4_0_block_count,
                                         const std::vector<int>& weight_shape, int device_id) {
    return device_input(MLQ_Q4_0, "cuda_q4_0_linear", x, q4_0_device, q4_0_block_count, weight_shape, device_id);
}

Tensor cuda_q4_1_linear(const Tensor& x, const std::vector<BlockQ4_1>& weight, const std::vector<int>& weight_shape,
                        const Tensor* bias, int device_id) {
    return host_weight(MLQ_Q4_1, "cuda_q4_1_linear", x, weight, weight_shape, bias, device_id);
}

Tensor cuda_q4_1_linear_device_weight(const Tensor& x, const void* q4_1_device, size_t q4_1_block_count,
                                      const std::vector<int>& weight_shape, const Tensor* bias, int device_id) {
    return device_weight(MLQ_Q4_1, "cuda_q4_1_linear", x, q4_1_device, q4_1_block_count, weight_shape, bias,
                         device_id);
}

CudaTensor cuda_q4_1_linear_device_input(const CudaTensor& x, const void* q4_1_device, size_t q4_1_block_count,
                                         const std::vector<int>& weight_shape, int device_id) {
    return device_input(MLQ_Q4_1, "cuda_q4_1_linear", x, q4_1_device, q4_1_block_count, weight_shape, device_id);
}

}  // namespace mini_llama

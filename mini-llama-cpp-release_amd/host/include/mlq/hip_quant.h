// HIP quantized linear, host-side C++ interface.  One function per reference
// entry of include/mini_llama/cuda_quant.h:11-86 with the same argument
// meaning (x [in] or [batch, in]; W [out, in]; optional host bias; device id)
// and the same error behaviour: std::runtime_error whose message starts with
// the caller ("hip_q4_0_linear: block count mismatch: expected N, got M").
// Calls are synchronous for host tensors, as in the reference.
#pragma once

#include "mlq/hip_runtime.h"
#include "mlq/quant_types.h"

#include <memory>
#include <string>
#include <vector>

namespace mlq {

bool hip_quant_built();

Tensor hip_q8_0_linear(const Tensor& x, const std::vector<BlockQ8_0>& weight,
                       const std::vector<int>& weight_shape, const Tensor* bias = nullptr,
                       int device_id = 0);
Tensor hip_q8_0_linear_device_weight(const Tensor& x, const void* q8_0_device, size_t q8_0_block_count,
                                     const std::vector<int>& weight_shape, const Tensor* bias = nullptr,
                                     int device_id = 0);
HipTensor hip_q8_0_linear_device_input(const HipTensor& x, const void* q8_0_device,
                                       size_t q8_0_block_count, const std::vector<int>& weight_shape,
                                       int device_id = 0);

Tensor hip_q4_0_linear(const Tensor& x, const std::vector<BlockQ4_0>& weight,
                       const std::vector<int>& weight_shape, const Tensor* bias = nullptr,
                       int device_id = 0);
Tensor hip_q4_0_linear_device_weight(const Tensor& x, const void* q4_0_device, size_t q4_0_block_count,
                                     const std::vector<int>& weight_shape, const Tensor* bias = nullptr,
                                     int device_id = 0);
HipTensor hip_q4_0_linear_device_input(const HipTensor& x, const void* q4_0_device,
                                       size_t q4_0_block_count, const std::vector<int>& weight_shape,
                                       int device_id = 0);

Tensor hip_q4_1_linear(const Tensor& x, const std::vector<BlockQ4_1>& weight,
                       const std::vector<int>& weight_shape, const Tensor* bias = nullptr,
                       int device_id = 0);
Tensor hip_q4_1_linear_device_weight(const Tensor& x, const void* q4_1_device, size_t q4_1_block_count,
                                     const std::vector<int>& weight_shape, const Tensor* bias = nullptr,
                                     int device_id = 0);
HipTensor hip_q4_1_linear_device_input(const HipTensor& x, const void* q4_1_device,
                                       size_t q4_1_block_count, const std::vector<int>& weight_shape,
                                       int device_id = 0);

// A linear weight resident on a device (cf. CudaUploadedWeight and
// upload_q*_linear_weight, include/mini_llama/model.h:40-47,
// src/model.cpp:145-272).  Validation messages mirror the upload's.
struct HipUploadedWeight {
    std::string name;
    QuantType type = QuantType::F32;
    std::vector<int> shape;
    size_t block_count = 0;
    HipDeviceBuffer buffer;
};

HipUploadedWeight hip_upload_linear_weight(const QuantizedTensor& weight, const std::string& name,
                                           int device_id = 0);

// forward_linear_device-style dispatch on an uploaded weight (src/forward.cpp:172-227).
HipTensor hip_linear_device(const HipTensor& x, const HipUploadedWeight& w, int device_id = 0);

// Greedy token of the logits w . x without downloading them: the output
// projection of compute_logits_device (src/forward.cpp:849-853) followed by
// MiniSampler::sample_greedy (src/sampler.cpp:91-95), i.e. the first index of
// the largest logit.  x is [in_features] on the device.  Throws the sampler's
// "sampler: logits must be finite" when a logit is infinite or NaN.
int hip_sample_greedy_device(const HipTensor& x, const HipUploadedWeight& w, int device_id = 0);

}  // namespace mlq

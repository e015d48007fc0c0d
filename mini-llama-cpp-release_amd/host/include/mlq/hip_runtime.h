// HIP device runtime for the host layer: device queries, an owning device
// buffer and a move-only f32 device tensor.  Mirrors the reference's CUDA
// runtime and tensor (include/mini_llama/cuda_runtime.h:8-77,
// include/mini_llama/cuda_tensor.h:12-63) on top of the C ABI in mlq_hip.h.
// Failures throw std::runtime_error carrying the library's message.
#pragma once

#include "mlq/quant_types.h"

#include <cstddef>
#include <string>
#include <vector>

namespace mlq {

bool hip_runtime_built();
int hip_device_count();
std::string hip_device_summary(int device_id = 0);

// Owning device allocation (cf. CudaDeviceBuffer, cuda_runtime.h:34-77).
class HipDeviceBuffer {
public:
    HipDeviceBuffer() = default;
    explicit HipDeviceBuffer(size_t bytes, int device_id = 0);
    ~HipDeviceBuffer();
    HipDeviceBuffer(const HipDeviceBuffer&) = delete;
    HipDeviceBuffer& operator=(const HipDeviceBuffer&) = delete;
    HipDeviceBuffer(HipDeviceBuffer&& o) noexcept;
    HipDeviceBuffer& operator=(HipDeviceBuffer&& o) noexcept;

    void reset();
    void reset(size_t bytes, int device_id = 0);
    void upload(const void* src, size_t bytes);
    void download(void* dst, size_t bytes) const;

    void* data() { return data_; }
    const void* data() const { return data_; }
    size_t bytes() const { return bytes_; }
    int device_id() const { return device_id_; }
    bool empty() const { return data_ == nullptr; }

private:
    void* data_ = nullptr;
    size_t bytes_ = 0;
    int device_id_ = 0;
};

// Move-only f32 tensor on a device (cf. CudaTensor, cuda_tensor.h:12-63).
class HipTensor {
public:
    HipTensor() = default;
    explicit HipTensor(const std::vector<int>& shape, int device_id = 0);
    HipTensor(HipTensor&&) noexcept = default;
    HipTensor& operator=(HipTensor&&) noexcept = default;

    void upload_from(const Tensor& src);
    Tensor download() const;

    void* data() { return buffer_.data(); }
    const void* data() const { return buffer_.data(); }
    const std::vector<int>& shape() const { return shape_; }
    int ndim() const { return static_cast<int>(shape_.size()); }
    size_t size() const { return numel_; }
    int device_id() const { return device_id_; }
    std::string shape_str() const { return shape_string(shape_); }

private:
    std::vector<int> shape_;
    size_t numel_ = 0;
    int device_id_ = 0;
    HipDeviceBuffer buffer_;
};

HipTensor hip_tensor_from_host(const Tensor& src, int device_id = 0);

}  // namespace mlq

// mini-llama.cpp's device-backend interface implemented on the MI355X HIP
// library: the drop-in a HIP build of the reference compiles in place of
// src/cuda_runtime.cpp, src/cuda_quant.cpp and src/cuda_quant.cu.
//
// The interface is the reference's own (include/mini_llama/cuda_runtime.h,
// include/mini_llama/cuda_quant.h): its types (Tensor, CudaTensor,
// CudaDeviceBuffer, BlockQ*), its function names and argument meanings, its
// validation order and messages (src/cuda_quant.cu:139-243, 253-255,
// 299-301), so the reference's callers -- model.cpp's weight upload
// (src/model.cpp:145-316), forward.cpp's forward_linear /
// forward_linear_device (src/forward.cpp:172-291) and the reference's own test
// (tests/test_cuda_quant.cpp) -- run unchanged on the HIP kernels.  Every
// device operation goes through the C ABI of include/mlq_hip.h; nothing here
// includes a HIP or CUDA header.
//
// Built by oracle/Makefile (target `dropin`) together with the reference's CPU
// sources where they lie; this file is test infrastructure of that build and
// is not part of libmlq_hip.so.
#include "mini_llama/cuda_quant.h"
#include "mini_llama/cuda_runtime.h"
#include "mini_llama/cuda_tensor.h"

#include "mlq_hip.h"

#include <cstdio>
#include <sstream>
#include <stdexcept>
#include <string>
#include <utility>

namespace mini_llama {

namespace {

thread_local int g_current_device = 0;  // cudaSetDevice's per-thread current device

[[noreturn]] void throw_hip(const std::string& what) {
    throw std::runtime_error("HIP runtime error in " + what + ": " + mlq_hip_last_error());
}

void check(int rc, const char* what) {
    if (rc != MLQ_OK) throw_hip(what);
}

// The library's stream of `device`: every launch below is issued there and
// waited for before returning, as the reference's calls are synchronous.
void sync_device(int device) {
    void* s = nullptr;
    check(mlq_hip_stream(device, &s), "mlq_hip_stream");
    check(mlq_hip_synchronize(s), "mlq_hip_synchronize");
}

}  // namespace

// ---- include/mini_llama/cuda_runtime.h -------------------------------------

bool cuda_runtime_built() { return true; }

int cuda_device_count() {
    int n = 0;
    check(mlq_hip_device_count(&n), "mlq_hip_device_count");
    return n;
}

void cuda_set_device(int device_id) {
    check(mlq_hip_init(device_id), "mlq_hip_init");
    g_current_device = device_id;
}

CudaDeviceInfo cuda_get_device_info(int device_id) {
    char buf[256] = {0};
    check(mlq_hip_device_info(device_id, buf, sizeof buf), "mlq_hip_device_info");
    CudaDeviceInfo info;
    info.id = device_id;
    info.name = buf;
    return info;
}

std::string cuda_format_device_info(const CudaDeviceInfo& info) {
    // The reference's layout (src/cuda_runtime.cpp:99-108); the HIP summary
    // string carries the architecture and memory in its name.
    std::ostringstream out;
    out << "device " << info.id << ": " << info.name;
    return out.str();
}

void* cuda_malloc_bytes(size_t bytes) {
    if (bytes == 0) return nullptr;
    void* p = nullptr;
    check(mlq_hip_malloc(g_current_device, bytes, &p), "mlq_hip_malloc");
    return p;
}

void cuda_free_bytes(void* ptr) {
    if (ptr != nullptr) check(mlq_hip_free(ptr), "mlq_hip_free");
}

void cuda_memcpy_bytes(void* dst, const void* src, size_t bytes, CudaMemcpyKind kind) {
    if (bytes == 0) return;
    switch (kind) {
        case CudaMemcpyKind::HostToDevice: check(mlq_hip_memcpy_htod(dst, src, bytes), "mlq_hip_memcpy_htod"); return;
        case CudaMemcpyKind::DeviceToHost: check(mlq_hip_memcpy_dtoh(dst, src, bytes), "mlq_hip_memcpy_dtoh"); return;
        case CudaMemcpyKind::DeviceToDevice:
            check(mlq_hip_memcpy_dtod(dst, src, bytes, nullptr), "mlq_hip_memcpy_dtod");
            sync_device(g_current_device);
            return;
    }
    throw std::runtime_error("unknown CUDA memcpy kind");
}

CudaDeviceBuffer::CudaDeviceBuffer(size_t bytes, int device_id) { reset(bytes, device_id); }

CudaDeviceBuffer::~CudaDeviceBuffer() { release_noexcept(); }

CudaDeviceBuffer::CudaDeviceBuffer(CudaDeviceBuffer&& other) noexcept
    : data_(std::exchange(other.data_, nullptr)),
      bytes_(std::exchange(other.bytes_, 0)),
      device_id_(std::exchange(other.device_id_, 0)) {}

CudaDeviceBuffer& CudaDeviceBuffer::operator=(CudaDeviceBuffer&& other) noexcept {
    if (this != &other) {
        release_noexcept();
        data_ = std::exchange(other.data_, nullptr);
        bytes_ = std::exchange(other.bytes_, 0);
        device_id_ = std::exchange(other.device_id_, 0);
    }
    return *this;
}

void CudaDeviceBuffer::reset() {
    if (data_ != nullptr) check(mlq_hip_free(data_), "mlq_hip_free");
    data_ = nullptr;
    bytes_ = 0;
    device_id_ = 0;
}

void CudaDeviceBuffer::reset(size_t bytes, int device_id) {
    reset();
    if (bytes == 0) return;
    cuda_set_device(device_id);
    void* p = nullptr;
    check(mlq_hip_malloc(device_id, bytes, &p), "mlq_hip_malloc");
    data_ = p;
    bytes_ = bytes;
    device_id_ = device_id;
}

void CudaDeviceBuffer::upload(const void* src, size_t bytes) {
    if (bytes > bytes_) throw std::runtime_error("CudaDeviceBuffer::upload size exceeds buffer");
    if (bytes == 0) return;
    check(mlq_hip_memcpy_htod(data_, src, bytes), "mlq_hip_memcpy_htod");
}

void CudaDeviceBuffer::download(void* dst, size_t bytes) const {
    if (bytes > bytes_) throw std::runtime_error("CudaDeviceBuffer::download size exceeds buffer");
    if (bytes == 0) return;
    check(mlq_hip_memcpy_dtoh(dst, data_, bytes), "mlq_hip_memcpy_dtoh");
}

void CudaDeviceBuffer::release_noexcept() noexcept {
    if (data_ != nullptr) (void)mlq_hip_free(data_);
    data_ = nullptr;
    bytes_ = 0;
}

// ---- include/mini_llama/cuda_quant.h ---------------------------------------

namespace {

int in_features_of(const std::vector<int>& xs, const std::string& xstr, const char* caller) {
    if (xs.size() == 1) return xs[0];
    if (xs.size() == 2) return xs[1];
    throw std::runtime_error(std::string(caller) +
                             ": expected x shape [in_features] or [batch, in_features], got " + xstr);
}

// Order and texts of the reference's checks (src/cuda_quant.cu:150-243).
void validate(const std::vector<int>& xs, const std::string& xstr, const std::vector<int>& ws, size_t blocks,
              const char* caller) {
    if (ws.size() != 2) throw std::runtime_error(std::string(caller) + ": expected W shape [out_features, in_features]");
    const int in = in_features_of(xs, xstr, caller);
    if (in <= 0 || ws[0] <= 0 || ws[1] <= 0) {
        throw std::runtime_error(std::string(caller) + ": empty tensors are not supported");
    }
    if (ws[1] != in) {
        throw std::runtime_error(std::string(caller) + ": dimension mismatch x=" + xstr + " W=[" +
                                 std::to_string(ws[0]) + ", " + std::to_string(ws[1]) + "]");
    }
    const size_t expected = static_cast<size_t>(ws[0]) * static_cast<size_t>((in + 31) / 32);
    if (blocks != expected) {
        throw std::runtime_error(std::string(caller) + ": block count mismatch: expected " + std::to_string(expected) +
                                 ", got " + std::to_string(blocks));
    }
}

void add_bias(Tensor& y, const Tensor& bias, int rows, int cols, const char* caller) {
    if (bias.ndim() != 1 || bias.shape[0] != cols) {
        throw std::runtime_error(std::string(caller) + ": expected bias shape [out_features]");
    }
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) y.data[static_cast<size_t>(r) * cols + c] += bias.data[c];
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
    sync_device(device_id);
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

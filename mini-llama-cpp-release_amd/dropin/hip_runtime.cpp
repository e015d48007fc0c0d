// The reference's device runtime interface (include/mini_llama/cuda_runtime.h:
// device count and properties, current device, CudaDeviceBuffer, copies) on
// the MI355X HIP library: a HIP build of the reference compiles this file in
// place of src/cuda_runtime.cpp.  Its types, function names, argument meanings
// and behaviour are the reference's; every device operation is a C ABI call
// (include/mlq_hip.h), so src/cuda_tensor.cpp, src/cuda_kv_cache.cpp,
// src/model.cpp and src/forward.cpp compile unchanged on top of it.
#include "mini_llama/cuda_runtime.h"

#include "hip_common.h"

#include <sstream>
#include <stdexcept>
#include <string>
#include <utility>

namespace mini_llama {

namespace hipdrop {

int& current_device() {
    thread_local int device = 0;
    return device;
}

}  // namespace hipdrop

using hipdrop::check;
using hipdrop::sync_device;

// ---- include/mini_llama/cuda_runtime.h -------------------------------------

bool cuda_runtime_built() { return true; }

int cuda_device_count() {
    int n = 0;
    check(mlq_hip_device_count(&n), "mlq_hip_device_count");
    return n;
}

void cuda_set_device(int device_id) {
    check(mlq_hip_init(device_id), "mlq_hip_init");
    hipdrop::current_device() = device_id;
}

CudaDeviceInfo cuda_get_device_info(int device_id) {
    mlq_device_props p;
    check(mlq_hip_device_props(device_id, &p), "mlq_hip_device_props");
    CudaDeviceInfo info;
    info.id = device_id;
    info.name = std::string(p.name) + " (" + p.arch + ", " + std::to_string(p.compute_units) + " CUs)";
    info.compute_major = p.major;  // gfx950: 9.5
    info.compute_minor = p.minor;
    info.total_memory_bytes = p.total_memory_bytes;
    info.driver_version = p.driver_version;
    info.runtime_version = p.runtime_version;
    return info;
}

std::string cuda_format_device_info(const CudaDeviceInfo& info) {
    // The reference's fields and order (src/cuda_runtime.cpp:99-108), HIP's
    // runtime named as such.
    const double total_gb = static_cast<double>(info.total_memory_bytes) / (1024.0 * 1024.0 * 1024.0);
    std::ostringstream out;
    out << "device " << info.id << ": " << info.name << ", compute capability " << info.compute_major << "."
        << info.compute_minor << ", total memory " << total_gb << " GB, hip runtime " << info.runtime_version
        << ", driver " << info.driver_version;
    return out.str();
}

void* cuda_malloc_bytes(size_t bytes) {
    if (bytes == 0) return nullptr;
    void* p = nullptr;
    check(mlq_hip_malloc(hipdrop::current_device(), bytes, &p), "mlq_hip_malloc");
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
            sync_device(hipdrop::current_device());
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

}  // namespace mini_llama

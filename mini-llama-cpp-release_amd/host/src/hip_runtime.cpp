// HIP runtime wrappers over the C ABI (see mlq/hip_runtime.h).
#include "mlq/hip_runtime.h"

#include "mlq_hip.h"

#include <stdexcept>
#include <utility>

namespace mlq {

namespace {

void check(int rc, const char* what) {
    if (rc != MLQ_OK) {
        throw std::runtime_error(std::string(what) + ": " + mlq_hip_last_error());
    }
}

}  // namespace

bool hip_runtime_built() { return mlq_hip_built() != 0; }

int hip_device_count() {
    int n = 0;
    check(mlq_hip_device_count(&n), "hip_device_count");
    return n;
}

std::string hip_device_summary(int device_id) {
    char buf[256] = {0};
    if (mlq_hip_device_info(device_id, buf, sizeof buf) != MLQ_OK) return mlq_hip_last_error();
    return buf;
}

HipDeviceBuffer::HipDeviceBuffer(size_t bytes, int device_id) { reset(bytes, device_id); }

HipDeviceBuffer::~HipDeviceBuffer() { reset(); }

HipDeviceBuffer::HipDeviceBuffer(HipDeviceBuffer&& o) noexcept
    : data_(std::exchange(o.data_, nullptr)), bytes_(std::exchange(o.bytes_, 0)), device_id_(o.device_id_) {}

HipDeviceBuffer& HipDeviceBuffer::operator=(HipDeviceBuffer&& o) noexcept {
    if (this != &o) {
        reset();
        data_ = std::exchange(o.data_, nullptr);
        bytes_ = std::exchange(o.bytes_, 0);
        device_id_ = o.device_id_;
    }
    return *this;
}

void HipDeviceBuffer::reset() {
    if (data_ != nullptr) {
        (void)mlq_hip_init(device_id_);
        (void)mlq_hip_free(data_);
    }
    data_ = nullptr;
    bytes_ = 0;
}

void HipDeviceBuffer::reset(size_t bytes, int device_id) {
    reset();
    void* p = nullptr;
    check(mlq_hip_malloc(device_id, bytes, &p), "HipDeviceBuffer");
    data_ = p;
    bytes_ = bytes;
    device_id_ = device_id;
}

void HipDeviceBuffer::upload(const void* src, size_t bytes) {
    if (bytes > bytes_) throw std::runtime_error("HipDeviceBuffer::upload: size exceeds buffer");
    check(mlq_hip_init(device_id_), "HipDeviceBuffer::upload");
    check(mlq_hip_memcpy_htod(data_, src, bytes), "HipDeviceBuffer::upload");
}

void HipDeviceBuffer::download(void* dst, size_t bytes) const {
    if (bytes > bytes_) throw std::runtime_error("HipDeviceBuffer::download: size exceeds buffer");
    check(mlq_hip_init(device_id_), "HipDeviceBuffer::download");
    check(mlq_hip_memcpy_dtoh(dst, data_, bytes), "HipDeviceBuffer::download");
}

HipTensor::HipTensor(const std::vector<int>& shape, int device_id) : shape_(shape), device_id_(device_id) {
    Tensor probe(shape);  // same dimension checks as the host tensor
    numel_ = probe.size();
    buffer_.reset(numel_ * sizeof(float), device_id);
}

void HipTensor::upload_from(const Tensor& src) {
    if (src.shape != shape_) throw std::runtime_error("HipTensor::upload_from: shape mismatch");
    buffer_.upload(src.data.data(), src.size() * sizeof(float));
}

Tensor HipTensor::download() const {
    Tensor t(shape_);
    buffer_.download(t.data.data(), t.size() * sizeof(float));
    return t;
}

HipTensor hip_tensor_from_host(const Tensor& src, int device_id) {
    HipTensor t(src.shape, device_id);
    t.upload_from(src);
    return t;
}

}  // namespace mlq

// The reference's op-by-op device interfaces of the forward pass on the MI355X
// HIP library: include/mini_llama/cuda_ops.h (RMSNorm, SiLU, elementwise
// product / sum, softmax, embedding lookup, RoPE), cuda_attention.h
// (single-token attention over the device KV cache) and cuda_matmul.h (F32
// matmul / linear).  A HIP build of the reference compiles this file in place
// of src/cuda_ops.cpp + src/cuda_ops.cu, src/cuda_attention.cpp +
// src/cuda_attention.cu and src/cuda_matmul.cpp (cuBLAS); src/cuda_kv_cache.cpp
// compiles unchanged over the runtime of hip_runtime.cpp.
//
// Argument checks and their messages are the reference's
// (src/cuda_ops.cu:171-318, 320-707; src/cuda_attention.cu:40-110;
// src/cuda_matmul.cpp:76-131, 134-236).  The kernels are the library's
// (csrc/ops.hip) through the C ABI.  Calls on device tensors are queued on the
// library stream of their device and return at once (every drop-in call and
// every copy uses that stream, so they run in call order; copies to the host
// wait for it); calls on host tensors return their result.
#include "mini_llama/cuda_attention.h"
#include "mini_llama/cuda_kv_cache.h"
#include "mini_llama/cuda_matmul.h"
#include "mini_llama/cuda_ops.h"
#include "mini_llama/cuda_runtime.h"
#include "mini_llama/cuda_tensor.h"

#include "hip_common.h"
#include "mlq/linear_checks.h"

#include <cmath>
#include <stdexcept>
#include <string>
#include <vector>

namespace mini_llama {

namespace {

using hipdrop::check;
using hipdrop::stream_of;
using hipdrop::throw_op;

const float* cf(const void* p) { return static_cast<const float*>(p); }
float* mf(void* p) { return static_cast<float*>(p); }

void require_same_shape(const Tensor& a, const Tensor& b, const char* caller) {
    if (a.shape != b.shape) {
        throw std::runtime_error(std::string(caller) + ": shape mismatch " + a.shape_str() + " vs " + b.shape_str());
    }
}

void require_same_shape(const CudaTensor& a, const CudaTensor& b, const char* caller) {
    if (a.shape() != b.shape()) {
        throw std::runtime_error(std::string(caller) + ": shape mismatch " + a.shape_str() + " vs " + b.shape_str());
    }
    if (a.device_id() != b.device_id()) {
        throw std::runtime_error(std::string(caller) + ": tensors are on different CUDA devices");
    }
}

void require_1d(int ndim, size_t size, const std::string& shape, const char* caller) {
    if (ndim != 1) throw std::runtime_error(std::string(caller) + ": expected 1D tensor, got " + shape);
    if (size == 0) throw std::runtime_error(std::string(caller) + ": empty tensor");
}

void require_1d(const Tensor& x, const char* caller) { require_1d(x.ndim(), x.size(), x.shape_str(), caller); }
void require_1d(const CudaTensor& x, const char* caller) { require_1d(x.ndim(), x.size(), x.shape_str(), caller); }

void require_eps(float eps, const char* caller) {
    if (!std::isfinite(eps) || eps <= 0.0f) {
        throw std::runtime_error(std::string(caller) + ": eps must be finite and positive");
    }
}

void require_device(const CudaTensor& x, int device_id, const char* caller) {
    if (x.device_id() != device_id) {
        throw std::runtime_error(std::string(caller) + ": input tensor is on a different CUDA device");
    }
}

// A host tensor's copy on `device` (the reference uploads its inputs per call).
CudaTensor to_device(const Tensor& t, int device) {
    CudaTensor d(t.shape, device);
    d.upload_from(t);
    return d;
}

// Elementwise op of the library (SiLU when b is null) into a new device tensor.
CudaTensor elementwise(int op, const CudaTensor& a, const CudaTensor* b, int device_id, const char* caller) {
    cuda_set_device(device_id);
    CudaTensor y(a.shape(), device_id);
    const float* bp = b != nullptr ? cf(b->data()) : nullptr;
    int rc = MLQ_OK;
    void* s = stream_of(device_id);
    switch (op) {
        case 0: rc = mlq_hip_silu(device_id, cf(a.data()), a.size(), mf(y.data()), s); break;
        case 1: rc = mlq_hip_mul(device_id, cf(a.data()), bp, a.size(), mf(y.data()), s); break;
        default: rc = mlq_hip_add(device_id, cf(a.data()), bp, a.size(), mf(y.data()), s); break;
    }
    if (rc != MLQ_OK) throw_op(caller);
    return y;
}

void rope_device(float* q, int n_heads, float* k, int n_kv_heads, int head_dim, int pos, float theta,
                 RopeType rope_type, int device_id, const char* caller) {
    const int neox = rope_type == RopeType::NeoX ? 1 : 0;
    void* s = stream_of(device_id);
    if (mlq_hip_rope(device_id, q, n_heads, head_dim, pos, theta, neox, s) != MLQ_OK) throw_op(caller);
    if (mlq_hip_rope(device_id, k, n_kv_heads, head_dim, pos, theta, neox, s) != MLQ_OK) throw_op(caller);
}

}  // namespace

// ---- include/mini_llama/cuda_ops.h -------------------------------------------

bool cuda_ops_built() { return true; }

CudaTensor cuda_rmsnorm_device_weight(const CudaTensor& x, const void* weight_data, const std::vector<int>& weight_shape,
                                      float eps, int device_id) {
    const char* caller = "cuda_rmsnorm_device_weight";
    require_1d(x, caller);
    if (weight_data == nullptr) throw std::runtime_error(std::string(caller) + ": weight data is null");
    if (x.shape() != weight_shape) throw std::runtime_error(std::string(caller) + ": x and weight shape mismatch");
    require_device(x, device_id, caller);
    require_eps(eps, caller);
    cuda_set_device(device_id);
    CudaTensor y(x.shape(), device_id);
    if (mlq_hip_rmsnorm(device_id, cf(x.data()), cf(weight_data), static_cast<int>(x.size()), eps, mf(y.data()),
                        stream_of(device_id)) != MLQ_OK) {
        throw_op(caller);
    }
    return y;
}

CudaTensor cuda_rmsnorm_device_input(const CudaTensor& x, const Tensor& weight, float eps, int device_id) {
    const char* caller = "cuda_rmsnorm_device_input";
    require_1d(x, caller);
    require_1d(weight, caller);
    if (x.shape() != weight.shape) throw std::runtime_error(std::string(caller) + ": x and weight shape mismatch");
    require_device(x, device_id, caller);
    require_eps(eps, caller);
    cuda_set_device(device_id);
    CudaTensor w = to_device(weight, device_id);
    return cuda_rmsnorm_device_weight(x, w.data(), weight.shape, eps, device_id);
}

Tensor cuda_rmsnorm(const Tensor& x, const Tensor& weight, float eps, int device_id) {
    const char* caller = "cuda_rmsnorm";
    require_1d(x, caller);
    require_1d(weight, caller);
    if (x.shape != weight.shape) throw std::runtime_error(std::string(caller) + ": x and weight shape mismatch");
    require_eps(eps, caller);
    cuda_set_device(device_id);
    CudaTensor xd = to_device(x, device_id);
    CudaTensor wd = to_device(weight, device_id);
    CudaTensor y(x.shape, device_id);
    if (mlq_hip_rmsnorm(device_id, cf(xd.data()), cf(wd.data()), static_cast<int>(x.size()), eps, mf(y.data()),
                        stream_of(device_id)) != MLQ_OK) {
        throw_op(caller);
    }
    return y.download();
}

CudaTensor cuda_silu_device_input(const CudaTensor& x, int device_id) {
    const char* caller = "cuda_silu_device_input";
    require_device(x, device_id, caller);
    return elementwise(0, x, nullptr, device_id, caller);
}

Tensor cuda_silu(const Tensor& x, int device_id) {
    cuda_set_device(device_id);
    if (x.size() == 0) return Tensor(x.shape, 0.0f);
    CudaTensor xd = to_device(x, device_id);
    return elementwise(0, xd, nullptr, device_id, "cuda_silu").download();
}

CudaTensor cuda_elementwise_mul_device_input(const CudaTensor& a, const CudaTensor& b, int device_id) {
    const char* caller = "cuda_elementwise_mul_device_input";
    require_same_shape(a, b, caller);
    require_device(a, device_id, caller);
    return elementwise(1, a, &b, device_id, caller);
}

Tensor cuda_elementwise_mul(const Tensor& a, const Tensor& b, int device_id) {
    require_same_shape(a, b, "cuda_elementwise_mul");
    cuda_set_device(device_id);
    if (a.size() == 0) return Tensor(a.shape, 0.0f);
    CudaTensor ad = to_device(a, device_id);
    CudaTensor bd = to_device(b, device_id);
    return elementwise(1, ad, &bd, device_id, "cuda_elementwise_mul").download();
}

CudaTensor cuda_elementwise_add_device_input(const CudaTensor& a, const CudaTensor& b, int device_id) {
    const char* caller = "cuda_elementwise_add_device_input";
    require_same_shape(a, b, caller);
    require_device(a, device_id, caller);
    return elementwise(2, a, &b, device_id, caller);
}

CudaTensor cuda_elementwise_add_device_weight(const CudaTensor& a, const void* b_data, const std::vector<int>& b_shape,
                                              int device_id) {
    const char* caller = "cuda_elementwise_add_device_weight";
    require_device(a, device_id, caller);
    if (b_data == nullptr) throw std::runtime_error(std::string(caller) + ": weight data is null");
    if (a.shape() != b_shape) throw std::runtime_error(std::string(caller) + ": input and weight shape mismatch");
    cuda_set_device(device_id);
    CudaTensor y(a.shape(), device_id);
    if (mlq_hip_add(device_id, cf(a.data()), cf(b_data), a.size(), mf(y.data()), stream_of(device_id)) != MLQ_OK) {
        throw_op(caller);
    }
    return y;
}

Tensor cuda_elementwise_add(const Tensor& a, const Tensor& b, int device_id) {
    require_same_shape(a, b, "cuda_elementwise_add");
    cuda_set_device(device_id);
    if (a.size() == 0) return Tensor(a.shape, 0.0f);
    CudaTensor ad = to_device(a, device_id);
    CudaTensor bd = to_device(b, device_id);
    return elementwise(2, ad, &bd, device_id, "cuda_elementwise_add").download();
}

Tensor cuda_softmax(const Tensor& x, int device_id) {
    const char* caller = "cuda_softmax";
    require_1d(x, caller);
    cuda_set_device(device_id);
    CudaTensor xd = to_device(x, device_id);
    CudaTensor y(x.shape, device_id);
    if (mlq_hip_softmax(device_id, cf(xd.data()), static_cast<int>(x.size()), mf(y.data()), stream_of(device_id)) !=
        MLQ_OK) {
        throw_op(caller);
    }
    return y.download();
}

CudaTensor cuda_embedding_lookup_device_weight(const void* embedding_data, const std::vector<int>& embedding_shape,
                                               int token_id, int device_id) {
    const char* caller = "cuda_embedding_lookup_device_weight";
    if (embedding_data == nullptr) throw std::runtime_error(std::string(caller) + ": embedding data is null");
    if (embedding_shape.size() != 2) throw std::runtime_error(std::string(caller) + ": expected 2D embedding weight");
    const int vocab = embedding_shape[0];
    const int dim = embedding_shape[1];
    if (vocab <= 0 || dim <= 0) throw std::runtime_error(std::string(caller) + ": embedding shape must be positive");
    if (token_id < 0 || token_id >= vocab) throw std::out_of_range(std::string(caller) + ": token id out of range");
    cuda_set_device(device_id);
    CudaTensor y({dim}, device_id);
    if (mlq_hip_embedding(device_id, cf(embedding_data), vocab, dim, token_id, mf(y.data()), stream_of(device_id)) !=
        MLQ_OK) {
        throw_op(caller);
    }
    return y;
}

void cuda_rope_device_input(CudaTensor& q, CudaTensor& k, int n_heads, int n_kv_heads, int head_dim, int pos,
                            float theta, RopeType rope_type, int device_id) {
    const char* caller = "cuda_rope_device_input";
    if (q.device_id() != device_id || k.device_id() != device_id) {
        throw std::runtime_error(std::string(caller) + ": input tensor is on a different CUDA device");
    }
    if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim % 2 != 0) {
        throw std::runtime_error(std::string(caller) + ": invalid head shape");
    }
    if (q.size() != static_cast<size_t>(n_heads) * static_cast<size_t>(head_dim)) {
        throw std::runtime_error(std::string(caller) + ": q shape mismatch");
    }
    if (k.size() != static_cast<size_t>(n_kv_heads) * static_cast<size_t>(head_dim)) {
        throw std::runtime_error(std::string(caller) + ": k shape mismatch");
    }
    if (pos < 0) throw std::out_of_range(std::string(caller) + ": position must be non-negative");
    if (!std::isfinite(theta) || theta <= 0.0f) {
        throw std::runtime_error(std::string(caller) + ": theta must be finite and positive");
    }
    cuda_set_device(device_id);
    rope_device(mf(q.data()), n_heads, mf(k.data()), n_kv_heads, head_dim, pos, theta, rope_type, device_id, caller);
}

void cuda_rope(Tensor& q, Tensor& k, int pos, float theta, RopeType rope_type, int device_id) {
    const char* caller = "cuda_rope";
    if (q.ndim() != 2 || k.ndim() != 2) throw std::runtime_error("cuda_rope: expected 2D tensors");
    if (pos < 0) throw std::out_of_range("cuda_rope: position must be non-negative");
    if (!std::isfinite(theta) || theta <= 0.0f) throw std::runtime_error("cuda_rope: theta must be finite and positive");
    if (q.shape[1] != k.shape[1]) {
        throw std::runtime_error("cuda_rope: q and k head_dim mismatch " + q.shape_str() + " vs " + k.shape_str());
    }
    if (q.shape[1] <= 0 || q.shape[1] % 2 != 0) throw std::runtime_error("cuda_rope: head_dim must be positive and even");
    cuda_set_device(device_id);
    CudaTensor qd = to_device(q, device_id);
    CudaTensor kd = to_device(k, device_id);
    rope_device(mf(qd.data()), q.shape[0], mf(kd.data()), k.shape[0], q.shape[1], pos, theta, rope_type, device_id,
                caller);
    qd.download_to(q);
    kd.download_to(k);
}

// ---- include/mini_llama/cuda_attention.h -------------------------------------

bool cuda_attention_built() { return true; }

namespace {

void validate_attention(const CudaKVCache& kv, int layer, int pos, int n_heads, int n_kv_heads, int head_dim,
                        const char* caller, const char* shape_msg) {
    if (kv.empty()) throw std::runtime_error(std::string(caller) + ": CUDA KV cache is empty");
    if (layer < 0 || layer >= kv.n_layers()) throw std::out_of_range(std::string(caller) + ": layer out of range");
    if (pos < 0 || pos >= kv.max_seq_len()) throw std::out_of_range(std::string(caller) + ": position out of range");
    if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0) {
        throw std::runtime_error(std::string(caller) + ": head counts and head_dim must be positive");
    }
    if (n_heads % n_kv_heads != 0) {
        throw std::runtime_error(std::string(caller) + ": n_heads must be divisible by n_kv_heads");
    }
    if (kv.n_kv_heads() != n_kv_heads || kv.head_dim() != head_dim) {
        throw std::runtime_error(std::string(caller) + ": " + shape_msg);
    }
}

void attention(const float* q, const CudaKVCache& kv, int layer, int pos, int n_heads, int n_kv_heads, int head_dim,
               float* out, int device_id, const char* caller) {
    if (mlq_hip_attention_decode(device_id, q, cf(kv.keys_data()), cf(kv.values_data()), kv.n_layers(), layer,
                                 kv.max_seq_len(), n_heads, n_kv_heads, head_dim, pos, out,
                                 stream_of(device_id)) != MLQ_OK) {
        throw_op(caller);
    }
}

}  // namespace

Tensor cuda_attention_decode(const Tensor& q, const CudaKVCache& kv_cache, int layer, int pos, int n_heads,
                             int n_kv_heads, int head_dim, int device_id) {
    const char* caller = "cuda_attention_decode";
    if (q.shape != std::vector<int>{n_heads, head_dim}) {
        throw std::runtime_error(std::string(caller) + ": expected q shape [" + std::to_string(n_heads) + ", " +
                                 std::to_string(head_dim) + "], got " + q.shape_str());
    }
    validate_attention(kv_cache, layer, pos, n_heads, n_kv_heads, head_dim, caller,
                       "KV cache shape does not match attention shape");
    cuda_set_device(device_id);
    CudaTensor qd = to_device(q, device_id);
    CudaTensor out({n_heads, head_dim}, device_id);
    attention(cf(qd.data()), kv_cache, layer, pos, n_heads, n_kv_heads, head_dim, mf(out.data()), device_id, caller);
    return out.download();
}

CudaTensor cuda_attention_decode_device_input(const CudaTensor& q, const CudaKVCache& kv_cache, int layer, int pos,
                                              int n_heads, int n_kv_heads, int head_dim, int device_id) {
    const char* caller = "cuda_attention_decode_device_input";
    if (q.device_id() != device_id) throw std::runtime_error(std::string(caller) + ": q tensor is on a different CUDA device");
    if (q.size() != static_cast<size_t>(n_heads) * static_cast<size_t>(head_dim)) {
        throw std::runtime_error(std::string(caller) + ": q shape mismatch");
    }
    validate_attention(kv_cache, layer, pos, n_heads, n_kv_heads, head_dim, caller,
                       "KV cache shape or device does not match attention shape");
    if (kv_cache.device_id() != device_id) {
        throw std::runtime_error(std::string(caller) + ": KV cache shape or device does not match attention shape");
    }
    cuda_set_device(device_id);
    CudaTensor out({n_heads * head_dim}, device_id);
    attention(cf(q.data()), kv_cache, layer, pos, n_heads, n_kv_heads, head_dim, mf(out.data()), device_id, caller);
    return out;
}

// ---- include/mini_llama/cuda_matmul.h ----------------------------------------

bool cuda_matmul_built() { return true; }

Tensor cuda_matmul(const Tensor& A, const Tensor& B, int device_id) {
    if (A.ndim() != 2 || B.ndim() != 2) throw std::runtime_error("cuda_matmul: expected A and B to be 2D tensors");
    if (A.shape[1] != B.shape[0]) {
        throw std::runtime_error("cuda_matmul: dimension mismatch " + A.shape_str() + " vs " + B.shape_str());
    }
    const int M = A.shape[0], K = A.shape[1], N = B.shape[1];
    cuda_set_device(device_id);
    CudaTensor ad = to_device(A, device_id);
    CudaTensor bd = to_device(B, device_id);
    CudaTensor c({M, N}, device_id);
    if (mlq_hip_matmul_f32(device_id, cf(ad.data()), cf(bd.data()), M, K, N, 0, mf(c.data()), stream_of(device_id)) !=
        MLQ_OK) {
        throw_op("cuda_matmul");
    }
    return c.download();
}

namespace {

int linear_in(const std::vector<int>& xs, const std::string& xstr, const std::vector<int>& ws, const char* caller) {
    if (ws.size() != 2) throw std::runtime_error(std::string(caller) + ": expected W shape [out_features, in_features]");
    const int in = mlq::checks::in_features_of(xs, xstr, caller);
    if (ws[1] != in) {
        throw std::runtime_error(std::string(caller) + ": dimension mismatch x=" + xstr + " W=[" +
                                 std::to_string(ws[0]) + ", " + std::to_string(ws[1]) + "]");
    }
    return in;
}

// y[rows][out] = x[rows][in] W^T with W [out][in] on the device.
void linear_f32(const float* x, const void* w, int rows, int in, int out, float* y, int device_id, const char* caller) {
    if (mlq_hip_matmul_f32(device_id, x, cf(w), rows, in, out, 1, y, stream_of(device_id)) != MLQ_OK) throw_op(caller);
}

}  // namespace

Tensor cuda_linear_device_weight(const Tensor& x, const void* w_device, const std::vector<int>& w_shape,
                                 const Tensor* bias, int device_id) {
    const char* caller = "cuda_linear";
    if (w_device == nullptr) throw std::runtime_error("cuda_linear: device weight pointer is null");
    const int in = linear_in(x.shape, x.shape_str(), w_shape, caller);
    const bool is_1d = x.ndim() == 1;
    const int rows = is_1d ? 1 : x.shape[0];
    const int out = w_shape[0];
    cuda_set_device(device_id);
    CudaTensor xd = to_device(x, device_id);
    CudaTensor yd(is_1d ? std::vector<int>{out} : std::vector<int>{rows, out}, device_id);
    linear_f32(cf(xd.data()), w_device, rows, in, out, mf(yd.data()), device_id, caller);
    Tensor y = yd.download();
    if (bias != nullptr) mlq::checks::add_bias(y.data.data(), bias->shape, bias->data.data(), rows, out, caller);
    return y;
}

Tensor cuda_linear(const Tensor& x, const Tensor& W, const Tensor* bias, int device_id) {
    if (W.ndim() != 2) throw std::runtime_error("cuda_linear: expected W shape [out_features, in_features]");
    cuda_set_device(device_id);
    CudaTensor wd = to_device(W, device_id);
    return cuda_linear_device_weight(x, wd.data(), W.shape, bias, device_id);
}

CudaTensor cuda_linear_device_input(const CudaTensor& x, const void* w_device, const std::vector<int>& w_shape,
                                    int device_id) {
    const char* caller = "cuda_linear_device_input";
    if (w_device == nullptr) throw std::runtime_error("cuda_linear_device_input: device weight pointer is null");
    if (x.device_id() != device_id) {
        throw std::runtime_error("cuda_linear_device_input: input tensor is on a different CUDA device");
    }
    const int in = linear_in(x.shape(), x.shape_str(), w_shape, caller);
    const bool is_1d = x.ndim() == 1;
    const int rows = is_1d ? 1 : x.shape()[0];
    const int out = w_shape[0];
    cuda_set_device(device_id);
    CudaTensor y(is_1d ? std::vector<int>{out} : std::vector<int>{rows, out}, device_id);
    linear_f32(cf(x.data()), w_device, rows, in, out, mf(y.data()), device_id, caller);
    return y;
}

}  // namespace mini_llama

// Device forward ops behind the reference's op-by-op device interfaces
// (include/mini_llama/cuda_ops.h, cuda_attention.h, cuda_matmul.h): RMSNorm,
// SiLU, elementwise product and sum, softmax, embedding row lookup, RoPE
// (normal and NeoX pairing), single-token attention over a KV cache and an
// F32 matrix product.  Each op reads and writes device buffers the caller
// owns and is launched on the caller's stream; nothing here allocates.
//
// These are the small kernels of a decode step that the quantized linears
// surround.  They move kilobytes per call and are launch-bound, so each is one
// grid-stride or one-workgroup kernel: a single launch per op (the reference
// uses two or three: a separate sum / max pass and a normalisation pass).
// Arithmetic follows the reference's CPU ops (src/ops.cpp:19-79, 109-176) in
// f32, with the sums taken as wavefront trees instead of a serial loop.

#include "mlq_kernels.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

namespace mlq {
namespace {

constexpr int kOpThreads = 256;
constexpr int kReduceThreads = 1024;
constexpr int kAttnWaves = 4;
constexpr int kMatTile = 16;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Sum (MAX = false) or maximum over the workgroup; the result in every thread.
template <bool MAX>
__device__ __forceinline__ float block_reduce(float v) {
    __shared__ float part[kReduceThreads / 64];
    v = MAX ? wave_max(v) : wave_sum(v);
    __syncthreads();  // `part` may still be read by an earlier call
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = part[0];
    const int waves = static_cast<int>(blockDim.x >> 6);
    for (int i = 1; i < waves; ++i) t = MAX ? fmaxf(t, part[i]) : t + part[i];
    return t;
}

// y = x * (1 / sqrt(mean(x^2) + eps)) * w  (src/ops.cpp:19-41), one workgroup.
__global__ __launch_bounds__(kReduceThreads) void op_rmsnorm_kernel(const float* __restrict__ x,
                                                                   const float* __restrict__ w, int n, float eps,
                                                                   float* __restrict__ y) {
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += x[i] * x[i];
    ss = block_reduce<false>(ss);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) y[i] = x[i] * scale * w[i];
}

// Elementwise ops over n elements (grid-stride).
enum class Ew { Silu, Mul, Add };

template <Ew OP>
__global__ __launch_bounds__(kOpThreads) void op_elementwise_kernel(const float* __restrict__ a,
                                                                   const float* __restrict__ b, size_t n,
                                                                   float* __restrict__ y) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float v = a[i];
        if (OP == Ew::Silu) y[i] = v / (1.0f + expf(-v));  // src/ops.cpp:72-79
        if (OP == Ew::Mul) y[i] = v * b[i];
        if (OP == Ew::Add) y[i] = v + b[i];
    }
}

// Softmax of one vector (src/ops.cpp:43-70), one workgroup: maximum, then
// exp(x - max) and its sum, then the division.
__global__ __launch_bounds__(kReduceThreads) void op_softmax_kernel(const float* __restrict__ x, int n,
                                                                   float* __restrict__ y) {
    float m = -INFINITY;
    for (int i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, x[i]);
    m = block_reduce<true>(m);
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float e = expf(x[i] - m);
        y[i] = e;
        s += e;
    }
    s = block_reduce<false>(s);
    for (int i = threadIdx.x; i < n; i += blockDim.x) y[i] = y[i] / s;
}

__global__ __launch_bounds__(kOpThreads) void op_embedding_kernel(const float* __restrict__ table, int dim,
                                                                 int token, float* __restrict__ y) {
    const float* row = table + static_cast<size_t>(token) * dim;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < dim; i += gridDim.x * blockDim.x) y[i] = row[i];
}

// RoPE of x [n_heads][head_dim] at position pos, one thread per rotated pair
// (src/ops.cpp:109-141): normal pairs (2i, 2i + 1), NeoX pairs (i, i + hd/2);
// the frequency of pair i is theta^(-2i / hd) in both.
__global__ __launch_bounds__(kOpThreads) void op_rope_kernel(float* __restrict__ x, int n_heads, int hd, int pos,
                                                            float theta, int neox) {
    const int half = hd / 2;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_heads * half) return;
    const int h = idx / half;
    const int i = idx % half;
    const float freq = 1.0f / powf(theta, static_cast<float>(2 * i) / static_cast<float>(hd));
    const float ang = static_cast<float>(pos) * freq;
    const float c = cosf(ang);
    const float s = sinf(ang);
    float* base = x + static_cast<size_t>(h) * hd;
    const int i0 = neox ? i : 2 * i;
    const int i1 = neox ? i + half : 2 * i + 1;
    const float x0 = base[i0];
    const float x1 = base[i1];
    base[i0] = x0 * c - x1 * s;
    base[i1] = x0 * s + x1 * c;
}

// Single-token attention of query head blockIdx.x over cache positions
// 0..pos of one layer (the math of src/forward.cpp:530-600: scores q.k *
// scale, softmax over the positions, probability-weighted sum of v).  The
// cache is [layer][max_seq][n_kv_heads][hd] f32, as CudaKVCache lays it out
// (src/cuda_kv_cache.cpp).  Four waves take every fourth position each and
// keep a running maximum, normaliser and weighted v sum (online softmax, so
// no score buffer is needed for any context length); the waves' states are
// merged through LDS.  Lane l holds elements l, l + 64, ... of the head.
template <int PER>
__global__ __launch_bounds__(64 * kAttnWaves) void op_attention_decode_kernel(
    const float* __restrict__ q, const float* __restrict__ keys, const float* __restrict__ values, int layer,
    int max_seq, int n_heads, int n_kv_heads, int hd, int pos, float scale, float* __restrict__ out) {
    __shared__ float st_m[kAttnWaves], st_l[kAttnWaves];
    __shared__ float st_acc[kAttnWaves][64 * PER];
    const int h = blockIdx.x;
    const int kvh = h / (n_heads / n_kv_heads);
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const size_t row = static_cast<size_t>(n_kv_heads) * hd;
    const size_t base = static_cast<size_t>(layer) * max_seq * row + static_cast<size_t>(kvh) * hd;
    float qv[PER], acc[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = lane + 64 * j;
        qv[j] = e < hd ? q[static_cast<size_t>(h) * hd + e] : 0.0f;
        acc[j] = 0.0f;
    }
    float m = -INFINITY, l = 0.0f;
    for (int t = wave; t <= pos; t += kAttnWaves) {
        const float* kt = keys + base + static_cast<size_t>(t) * row;
        const float* vt = values + base + static_cast<size_t>(t) * row;
        float d = 0.0f;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int e = lane + 64 * j;
            if (e < hd) d += qv[j] * kt[e];
        }
        const float s = wave_sum(d) * scale;
        const float mn = fmaxf(m, s);
        const float c = expf(m - mn);  // 0 on the wave's first position (m = -inf)
        const float p = expf(s - mn);
        l = l * c + p;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int e = lane + 64 * j;
            acc[j] = acc[j] * c + (e < hd ? p * vt[e] : 0.0f);
        }
        m = mn;
    }
    if (lane == 0) {
        st_m[wave] = m;
        st_l[wave] = l;
    }
#pragma unroll
    for (int j = 0; j < PER; ++j) st_acc[wave][lane + 64 * j] = acc[j];
    __syncthreads();
    // Merge: position 0 exists, so wave 0's maximum is finite and so is M.
    float M = st_m[0];
    for (int w = 1; w < kAttnWaves; ++w) M = fmaxf(M, st_m[w]);
    float L = 0.0f, f[kAttnWaves];
    for (int w = 0; w < kAttnWaves; ++w) {
        f[w] = st_l[w] > 0.0f ? expf(st_m[w] - M) : 0.0f;
        L += st_l[w] * f[w];
    }
    for (int e = threadIdx.x; e < hd; e += blockDim.x) {
        float v = 0.0f;
        for (int w = 0; w < kAttnWaves; ++w) v += st_acc[w][e] * f[w];
        out[static_cast<size_t>(h) * hd + e] = v / L;
    }
}

// C[M][N] = A[M][K] * op(B) in f32, op(B)[k][n] = B[k * N + n], or
// B[n * K + k] when B is stored transposed (a linear's W [N][K]).  16 x 16
// output tiles with the operands staged through LDS, K in steps of 16.
__global__ __launch_bounds__(kMatTile * kMatTile) void op_matmul_f32_kernel(const float* __restrict__ A,
                                                                           const float* __restrict__ B, int M,
                                                                           int K, int N, int bt,
                                                                           float* __restrict__ C) {
    __shared__ float ta[kMatTile][kMatTile + 1];
    __shared__ float tb[kMatTile][kMatTile + 1];
    const int tx = threadIdx.x % kMatTile;
    const int ty = threadIdx.x / kMatTile;
    const int m = blockIdx.y * kMatTile + ty;
    const int n = blockIdx.x * kMatTile + tx;
    float acc = 0.0f;
    for (int k0 = 0; k0 < K; k0 += kMatTile) {
        const int ka = k0 + tx;
        ta[ty][tx] = (m < M && ka < K) ? A[static_cast<size_t>(m) * K + ka] : 0.0f;
        const int kb = k0 + ty;
        const int nb = blockIdx.x * kMatTile + tx;
        float bv = 0.0f;
        if (kb < K && nb < N) bv = bt ? B[static_cast<size_t>(nb) * K + kb] : B[static_cast<size_t>(kb) * N + nb];
        tb[ty][tx] = bv;
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kMatTile; ++kk) acc += ta[ty][kk] * tb[kk][tx];
        __syncthreads();
    }
    if (m < M && n < N) C[static_cast<size_t>(m) * N + n] = acc;
}

unsigned ew_grid(size_t n) {
    const size_t g = (n + kOpThreads - 1) / kOpThreads;
    return static_cast<unsigned>(g < 4096 ? (g > 0 ? g : 1) : 4096);
}

unsigned reduce_threads(int n) {
    // One wave for short vectors (the tiny model's 32 elements), up to 1024.
    unsigned t = 64;
    while (t < kReduceThreads && static_cast<int>(t) < n) t <<= 1;
    return t;
}

}  // namespace

hipError_t launch_op_rmsnorm(const float* x, const float* w, int n, float eps, float* y, hipStream_t s) {
    hipLaunchKernelGGL(op_rmsnorm_kernel, dim3(1), dim3(reduce_threads(n)), 0, s, x, w, n, eps, y);
    return hipGetLastError();
}

hipError_t launch_op_elementwise(int op, const float* a, const float* b, size_t n, float* y, hipStream_t s) {
    switch (op) {
        case kOpSilu:
            hipLaunchKernelGGL(op_elementwise_kernel<Ew::Silu>, dim3(ew_grid(n)), dim3(kOpThreads), 0, s, a, b, n, y);
            break;
        case kOpMul:
            hipLaunchKernelGGL(op_elementwise_kernel<Ew::Mul>, dim3(ew_grid(n)), dim3(kOpThreads), 0, s, a, b, n, y);
            break;
        case kOpAdd:
            hipLaunchKernelGGL(op_elementwise_kernel<Ew::Add>, dim3(ew_grid(n)), dim3(kOpThreads), 0, s, a, b, n, y);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_op_softmax(const float* x, int n, float* y, hipStream_t s) {
    hipLaunchKernelGGL(op_softmax_kernel, dim3(1), dim3(reduce_threads(n)), 0, s, x, n, y);
    return hipGetLastError();
}

hipError_t launch_op_embedding(const float* table, int dim, int token, float* y, hipStream_t s) {
    hipLaunchKernelGGL(op_embedding_kernel, dim3(ew_grid(static_cast<size_t>(dim))), dim3(kOpThreads), 0, s, table,
                       dim, token, y);
    return hipGetLastError();
}

hipError_t launch_op_rope(float* x, int n_heads, int head_dim, int pos, float theta, bool neox, hipStream_t s) {
    const int pairs = n_heads * (head_dim / 2);
    hipLaunchKernelGGL(op_rope_kernel, dim3((pairs + kOpThreads - 1) / kOpThreads), dim3(kOpThreads), 0, s, x,
                       n_heads, head_dim, pos, theta, neox ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_op_attention_decode(const float* q, const float* keys, const float* values, int layer,
                                      int max_seq, int n_heads, int n_kv_heads, int head_dim, int pos,
                                      float* out, hipStream_t s) {
    const float scale = 1.0f / std::sqrt(static_cast<float>(head_dim));
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(n_heads), dim3(64 * kAttnWaves), 0, s, q, keys, values, layer, max_seq,
                           n_heads, n_kv_heads, head_dim, pos, scale, out);
    };
    if (head_dim <= 64) {
        go(op_attention_decode_kernel<1>);
    } else if (head_dim <= 128) {
        go(op_attention_decode_kernel<2>);
    } else if (head_dim <= 256) {
        go(op_attention_decode_kernel<4>);
    } else if (head_dim <= kOpAttnMaxHeadDim) {
        go(op_attention_decode_kernel<kOpAttnMaxHeadDim / 64>);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_op_matmul_f32(const float* a, const float* b, int m, int k, int n, bool b_transposed, float* c,
                                hipStream_t s) {
    const dim3 grid((n + kMatTile - 1) / kMatTile, (m + kMatTile - 1) / kMatTile);
    hipLaunchKernelGGL(op_matmul_f32_kernel, grid, dim3(kMatTile * kMatTile), 0, s, a, b, m, k, n,
                       b_transposed ? 1 : 0, c);
    return hipGetLastError();
}

}  // namespace mlq

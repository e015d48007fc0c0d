// Device-side weight quantizer (f32 -> Q8_0 / Q4_0 / Q4_1 blocks) and the
// synthetic normal generator used by benchmarks.
//
// The quantizers produce the same bytes as the reference's host routines:
//   quantize_to_q8_0  src/quant.cpp:112-170
//   quantize_to_q4_0  src/quant.cpp:207-270
//   Q4_1              tests/test_cuda_quant.cpp:129-180 (the only Q4_1 quantizer
//                     the reference has; its parity tests use it)
// Every step is an IEEE f32 operation with one rounding (|v|, max, a / 127,
// 1 / d, v * inv, v * inv + 8, (v - m) * inv) or integer work, so the device
// result matches the host bit for bit: hipcc divides with correct rounding
// (no fast-math), roundf rounds half away from zero like std::round, and no
// expression here can be contracted into an fma.  The scale is encoded with the
// reference's binary16 rule (round half up in magnitude at the first dropped
// bit, overflow and NaN to Inf, src/quant.cpp:19-55), not the hardware cvt.
//
// One thread quantizes one block; a block's 32 floats are read as 8 float4 when
// the row is 16-byte aligned and in range, element-wise otherwise.

#include "mlq_kernels.h"

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mlq {
namespace {

__device__ __forceinline__ uint32_t f32_bits(float v) { return __builtin_bit_cast(uint32_t, v); }

// f32 -> binary16 with the reference's rounding (see header comment).
__device__ uint16_t half_round_up(float value) {
    const uint32_t u = f32_bits(value);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const int e = static_cast<int>((u >> 23) & 0xffu) - 112;
    const uint32_t frac = u & 0x7fffffu;
    if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return static_cast<uint16_t>(sign);
        uint32_t sig = (frac | 0x800000u) >> (1 - e);
        sig += (sig & 0x1000u) << 1;  // +0x2000 when the first dropped bit is set
        return static_cast<uint16_t>(sign | (sig >> 13));
    }
    uint32_t sig = frac + ((frac & 0x1000u) << 1);
    int eh = e;
    if (sig & 0x800000u) {
        sig = 0;
        if (++eh >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    }
    return static_cast<uint16_t>(sign | (static_cast<uint32_t>(eh) << 10) | (sig >> 13));
}

__device__ __forceinline__ float half_value(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);  // exact (v_cvt_f32_f16)
}

__device__ __forceinline__ int round_int(float v) { return static_cast<int>(roundf(v)); }

template <int QT> struct QB;
template <> struct QB<1> { static constexpr int BB = 34; };
template <> struct QB<2> { static constexpr int BB = 18; };
template <> struct QB<3> { static constexpr int BB = 20; };

template <int QT>
__global__ __launch_bounds__(256) void quantize_kernel(const float* __restrict__ src, int rows,
                                                       int row_len, uint8_t* __restrict__ dst) {
    const int nb = (row_len + kQK - 1) / kQK;
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<long long>(rows) * nb) return;
    const int r = static_cast<int>(idx / nb);
    const int b = static_cast<int>(idx % nb);
    const float* p = src + static_cast<size_t>(r) * row_len + b * kQK;
    const int len = min(kQK, row_len - b * kQK);

    float v[kQK];
    if (len == kQK && (reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
#pragma unroll
        for (int i = 0; i < kQK / 4; ++i) {
            const float4 f = reinterpret_cast<const float4*>(p)[i];
            v[4 * i] = f.x;
            v[4 * i + 1] = f.y;
            v[4 * i + 2] = f.z;
            v[4 * i + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < kQK; ++i) v[i] = (i < len) ? p[i] : 0.0f;
    }

    uint8_t out[QB<QT>::BB];
#pragma unroll
    for (int i = 0; i < QB<QT>::BB; ++i) out[i] = 0;

    if (QT == 1 || QT == 2) {
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < kQK; ++i) {
            const float a = fabsf(v[i]);
            if (i < len && a > amax) amax = a;
        }
        if (amax > 0.0f) {
            const uint16_t dh = half_round_up(amax / (QT == 1 ? 127.0f : 7.0f));
            const float dq = half_value(dh);
            const float inv = (dq == 0.0f) ? 0.0f : 1.0f / dq;
            out[0] = static_cast<uint8_t>(dh & 0xff);
            out[1] = static_cast<uint8_t>(dh >> 8);
            if (QT == 1) {
#pragma unroll
                for (int i = 0; i < kQK; ++i) {
                    int q = round_int(v[i] * inv);
                    q = max(-127, min(127, q));
                    out[2 + i] = static_cast<uint8_t>(static_cast<int8_t>(i < len ? q : 0));
                }
            } else {
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const float lo = (j < len) ? v[j] * inv : 0.0f;
                    const float hi = (j + 16 < len) ? v[j + 16] * inv : 0.0f;
                    const int qlo = max(0, min(15, round_int(lo + 8.0f)));
                    const int qhi = max(0, min(15, round_int(hi + 8.0f)));
                    out[2 + j] = static_cast<uint8_t>(qlo | (qhi << 4));
                }
            }
        }
    } else {
        float lo = __builtin_inff();
        float hi = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < kQK; ++i) {
            if (i < len) {
                // std::min / std::max semantics: keep the first operand unless
                // the second compares strictly smaller / larger.
                lo = (v[i] < lo) ? v[i] : lo;
                hi = (hi < v[i]) ? v[i] : hi;
            }
        }
        const float range = hi - lo;
        uint16_t dh = 0;
        uint16_t mh;
        if (range > 0.0f) {
            dh = half_round_up(range / 15.0f);
            mh = half_round_up(lo);
            const float dq = half_value(dh);
            const float mq = half_value(mh);
            const float inv = (dq == 0.0f) ? 0.0f : 1.0f / dq;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                int q0 = (j < len) ? round_int((v[j] - mq) * inv) : 0;
                int q1 = (j + 16 < len) ? round_int((v[j + 16] - mq) * inv) : 0;
                q0 = max(0, min(15, q0));
                q1 = max(0, min(15, q1));
                out[4 + j] = static_cast<uint8_t>(q0 | (q1 << 4));
            }
        } else {
            mh = half_round_up(lo == __builtin_inff() ? 0.0f : lo);
        }
        out[0] = static_cast<uint8_t>(dh & 0xff);
        out[1] = static_cast<uint8_t>(dh >> 8);
        out[2] = static_cast<uint8_t>(mh & 0xff);
        out[3] = static_cast<uint8_t>(mh >> 8);
    }

    uint8_t* q = dst + static_cast<size_t>(idx) * QB<QT>::BB;
    // Blocks are 2-byte aligned (Q4_1: 4-byte); store as 16-bit halves.
    uint16_t* q16 = reinterpret_cast<uint16_t*>(q);
#pragma unroll
    for (int i = 0; i < QB<QT>::BB / 2; ++i) {
        q16[i] = static_cast<uint16_t>(out[2 * i] | (out[2 * i + 1] << 8));
    }
}

// splitmix64 (Steele, Lea, Flood 2014) on the element pair index, Box-Muller
// on the two 32-bit halves' top 24 bits.
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void fill_normal_kernel(float* __restrict__ dst, size_t n,
                                                          uint64_t seed, float mean,
                                                          float stddev) {
    const size_t pair = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t i0 = pair * 2;
    if (i0 >= n) return;
    const uint64_t h = splitmix64(seed ^ splitmix64(pair));
    const float u1 = (static_cast<float>(static_cast<uint32_t>(h >> 40)) + 1.0f) * (1.0f / 16777217.0f);
    const float u2 = static_cast<float>(static_cast<uint32_t>(h >> 8) & 0xffffffu) * (1.0f / 16777216.0f);
    const float rad = sqrtf(-2.0f * logf(u1));
    float s, c;
    sincosf(6.283185307179586f * u2, &s, &c);
    dst[i0] = mean + stddev * rad * c;
    if (i0 + 1 < n) dst[i0 + 1] = mean + stddev * rad * s;
}

template <int QT>
hipError_t launch_q(const float* src, int rows, int row_len, void* dst, hipStream_t stream) {
    const long long n = static_cast<long long>(rows) * ((row_len + kQK - 1) / kQK);
    const long long grid = (n + 255) / 256;
    hipLaunchKernelGGL((quantize_kernel<QT>), dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                       stream, src, rows, row_len, static_cast<uint8_t*>(dst));
    return hipGetLastError();
}

}  // namespace

hipError_t launch_quantize(int qtype, const float* src, int rows, int row_len, void* dst,
                           hipStream_t stream) {
    switch (qtype) {
        case 1: return launch_q<1>(src, rows, row_len, dst, stream);
        case 2: return launch_q<2>(src, rows, row_len, dst, stream);
        case 3: return launch_q<3>(src, rows, row_len, dst, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_fill_normal(float* dst, size_t n, uint64_t seed, float mean, float stddev,
                              hipStream_t stream) {
    const size_t pairs = (n + 1) / 2;
    const size_t grid = (pairs + 255) / 256;
    hipLaunchKernelGGL(fill_normal_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0, stream,
                       dst, n, seed, mean, stddev);
    return hipGetLastError();
}

}  // namespace mlq

// The prefill GEMM's split x, written per token row by a workgroup of 256
// threads.  Shared by the GEMM's own split kernel (gemm.hip) and by decoder
// kernels that produce a GEMM input and write it split straight away
// (decoder.hip), so both give the same halves.
//
// Layout (token-major): xs [npad][nb][64 halves] = per block the 32 scaled
// elements' fp16 hi then lo, in the k order of the GEMM's weight fragments;
// bsum [npad][nb] = per block the sum of the scaled elements (Q4_1's offset
// term); scale [npad] = the token's power-of-two scale s_n, chosen so that
// max|x_n| / s_n lies in [2^13, 2^14).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

namespace mlq {
namespace {

// Half blocks (16 elements) a thread holds: thread t holds half blocks
// t + 256 c, c < kXsCache, so rows of up to 16 384 elements are split from
// registers.
constexpr int kXsCache = 4;

typedef _Float16 xs_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 xs_h4 __attribute__((ext_vector_type(4)));

// max |x| over the workgroup (every thread gets it); `red` is 4 floats of LDS.
__device__ __forceinline__ float xsplit_row_max(float mx, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Power-of-two scale of a row with max |x| = mx: inv = 1 / s, sc = s.
__device__ __forceinline__ void xsplit_scale(float mx, float& inv, float& sc) {
    inv = 1.0f;
    sc = 1.0f;
    if (mx > 0.0f && mx <= 3.0e38f) {
        int ex = 0;
        (void)frexpf(mx, &ex);  // mx in [2^(ex-1), 2^ex)
        const int e = min(126, max(-126, 14 - ex));
        inv = ldexpf(1.0f, e);
        sc = ldexpf(1.0f, -e);
    }
}

// Scales, splits and stores half block hb of token row n (v: its 16
// elements).  Called by every lane (the shuffle pairs half blocks hb and
// hb ^ 1, held by adjacent lanes); lanes with hb >= 2 nb store nothing.
template <int QT>
__device__ __forceinline__ void xsplit_emit_half(int n, int nb, int hb, float (&v)[16], float inv,
                                                 _Float16* __restrict__ xs, float* __restrict__ bsum) {
    const bool have = hb < 2 * nb;
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] *= inv;
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) sum += (v[4 * q] + v[4 * q + 1]) + (v[4 * q + 2] + v[4 * q + 3]);
    const float other = __shfl_xor(sum, 1, 64);
    const int b = hb >> 1;
    const int half = hb & 1;
    if (!have) return;
    if (half == 0) {
        // block sum in the order (elements 0..15) + (16..31), 4-element groups
        bsum[static_cast<size_t>(n) * nb + b] = sum + other;
    }
    _Float16 hi[16], lo[16];
    // hi/lo in slot order of this half block
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        int e;  // element (0..15 within the half) that lands in the j-th slot of the half
        if (QT == 1) {
            e = j;
        } else {
            const int t = j & 3;
            e = 4 * (j >> 2) + ((t == 1) ? 2 : (t == 2) ? 1 : t);
        }
        const float f = v[e];
        const _Float16 h = static_cast<_Float16>(f);
        hi[j] = h;
        lo[j] = static_cast<_Float16>(f - static_cast<float>(h));
    }
    _Float16* dst = xs + (static_cast<size_t>(n) * nb + b) * 64;
    if (QT == 1) {
        // slots 16*half .. +15 (two 16-byte chunks) for hi, +32 for lo
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            *reinterpret_cast<xs_h8*>(dst + 16 * half + 8 * c) =
                xs_h8{hi[8 * c], hi[8 * c + 1], hi[8 * c + 2], hi[8 * c + 3], hi[8 * c + 4], hi[8 * c + 5],
                      hi[8 * c + 6], hi[8 * c + 7]};
            *reinterpret_cast<xs_h8*>(dst + 32 + 16 * half + 8 * c) =
                xs_h8{lo[8 * c], lo[8 * c + 1], lo[8 * c + 2], lo[8 * c + 3], lo[8 * c + 4], lo[8 * c + 5],
                      lo[8 * c + 6], lo[8 * c + 7]};
        }
    } else {
        // group g's slots 8g + 4*half .. +3 hold this half's elements 4g .. 4g+3
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            *reinterpret_cast<xs_h4*>(dst + 8 * g + 4 * half) = xs_h4{hi[4 * g], hi[4 * g + 1], hi[4 * g + 2], hi[4 * g + 3]};
            *reinterpret_cast<xs_h4*>(dst + 32 + 8 * g + 4 * half) =
                xs_h4{lo[4 * g], lo[4 * g + 1], lo[4 * g + 2], lo[4 * g + 3]};
        }
    }
}

// The whole split of token row n from the values the workgroup holds (thread
// t: half blocks t + 256 c in v[c], zeros past the row; 2 nb <= 256 C):
// the row's maximum, its scale (stored by thread 0) and every half block.
template <int QT, int C>
__device__ __forceinline__ void xsplit_emit_row(int n, int nb, float (&v)[C][16], _Float16* __restrict__ xs,
                                                float* __restrict__ bsum, float* __restrict__ scale, float* red) {
    float mx = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(v[c][i]));
    mx = xsplit_row_max(mx, red);
    float inv, sc;
    xsplit_scale(mx, inv, sc);
    if (threadIdx.x == 0) scale[n] = sc;
    const int iters = (2 * nb + 255) / 256;  // uniform across the workgroup
#pragma unroll
    for (int c = 0; c < C; ++c)
        if (c < iters) xsplit_emit_half<QT>(n, nb, static_cast<int>(threadIdx.x) + 256 * c, v[c], inv, xs, bsum);
}

}  // namespace
}  // namespace mlq

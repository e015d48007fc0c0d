// Batched prefill GEMM for Q8_0 / Q4_0 / Q4_1 weights on gfx950 (MI355X).
//
// Y[N, M] = X[N, K] . W[M, K]^T with N token rows (the rows > 1 case of the
// reference's linear, src/quant.cpp:384-386, 412, and of cuda_q*_linear with a
// [batch, in] x, src/cuda_quant.cu:270).  Two launches:
//
//  1. xsplit: per token n, a power-of-two scale s_n puts max|x_n| / s_n in
//     [2^13, 2^14); each scaled element x' is split into x' = hi + lo with
//     hi = fp16(x') and lo = fp16(x' - hi) (~22 significant bits in total) and
//     written in the k order the weight fragments use, plus per-block sums of
//     x' (Q4_1 offset term).
//  2. gemm: v_mfma_f32_16x16x32_f16 with A = X fragments (16 tokens x 32 k,
//     hi then lo) and B = weight fragments (32 k x 16 weight rows) holding the
//     block's integer codes as exact fp16 values (q, q - 8 or the Q8_0 byte).
//     One block is one MFMA K step; each block's product starts from zero and is
//     folded into the running f32 sum with the block scale d (and + m * sum(x')
//     for Q4_1): y = s_n * sum_b (d_b * sum_k q x' + m_b * sum_k x').
//     Products are exact, so the result carries only f32 accumulation error,
//     like the GEMV.  Rounding x to fp16 without the lo half would not meet the
//     1e-3 tolerance for Q8_0.
//  3. When K is split across workgroups (to fill 256 CUs at small N), partial
//     sums go to a workspace and a reduce kernel adds them in a fixed order.
//
// MFMA operand layouts (16x16x32 f16): lane l supplies row/column l % 16 and
// the eight k slots 8*(l/16) .. 8*(l/16)+7 of A and B; the result holds
// D[4*(l/16) + i][l % 16], i = 0..3.  The k order inside a block is free as long
// as A and B agree; it is chosen so that each lane's eight weight codes come
// from one aligned dword of nibbles (Q4: bytes 4g..4g+3 give elements
// {4g, 4g+2, 4g+1, 4g+3} from low nibbles and the same +16 from high nibbles)
// or two dwords of bytes (Q8_0: elements 8g..8g+7).
//
// Weight rows are read as dwords of 2-block pairs (36 / 68 / 40 bytes), which
// needs an even block count per row; other shapes use the GEMV kernels per row.

#include "mlq_kernels.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

namespace mlq {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h_lo(uint32_t v) { return (float)__builtin_bit_cast(h2_t, v).x; }
__device__ __forceinline__ float h_hi(uint32_t v) { return (float)__builtin_bit_cast(h2_t, v).y; }

template <int QT> struct GFmt;
template <> struct GFmt<1> { static constexpr int DW = 17; };
template <> struct GFmt<2> { static constexpr int DW = 9; };
template <> struct GFmt<3> { static constexpr int DW = 10; };

// k (within the block) of fragment slot j for lane group g.
template <int QT>
__device__ __forceinline__ int slot_k(int g, int j) {
    if (QT == 1) return 8 * g + j;
    const int base = (j < 4) ? 4 * g : 16 + 4 * g;
    const int t = j & 3;  // 0, 2, 1, 3 order within the byte quad
    return base + ((t == 1) ? 2 : (t == 2) ? 1 : t);
}

// ---------------------------------------------------------------------------
// xsplit: one workgroup per (padded) token row.
template <int QT>
__global__ __launch_bounds__(256) void xsplit_kernel(const float* __restrict__ x, int N, int K,
                                                     int nb, int npad, _Float16* __restrict__ xs,
                                                     float* __restrict__ bsum,
                                                     float* __restrict__ scale) {
    const int n = blockIdx.x;
    const bool valid = n < N;
    const float* xr = x + static_cast<size_t>(valid ? n : 0) * K;
    __shared__ float red[4];

    float mx = 0.0f;
    if (valid) {
        for (int k = threadIdx.x; k < K; k += 256) mx = fmaxf(mx, fabsf(xr[k]));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));

    // power-of-two scale: mx * inv in [2^13, 2^14)
    float inv = 1.0f, s = 1.0f;
    if (mx > 0.0f && mx <= 3.0e38f) {
        int ex = 0;
        (void)frexpf(mx, &ex);  // mx in [2^(ex-1), 2^ex)
        const int e = min(126, max(-126, 14 - ex));
        inv = ldexpf(1.0f, e);
        s = ldexpf(1.0f, -e);
    }
    if (threadIdx.x == 0) scale[n] = s;

    for (int b = threadIdx.x; b < nb; b += 256) {
        float v[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const int k = b * 32 + i;
            v[i] = (valid && k < K) ? xr[k] * inv : 0.0f;
        }
        float sum = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; ++q) sum += (v[4 * q] + v[4 * q + 1]) + (v[4 * q + 2] + v[4 * q + 3]);
        bsum[static_cast<size_t>(b) * npad + n] = sum;
        _Float16 hi[32], lo[32];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float f = v[slot_k<QT>(g, j)];
                const _Float16 h = static_cast<_Float16>(f);
                hi[8 * g + j] = h;
                lo[8 * g + j] = static_cast<_Float16>(f - static_cast<float>(h));
            }
        }
        u32x4* dst = reinterpret_cast<u32x4*>(xs + (static_cast<size_t>(b) * npad + n) * 64);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            dst[q] = __builtin_bit_cast(u32x4, f16x8{hi[8 * q], hi[8 * q + 1], hi[8 * q + 2], hi[8 * q + 3],
                                                      hi[8 * q + 4], hi[8 * q + 5], hi[8 * q + 6], hi[8 * q + 7]});
            dst[4 + q] = __builtin_bit_cast(u32x4, f16x8{lo[8 * q], lo[8 * q + 1], lo[8 * q + 2], lo[8 * q + 3],
                                                          lo[8 * q + 4], lo[8 * q + 5], lo[8 * q + 6], lo[8 * q + 7]});
        }
    }
}

// ---------------------------------------------------------------------------
// Weight fragment: the lane's 8 exact fp16 codes of one block, plus the block's
// d (and m for Q4_1) as f32.
struct WFrag {
    f16x8 b;
    float d;
    float m;
};

__device__ __forceinline__ uint32_t bias_sub(uint32_t v, uint32_t neg_bias2) {
    const h2_t r = __builtin_bit_cast(h2_t, v) + __builtin_bit_cast(h2_t, neg_bias2);
    return __builtin_bit_cast(uint32_t, r);
}

// Q4 nibble dword (bytes 4g..4g+3 of qs) -> 8 fp16 codes in slot order.
__device__ __forceinline__ f16x8 nibbles_to_f16(uint32_t q, uint32_t neg_bias2, uint32_t mask,
                                                uint32_t magic) {
    const uint32_t t0 = (q & mask) | magic;
    const uint32_t t1 = ((q >> 8) & mask) | magic;
    const uint32_t t2 = ((q >> 4) & mask) | magic;
    const uint32_t t3 = ((q >> 12) & mask) | magic;
    const u32x4 r{bias_sub(t0, neg_bias2), bias_sub(t1, neg_bias2), bias_sub(t2, neg_bias2),
                  bias_sub(t3, neg_bias2)};
    return __builtin_bit_cast(f16x8, r);
}

// Q8_0 byte dwords (qs bytes 8g..8g+7) -> 8 fp16 codes.
__device__ __forceinline__ f16x8 bytes_to_f16(uint32_t a, uint32_t b, uint32_t neg_bias2) {
    const uint32_t ax = a ^ 0x80808080u;
    const uint32_t bx = b ^ 0x80808080u;
    const uint32_t mb = 0x64646464u;
    const u32x4 r{bias_sub(__builtin_amdgcn_perm(mb, ax, 0x04010400u), neg_bias2),
                  bias_sub(__builtin_amdgcn_perm(mb, ax, 0x04030402u), neg_bias2),
                  bias_sub(__builtin_amdgcn_perm(mb, bx, 0x04010400u), neg_bias2),
                  bias_sub(__builtin_amdgcn_perm(mb, bx, 0x04030402u), neg_bias2)};
    return __builtin_bit_cast(f16x8, r);
}

template <int QT>
__device__ __forceinline__ void load_pair(const uint32_t* pw, int g, uint32_t (&r)[7]) {
    if (QT == 2) {  // Q4_0 pair: 9 dwords
        r[0] = pw[0];
        r[1] = pw[g];
        r[2] = pw[g + 1];
        r[3] = pw[4];
        r[4] = pw[5 + g];
    } else if (QT == 1) {  // Q8_0 pair: 17 dwords
        r[0] = pw[0];
        r[1] = pw[2 * g];
        r[2] = pw[2 * g + 1];
        r[3] = pw[2 * g + 2];
        r[4] = pw[8];
        r[5] = pw[9 + 2 * g];
        r[6] = pw[10 + 2 * g];
    } else {  // Q4_1 pair: 10 dwords, blocks 4-byte aligned
        r[0] = pw[0];
        r[1] = pw[1 + g];
        r[2] = pw[5];
        r[3] = pw[6 + g];
    }
}

template <int QT>
__device__ __forceinline__ void decode_pair(const uint32_t (&r)[7], WFrag& f0, WFrag& f1,
                                            uint32_t mask, uint32_t magic) {
    if (QT == 2) {
        const uint32_t nb2 = 0xE408E408u;  // {-1032.0h, -1032.0h}
        f0.b = nibbles_to_f16(__builtin_amdgcn_alignbit(r[2], r[1], 16), nb2, mask, magic);
        f0.d = h_lo(r[0]);
        f1.b = nibbles_to_f16(r[4], nb2, mask, magic);
        f1.d = h_hi(r[3]);
        f0.m = f1.m = 0.0f;
    } else if (QT == 1) {
        const uint32_t nb2 = 0xE480E480u;  // {-1152.0h, -1152.0h}
        f0.b = bytes_to_f16(__builtin_amdgcn_alignbit(r[2], r[1], 16),
                            __builtin_amdgcn_alignbit(r[3], r[2], 16), nb2);
        f0.d = h_lo(r[0]);
        f1.b = bytes_to_f16(r[5], r[6], nb2);
        f1.d = h_hi(r[4]);
        f0.m = f1.m = 0.0f;
    } else {
        const uint32_t nb2 = 0xE400E400u;  // {-1024.0h, -1024.0h}
        f0.b = nibbles_to_f16(r[1], nb2, mask, magic);
        f0.d = h_lo(r[0]);
        f0.m = h_hi(r[0]);
        f1.b = nibbles_to_f16(r[3], nb2, mask, magic);
        f1.d = h_lo(r[2]);
        f1.m = h_hi(r[2]);
    }
}

// One wave per workgroup; the wave owns 16*TM weight rows x 16*TN tokens and
// the pairs [p0, p1) of K.
template <int QT, int TM, int TN>
__global__ __launch_bounds__(64) void gemm_mfma_kernel(
    const uint8_t* __restrict__ W, const _Float16* __restrict__ xs, const float* __restrict__ bsum,
    const float* __restrict__ scale, float* __restrict__ y, float* __restrict__ part, int M, int N,
    int npad, int nb, int pairs_per_split) {
    constexpr int DW = GFmt<QT>::DW;
    const int lane = threadIdx.x;
    const int i16 = lane & 15;
    const int g = lane >> 4;
    const int m_base = blockIdx.x * (16 * TM);
    const int n_base = blockIdx.y * (16 * TN);
    const int np = nb >> 1;
    const int p0 = blockIdx.z * pairs_per_split;
    const int p1 = min(np, p0 + pairs_per_split);

    uint32_t mask = 0x000F000Fu, magic = 0x64006400u;
    asm volatile("" : "+v"(mask), "+v"(magic));

    const uint32_t* wrow[TM];
#pragma unroll
    for (int r = 0; r < TM; ++r) {
        const int m = min(m_base + 16 * r + i16, M - 1);
        wrow[r] = reinterpret_cast<const uint32_t*>(W) + static_cast<size_t>(m) * np * DW;
    }

    f32x4 acc[TN][TM];
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int r = 0; r < TM; ++r) acc[t][r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const f32x4 zero{0.0f, 0.0f, 0.0f, 0.0f};

    for (int p = p0; p < p1; ++p) {
        uint32_t raw[TM][7];
#pragma unroll
        for (int r = 0; r < TM; ++r) load_pair<QT>(wrow[r] + static_cast<size_t>(p) * DW, g, raw[r]);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int b = 2 * p + h;
            f16x8 ahi[TN], alo[TN];
            f32x4 sv[TN];
#pragma unroll
            for (int t = 0; t < TN; ++t) {
                const _Float16* src = xs + (static_cast<size_t>(b) * npad + n_base + 16 * t + i16) * 64 + 8 * g;
                ahi[t] = *reinterpret_cast<const f16x8*>(src);
                alo[t] = *reinterpret_cast<const f16x8*>(src + 32);
                if (QT == 3) {
                    sv[t] = *reinterpret_cast<const f32x4*>(bsum + static_cast<size_t>(b) * npad + n_base + 16 * t + 4 * g);
                }
            }
#pragma unroll
            for (int r = 0; r < TM; ++r) {
                WFrag f0, f1;
                decode_pair<QT>(raw[r], f0, f1, mask, magic);
                const WFrag& f = h ? f1 : f0;
#pragma unroll
                for (int t = 0; t < TN; ++t) {
                    f32x4 blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[t], f.b, zero, 0, 0, 0);
                    blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[t], f.b, blk, 0, 0, 0);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        acc[t][r][q] = __builtin_fmaf(f.d, blk[q], acc[t][r][q]);
                        if (QT == 3) acc[t][r][q] = __builtin_fmaf(f.m, sv[t][q], acc[t][r][q]);
                    }
                }
            }
        }
    }

#pragma unroll
    for (int t = 0; t < TN; ++t) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n = n_base + 16 * t + 4 * g + q;
            if (n >= N) continue;
            const float sn = scale[n];
#pragma unroll
            for (int r = 0; r < TM; ++r) {
                const int m = m_base + 16 * r + i16;
                if (m >= M) continue;
                if (part == nullptr) {
                    y[static_cast<size_t>(n) * M + m] = acc[t][r][q] * sn;
                } else {
                    part[(static_cast<size_t>(blockIdx.z) * npad + n) * M + m] = acc[t][r][q];
                }
            }
        }
    }
}

__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part,
                                                            const float* __restrict__ scale,
                                                            float* __restrict__ y, int M, int N,
                                                            int npad, int splits) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= static_cast<size_t>(N) * M) return;
    const int n = static_cast<int>(idx / M);
    const int m = static_cast<int>(idx % M);
    float s = 0.0f;
    for (int k = 0; k < splits; ++k) s += part[(static_cast<size_t>(k) * npad + n) * M + m];
    y[idx] = s * scale[n];
}

// ---------------------------------------------------------------------------
struct GemmCfg {
    int tm, tn, splits, pairs_per_split, npad;
};

GemmCfg choose(const LinearShape& s) {
    GemmCfg c;
    c.tm = 4;
    c.tn = s.rows <= 16 ? 1 : (s.rows <= 32 ? 2 : 4);
    c.npad = (s.rows + 16 * c.tn - 1) / (16 * c.tn) * (16 * c.tn);
    const int np = s.nb / 2;
    const long long waves = static_cast<long long>((s.M + 16 * c.tm - 1) / (16 * c.tm)) * (c.npad / (16 * c.tn));
    int splits = static_cast<int>((1024 + waves - 1) / waves);
    splits = max(1, min(splits, np / 2));  // at least two pairs per split
    c.pairs_per_split = (np + splits - 1) / splits;
    c.splits = (np + c.pairs_per_split - 1) / c.pairs_per_split;
    return c;
}

struct WsLayout {
    size_t xs, bsum, scale, part, total;
};

WsLayout layout(const LinearShape& s, const GemmCfg& c) {
    auto up = [](size_t v) { return (v + 255) & ~static_cast<size_t>(255); };
    WsLayout l;
    l.xs = 0;
    l.bsum = up(static_cast<size_t>(s.nb) * c.npad * 64 * sizeof(_Float16));
    l.scale = l.bsum + up(static_cast<size_t>(s.nb) * c.npad * sizeof(float));
    l.part = l.scale + up(static_cast<size_t>(c.npad) * sizeof(float));
    l.total = l.part + (c.splits > 1 ? up(static_cast<size_t>(c.splits) * c.npad * s.M * sizeof(float)) : 0);
    return l;
}

template <int QT, int TM, int TN>
hipError_t launch_t(const LinearShape& s, const GemmCfg& c, const WsLayout& l, const void* w,
                    const float* x, float* y, char* ws, hipStream_t stream) {
    _Float16* xs = reinterpret_cast<_Float16*>(ws + l.xs);
    float* bsum = reinterpret_cast<float*>(ws + l.bsum);
    float* scale = reinterpret_cast<float*>(ws + l.scale);
    float* part = c.splits > 1 ? reinterpret_cast<float*>(ws + l.part) : nullptr;
    hipLaunchKernelGGL((xsplit_kernel<QT>), dim3(c.npad), dim3(256), 0, stream, x, s.rows, s.K, s.nb,
                       c.npad, xs, bsum, scale);
    dim3 grid((s.M + 16 * TM - 1) / (16 * TM), c.npad / (16 * TN), c.splits);
    hipLaunchKernelGGL((gemm_mfma_kernel<QT, TM, TN>), grid, dim3(64), 0, stream,
                       static_cast<const uint8_t*>(w), xs, bsum, scale, y, part, s.M, s.rows, c.npad, s.nb,
                       c.pairs_per_split);
    if (part != nullptr) {
        const size_t total = static_cast<size_t>(s.rows) * s.M;
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                           stream, part, scale, y, s.M, s.rows, c.npad, c.splits);
    }
    return hipGetLastError();
}

template <int QT>
hipError_t launch_q(const LinearShape& s, const GemmCfg& c, const WsLayout& l, const void* w,
                    const float* x, float* y, char* ws, hipStream_t stream) {
    switch (c.tn) {
        case 1: return launch_t<QT, 4, 1>(s, c, l, w, x, y, ws, stream);
        case 2: return launch_t<QT, 4, 2>(s, c, l, w, x, y, ws, stream);
        default: return launch_t<QT, 4, 4>(s, c, l, w, x, y, ws, stream);
    }
}

}  // namespace

bool gemm_supported(const LinearShape& s) {
    return s.rows > 1 && s.nb % 2 == 0 && s.nb >= 2 && (s.qtype >= 1 && s.qtype <= 3);
}

size_t gemm_workspace_bytes(const LinearShape& s) {
    if (!gemm_supported(s)) return 0;
    return layout(s, choose(s)).total;
}

hipError_t launch_gemm(const LinearShape& s, const void* w, const float* x, float* y, void* ws,
                       size_t ws_bytes, hipStream_t stream) {
    if (!gemm_supported(s)) return hipErrorNotSupported;
    const GemmCfg c = choose(s);
    const WsLayout l = layout(s, c);
    if (ws == nullptr || ws_bytes < l.total) return hipErrorInvalidValue;
    char* base = static_cast<char*>(ws);
    switch (s.qtype) {
        case 1: return launch_q<1>(s, c, l, w, x, y, base, stream);
        case 2: return launch_q<2>(s, c, l, w, x, y, base, stream);
        default: return launch_q<3>(s, c, l, w, x, y, base, stream);
    }
}

const char* gemm_kernel_name(const LinearShape& s) {
    static thread_local char buf[96];
    const GemmCfg c = choose(s);
    const char* fmt = s.qtype == 1 ? "q8_0" : s.qtype == 2 ? "q4_0" : "q4_1";
    snprintf(buf, sizeof buf, "gemm_mfma_%s_tm%d_tn%d_splitk%d", fmt, c.tm, c.tn, c.splits);
    return buf;
}

}  // namespace mlq

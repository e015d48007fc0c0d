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
// xsplit: one workgroup per (padded) token row; thread t takes the half blocks
// t, t + 256, ... (16 consecutive floats each, so a wave reads 4 KB contiguous).
// Pass 1 finds max|x| of the row, pass 2 (L2 hits) scales, splits and writes
// each half block's 16 hi and 16 lo halves into its fragment slots.
template <int QT>
__global__ __launch_bounds__(256) void xsplit_kernel(const float* __restrict__ x, int N, int K,
                                                     int nb, int npad, _Float16* __restrict__ xs,
                                                     float* __restrict__ bsum,
                                                     float* __restrict__ scale) {
    const int n = blockIdx.x;
    const bool valid = n < N;
    const float* xr = x + static_cast<size_t>(valid ? n : 0) * K;
    __shared__ float red[4];
    const int nhb = 2 * nb;

    auto load16 = [&](int hb, float (&v)[16]) {
        const int k0 = hb * 16;
        if (valid && k0 + 16 <= K && (reinterpret_cast<uintptr_t>(xr + k0) & 15u) == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 f = reinterpret_cast<const float4*>(xr + k0)[i];
                v[4 * i] = f.x;
                v[4 * i + 1] = f.y;
                v[4 * i + 2] = f.z;
                v[4 * i + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = (valid && k0 + i < K) ? xr[k0 + i] : 0.0f;
        }
    };

    float mx = 0.0f;
    for (int hb = threadIdx.x; hb < nhb; hb += 256) {
        float v[16];
        load16(hb, v);
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(v[i]));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));

    // power-of-two scale: mx * inv in [2^13, 2^14)
    float inv = 1.0f, sc = 1.0f;
    if (mx > 0.0f && mx <= 3.0e38f) {
        int ex = 0;
        (void)frexpf(mx, &ex);  // mx in [2^(ex-1), 2^ex)
        const int e = min(126, max(-126, 14 - ex));
        inv = ldexpf(1.0f, e);
        sc = ldexpf(1.0f, -e);
    }
    if (threadIdx.x == 0) scale[n] = sc;

    // The loop bound is uniform per wave pair, so the shuffle partner exists.
    const int iters = (nhb + 255) / 256;
    for (int it = 0; it < iters; ++it) {
        const int hb = threadIdx.x + 256 * it;
        const bool have = hb < nhb;
        float v[16];
        if (have) {
            load16(hb, v);
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] *= inv;
        float sum = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) sum += (v[4 * q] + v[4 * q + 1]) + (v[4 * q + 2] + v[4 * q + 3]);
        const float other = __shfl_xor(sum, 1, 64);
        const int b = hb >> 1;
        const int half = hb & 1;
        if (!have) continue;
        if (half == 0) {
            // block sum in the order (elements 0..15) + (16..31), 4-element groups
            bsum[static_cast<size_t>(b) * npad + n] = sum + other;
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
        _Float16* dst = xs + (static_cast<size_t>(b) * npad + n) * 64;
        if (QT == 1) {
            // slots 16*half .. +15 (two 16-byte chunks) for hi, +32 for lo
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                *reinterpret_cast<f16x8*>(dst + 16 * half + 8 * c) =
                    f16x8{hi[8 * c], hi[8 * c + 1], hi[8 * c + 2], hi[8 * c + 3], hi[8 * c + 4], hi[8 * c + 5],
                          hi[8 * c + 6], hi[8 * c + 7]};
                *reinterpret_cast<f16x8*>(dst + 32 + 16 * half + 8 * c) =
                    f16x8{lo[8 * c], lo[8 * c + 1], lo[8 * c + 2], lo[8 * c + 3], lo[8 * c + 4], lo[8 * c + 5],
                          lo[8 * c + 6], lo[8 * c + 7]};
            }
        } else {
            // group g's slots 8g + 4*half .. +3 hold this half's elements 4g .. 4g+3
            typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                *reinterpret_cast<f16x4*>(dst + 8 * g + 4 * half) =
                    f16x4{hi[4 * g], hi[4 * g + 1], hi[4 * g + 2], hi[4 * g + 3]};
                *reinterpret_cast<f16x4*>(dst + 32 + 8 * g + 4 * half) =
                    f16x4{lo[4 * g], lo[4 * g + 1], lo[4 * g + 2], lo[4 * g + 3]};
            }
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

// Tiled MFMA kernel: a workgroup of four waves owns BM weight rows x BN tokens
// and the pairs [p0, p1) of K.  Per pair, the workgroup copies the raw weight
// dwords (BM rows x one pair) and the split x fragments (2 blocks x BN tokens x
// 32 hi + 32 lo halves) from global memory into LDS, double-buffered, so every
// weight byte is read once per token tile and every x fragment once per row
// tile.  The waves are arranged WM x WN over the tile; a wave decodes the codes
// of its own row tiles from LDS and multiplies them with every token tile it
// owns.
constexpr int kGemmThreads = 256;
constexpr int kGemmMaxTiles = 65536;  // split-K arrival counters in the workspace
constexpr int kXRowHalves = 72;  // 64 halves of one token's block + 8 of padding (bank spread)

template <int QT, int BM, int BN>
struct TileLds {
    static constexpr int DW = GFmt<QT>::DW;
    static constexpr int w_dwords = BM * DW;                 // raw pair dwords, row-major
    static constexpr int x_halves = 2 * BN * kXRowHalves;    // [block][token][72]
    static constexpr int s_floats = QT == 3 ? 2 * BN : 0;    // Q4_1 block sums [block][token]
    static constexpr int stage_bytes = w_dwords * 4 + x_halves * 2 + s_floats * 4;
    static constexpr int bytes = 2 * stage_bytes;
};

template <int QT, int BM, int BN>
__device__ __forceinline__ void tile_load_global(const uint32_t* const (&wrow)[(BM * GFmt<QT>::DW + kGemmThreads - 1) / kGemmThreads],
                                                 const _Float16* __restrict__ xs, const float* __restrict__ bsum,
                                                 int npad, int n_base, int p,
                                                 uint32_t (&wr)[(BM * GFmt<QT>::DW + kGemmThreads - 1) / kGemmThreads],
                                                 u32x4 (&xr)[(2 * BN * 8 + kGemmThreads - 1) / kGemmThreads],
                                                 float (&sr)[QT == 3 ? (2 * BN + kGemmThreads - 1) / kGemmThreads : 1]) {
    constexpr int DW = GFmt<QT>::DW;
    constexpr int WN_ = (BM * DW + kGemmThreads - 1) / kGemmThreads;
    constexpr int XN = (2 * BN * 8 + kGemmThreads - 1) / kGemmThreads;
    // Unconditional loads (indices clamped where the tile is not a multiple of
    // the thread count; the copies past the end are never stored), so the
    // compiler can count them in order instead of waiting for all of them.
#pragma unroll
    for (int j = 0; j < WN_; ++j) wr[j] = wrow[j][static_cast<size_t>(p) * DW];
#pragma unroll
    for (int j = 0; j < XN; ++j) {
        const int idx = min(static_cast<int>(threadIdx.x) + j * kGemmThreads, 2 * BN * 8 - 1);  // [h][t][c]
        const int c = idx & 7;
        const int t = (idx >> 3) % BN;
        const int h = (idx >> 3) / BN;
        const size_t off = (static_cast<size_t>(2 * p + h) * npad + n_base + t) * 64 + 8 * c;
        xr[j] = *reinterpret_cast<const u32x4*>(xs + off);
    }
    if (QT == 3) {
#pragma unroll
        for (int j = 0; j < (2 * BN + kGemmThreads - 1) / kGemmThreads; ++j) {
            const int idx = min(static_cast<int>(threadIdx.x) + j * kGemmThreads, 2 * BN - 1);
            const int t = idx % BN;
            const int h = idx / BN;
            sr[j] = bsum[static_cast<size_t>(2 * p + h) * npad + n_base + t];
        }
    }
}

template <int QT, int BM, int BN>
__device__ __forceinline__ void tile_store_lds(char* stage,
                                               const uint32_t (&wr)[(BM * GFmt<QT>::DW + kGemmThreads - 1) / kGemmThreads],
                                               const u32x4 (&xr)[(2 * BN * 8 + kGemmThreads - 1) / kGemmThreads],
                                               const float (&sr)[QT == 3 ? (2 * BN + kGemmThreads - 1) / kGemmThreads : 1]) {
    using L = TileLds<QT, BM, BN>;
    constexpr int DW = GFmt<QT>::DW;
    uint32_t* wl = reinterpret_cast<uint32_t*>(stage);
    _Float16* xl = reinterpret_cast<_Float16*>(stage + L::w_dwords * 4);
    float* sl = reinterpret_cast<float*>(stage + L::w_dwords * 4 + L::x_halves * 2);
#pragma unroll
    for (int j = 0; j < (BM * DW + kGemmThreads - 1) / kGemmThreads; ++j) {
        const int idx = threadIdx.x + j * kGemmThreads;
        if (idx < BM * DW) wl[idx] = wr[j];
    }
#pragma unroll
    for (int j = 0; j < (2 * BN * 8 + kGemmThreads - 1) / kGemmThreads; ++j) {
        const int idx = threadIdx.x + j * kGemmThreads;
        if (idx < 2 * BN * 8) {
            const int c = idx & 7;
            const int row = idx >> 3;  // h * BN + t
            *reinterpret_cast<u32x4*>(xl + row * kXRowHalves + 8 * c) = xr[j];
        }
    }
    if (QT == 3) {
#pragma unroll
        for (int j = 0; j < (2 * BN + kGemmThreads - 1) / kGemmThreads; ++j) {
            const int idx = threadIdx.x + j * kGemmThreads;
            if (idx < 2 * BN) sl[idx] = sr[j];
        }
    }
}

// Weight fragment of block h (0/1) of the pair for row `row` of the tile, from
// the raw pair dwords in LDS.
template <int QT>
__device__ __forceinline__ void lds_wfrag(const uint32_t* wl, int row, int g, int h, WFrag& f, uint32_t mask,
                                          uint32_t magic) {
    constexpr int DW = GFmt<QT>::DW;
    const uint32_t* pw = wl + row * DW;
    if (QT == 2) {
        const uint32_t nb2 = 0xE408E408u;  // {-1032.0h, -1032.0h}
        if (h == 0) {
            f.b = nibbles_to_f16(__builtin_amdgcn_alignbit(pw[g + 1], pw[g], 16), nb2, mask, magic);
            f.d = h_lo(pw[0]);
        } else {
            f.b = nibbles_to_f16(pw[5 + g], nb2, mask, magic);
            f.d = h_hi(pw[4]);
        }
        f.m = 0.0f;
    } else if (QT == 1) {
        const uint32_t nb2 = 0xE480E480u;  // {-1152.0h, -1152.0h}
        if (h == 0) {
            f.b = bytes_to_f16(__builtin_amdgcn_alignbit(pw[2 * g + 1], pw[2 * g], 16),
                               __builtin_amdgcn_alignbit(pw[2 * g + 2], pw[2 * g + 1], 16), nb2);
            f.d = h_lo(pw[0]);
        } else {
            f.b = bytes_to_f16(pw[9 + 2 * g], pw[10 + 2 * g], nb2);
            f.d = h_hi(pw[8]);
        }
        f.m = 0.0f;
    } else {
        const uint32_t nb2 = 0xE400E400u;  // {-1024.0h, -1024.0h}
        const int o = 5 * h;
        f.b = nibbles_to_f16(pw[o + 1 + g], nb2, mask, magic);
        f.d = h_lo(pw[o]);
        f.m = h_hi(pw[o]);
    }
}

template <int QT, int BM, int BN, int WM, int WN, int D>
__global__ __launch_bounds__(kGemmThreads) void gemm_tile_kernel(
    const uint8_t* __restrict__ W, const _Float16* __restrict__ xs, const float* __restrict__ bsum,
    const float* __restrict__ scale, float* __restrict__ y, float* __restrict__ part,
    unsigned* __restrict__ tile_count, int M, int N, int npad, int nb, int pairs_per_split) {
    using L = TileLds<QT, BM, BN>;
    constexpr int DW = GFmt<QT>::DW;
    constexpr int RT = BM / (16 * WM);  // row tiles per wave
    constexpr int TT = BN / (16 * WN);  // token tiles per wave
    constexpr int WLD = (BM * DW + kGemmThreads - 1) / kGemmThreads;
    constexpr int XLD = (2 * BN * 8 + kGemmThreads - 1) / kGemmThreads;
    constexpr int SLD = QT == 3 ? (2 * BN + kGemmThreads - 1) / kGemmThreads : 1;
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN;
    const int wn = wave % WN;
    const int i16 = lane & 15;
    const int g = lane >> 4;
    const int m_base = blockIdx.x * BM;
    const int n_base = blockIdx.y * BN;
    const int np = nb >> 1;
    const int p0 = blockIdx.z * pairs_per_split;
    const int p1 = min(np, p0 + pairs_per_split);

    uint32_t mask = 0x000F000Fu, magic = 0x64006400u;
    asm volatile("" : "+v"(mask), "+v"(magic));

    // Global row pointers of the raw-weight dwords this thread copies.
    const uint32_t* wrow[WLD];
#pragma unroll
    for (int j = 0; j < WLD; ++j) {
        const int idx = min(static_cast<int>(threadIdx.x) + j * kGemmThreads, BM * DW - 1);
        const int r = idx / DW;
        const int m = min(m_base + r, M - 1);  // rows past M copy row M-1; results dropped
        wrow[j] = reinterpret_cast<const uint32_t*>(W) + static_cast<size_t>(m) * np * DW + (idx - r * DW);
    }

    f32x4 acc[RT][TT];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[r][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const f32x4 zero{0.0f, 0.0f, 0.0f, 0.0f};

    // Pipeline: pair q's global loads are issued D pairs ahead into register
    // set q % D; at step q they go to LDS buffer q & 1, the workgroup syncs, the
    // loads for pair q + D are issued into the freed set, and the waves compute
    // pair q from LDS.  One barrier per pair: the buffer written at step q was
    // last read at step q - 2, before the barrier of step q - 1.
    uint32_t wr[D][WLD];
    u32x4 xr[D][XLD];
    float sr[D][SLD];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (p0 + d < p1) tile_load_global<QT, BM, BN>(wrow, xs, bsum, npad, n_base, p0 + d, wr[d], xr[d], sr[d]);
    }

    // Step q: LDS buffer (q - p0) & 1 <- register set d; barrier; optionally
    // request pair q + D into set d; compute pair q.
    auto step = [&](int q, auto& wrd, auto& xrd, auto& srd, bool refill) {
        char* cur = smem + ((q - p0) & 1) * L::stage_bytes;
        tile_store_lds<QT, BM, BN>(cur, wrd, xrd, srd);
        __syncthreads();
        if (refill) tile_load_global<QT, BM, BN>(wrow, xs, bsum, npad, n_base, q + D, wrd, xrd, srd);
        const uint32_t* wl = reinterpret_cast<const uint32_t*>(cur);
        const _Float16* xl = reinterpret_cast<const _Float16*>(cur + L::w_dwords * 4);
        const float* sl = reinterpret_cast<const float*>(cur + L::w_dwords * 4 + L::x_halves * 2);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            f16x8 ahi[TT], alo[TT];
            f32x4 sv[TT];
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const int tok = (wn * TT + t) * 16 + i16;
                const _Float16* src = xl + (h * BN + tok) * kXRowHalves + 8 * g;
                ahi[t] = *reinterpret_cast<const f16x8*>(src);
                alo[t] = *reinterpret_cast<const f16x8*>(src + 32);
                if (QT == 3) sv[t] = *reinterpret_cast<const f32x4*>(sl + h * BN + (wn * TT + t) * 16 + 4 * g);
            }
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                WFrag f;
                lds_wfrag<QT>(wl, (wm * RT + r) * 16 + i16, g, h, f, mask, magic);
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    f32x4 blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[t], f.b, zero, 0, 0, 0);
                    blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[t], f.b, blk, 0, 0, 0);
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) {
                        acc[r][t][qq] = __builtin_fmaf(f.d, blk[qq], acc[r][t][qq]);
                        if (QT == 3) acc[r][t][qq] = __builtin_fmaf(f.m, sv[t][qq], acc[r][t][qq]);
                    }
                }
            }
        }
    };

    // Steady state: every step refills its set (no conditional loads).
    int q = p0;
    for (; q + 2 * D <= p1; q += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) step(q + d, wr[d], xr[d], sr[d], true);
    }
    // Drain: the remaining pairs (at most 2D - 1) refill only while pairs remain.
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (q + d < p1) step(q + d, wr[d], xr[d], sr[d], q + d + D < p1);
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (q + D + d < p1) step(q + D + d, wr[d], xr[d], sr[d], false);
    }
    __syncthreads();

    if (part == nullptr) {
#pragma unroll
        for (int t = 0; t < TT; ++t) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n_base + (wn * TT + t) * 16 + 4 * g + q;
                if (n >= N) continue;
                const float sn = scale[n];
#pragma unroll
                for (int r = 0; r < RT; ++r) {
                    const int m = m_base + (wm * RT + r) * 16 + i16;
                    if (m < M) y[static_cast<size_t>(n) * M + m] = acc[r][t][q] * sn;
                }
            }
        }
        return;
    }

    // Split K: write this split's partial tile with agent-scope stores, then
    // count in; the workgroup that completes the count sums the tile's
    // partials in split order (deterministic), writes y and resets the count.
#pragma unroll
    for (int t = 0; t < TT; ++t) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n = n_base + (wn * TT + t) * 16 + 4 * g + q;
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const int m = m_base + (wm * RT + r) * 16 + i16;
                if (n < N && m < M) {
                    __hip_atomic_store(part + (static_cast<size_t>(blockIdx.z) * npad + n) * M + m, acc[r][t][q],
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __shared__ unsigned last;
    __syncthreads();
    const unsigned tile = blockIdx.y * gridDim.x + blockIdx.x;
    if (threadIdx.x == 0) {
        const unsigned done = __hip_atomic_fetch_add(tile_count + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = done == gridDim.z - 1 ? 1u : 0u;
    }
    __syncthreads();
    if (last == 0u) return;
    // Every thread sums E tile elements over the splits in split order, with
    // all loads of four splits in flight at once (the loads bypass stale
    // caches, so each is a memory round trip).
    constexpr int E = (BM * BN) / kGemmThreads;
    static_assert((BM * BN) % kGemmThreads == 0, "tile must be a multiple of the workgroup");
    float sum[E];
    size_t off[E];
#pragma unroll
    for (int i = 0; i < E; ++i) {
        const int e = threadIdx.x + i * kGemmThreads;
        const int n = min(n_base + e / BM, N - 1);  // clamped; out-of-range results are not stored
        const int m = min(m_base + e % BM, M - 1);
        off[i] = static_cast<size_t>(n) * M + m;
        sum[i] = 0.0f;
    }
    const size_t zstride = static_cast<size_t>(npad) * M;
    const unsigned S = gridDim.z;
    unsigned k = 0;
    for (; k + 4 <= S; k += 4) {
        float v[4][E];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int i = 0; i < E; ++i)
                v[u][i] = __hip_atomic_load(part + (k + u) * zstride + off[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int i = 0; i < E; ++i) sum[i] += v[u][i];
    }
    for (; k < S; ++k) {
#pragma unroll
        for (int i = 0; i < E; ++i)
            sum[i] += __hip_atomic_load(part + k * zstride + off[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int i = 0; i < E; ++i) {
        const int e = threadIdx.x + i * kGemmThreads;
        const int n = n_base + e / BM;
        const int m = m_base + e % BM;
        if (n < N && m < M) y[static_cast<size_t>(n) * M + m] = sum[i] * scale[n];
    }
    if (threadIdx.x == 0) __hip_atomic_store(tile_count + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Tile configurations: skinny N (decode-like batches) streams each weight
// byte once with one 16-row tile per wave; wide N (prefill) gives each wave
// 64 rows x 32 tokens so decoded weight fragments and x fragments are reused
// across several MFMAs.  K is split across workgroups until the grid covers
// the CUs (partials reduced in a fixed order).
enum class Tile { N16, N32, N64, Wide };

// Pairs in flight per workgroup (register sets of the load pipeline).
constexpr int kDepthN16 = 4;
constexpr int kDepthN32 = 4;
constexpr int kDepthN64 = 4;
constexpr int kDepthWide = 2;

struct GemmCfg {
    Tile tile;
    int bm, bn, splits, pairs_per_split, npad, lds;
};

template <int QT>
int tile_lds(Tile t) {
    switch (t) {
        case Tile::N16: return TileLds<QT, 64, 16>::bytes;
        case Tile::N32: return TileLds<QT, 64, 32>::bytes;
        case Tile::N64: return TileLds<QT, 64, 64>::bytes;
        default: return TileLds<QT, 128, 64>::bytes;
    }
}

GemmCfg choose(const LinearShape& s) {
    GemmCfg c;
    if (s.rows <= 16) {
        c.tile = Tile::N16, c.bm = 64, c.bn = 16;
    } else if (s.rows <= 32) {
        c.tile = Tile::N32, c.bm = 64, c.bn = 32;
    } else if (s.rows <= 64) {
        c.tile = Tile::N64, c.bm = 64, c.bn = 64;
    } else {
        c.tile = Tile::Wide, c.bm = 128, c.bn = 64;
    }
    c.lds = s.qtype == 1 ? tile_lds<1>(c.tile) : s.qtype == 2 ? tile_lds<2>(c.tile) : tile_lds<3>(c.tile);
    c.npad = (s.rows + c.bn - 1) / c.bn * c.bn;
    const int np = s.nb / 2;
    const long long tiles = static_cast<long long>((s.M + c.bm - 1) / c.bm) * (c.npad / c.bn);
    // About one workgroup per CU (two for the narrow tiles), and at least two
    // prefetch depths of pairs per split so each workgroup's pipeline fills.
    const int depth = c.tile == Tile::N16 ? kDepthN16 : c.tile == Tile::N32 ? kDepthN32
                    : c.tile == Tile::N64 ? kDepthN64 : kDepthWide;
    const long long target = c.tile == Tile::Wide ? 256 : 512;
    int splits = static_cast<int>((target + tiles - 1) / tiles);
    splits = max(1, min(splits, np / (2 * depth)));
    if (tiles > kGemmMaxTiles) splits = 1;
    c.pairs_per_split = (np + splits - 1) / splits;
    c.splits = (np + c.pairs_per_split - 1) / c.pairs_per_split;
    return c;
}

struct WsLayout {
    size_t xs, bsum, scale, count, part, total;
};

// The split-K arrival counters sit at the start of every layout: all shapes
// that share a workspace share them, and every launch leaves them at zero.
WsLayout layout(const LinearShape& s, const GemmCfg& c) {
    auto up = [](size_t v) { return (v + 255) & ~static_cast<size_t>(255); };
    WsLayout l;
    l.count = 0;
    l.xs = up(static_cast<size_t>(kGemmMaxTiles) * sizeof(unsigned));
    l.bsum = l.xs + up(static_cast<size_t>(s.nb) * c.npad * 64 * sizeof(_Float16));
    l.scale = l.bsum + up(static_cast<size_t>(s.nb) * c.npad * sizeof(float));
    l.part = l.scale + up(static_cast<size_t>(c.npad) * sizeof(float));
    l.total = l.part + (c.splits > 1 ? up(static_cast<size_t>(c.splits) * c.npad * s.M * sizeof(float)) : 0);
    return l;
}

template <int QT, int BM, int BN, int WM, int WN, int D>
hipError_t launch_t(const LinearShape& s, const GemmCfg& c, const WsLayout& l, const void* w,
                    const float* x, float* y, char* ws, hipStream_t stream) {
    _Float16* xs = reinterpret_cast<_Float16*>(ws + l.xs);
    float* bsum = reinterpret_cast<float*>(ws + l.bsum);
    float* scale = reinterpret_cast<float*>(ws + l.scale);
    float* part = c.splits > 1 ? reinterpret_cast<float*>(ws + l.part) : nullptr;
    unsigned* count = reinterpret_cast<unsigned*>(ws + l.count);
    hipLaunchKernelGGL((xsplit_kernel<QT>), dim3(c.npad), dim3(256), 0, stream, x, s.rows, s.K, s.nb,
                       c.npad, xs, bsum, scale);
    dim3 grid((s.M + BM - 1) / BM, c.npad / BN, c.splits);
    constexpr int lds = TileLds<QT, BM, BN>::bytes;
    hipLaunchKernelGGL((gemm_tile_kernel<QT, BM, BN, WM, WN, D>), grid, dim3(kGemmThreads), lds, stream,
                       static_cast<const uint8_t*>(w), xs, bsum, scale, y, part, count, s.M, s.rows, c.npad,
                       s.nb, c.pairs_per_split);
    return hipGetLastError();
}

template <int QT>
hipError_t launch_q(const LinearShape& s, const GemmCfg& c, const WsLayout& l, const void* w,
                    const float* x, float* y, char* ws, hipStream_t stream) {
    switch (c.tile) {
        case Tile::N16: return launch_t<QT, 64, 16, 4, 1, kDepthN16>(s, c, l, w, x, y, ws, stream);
        case Tile::N32: return launch_t<QT, 64, 32, 4, 1, kDepthN32>(s, c, l, w, x, y, ws, stream);
        case Tile::N64: return launch_t<QT, 64, 64, 4, 1, kDepthN64>(s, c, l, w, x, y, ws, stream);
        default: return launch_t<QT, 128, 64, 2, 2, kDepthWide>(s, c, l, w, x, y, ws, stream);
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
    snprintf(buf, sizeof buf, "gemm_tile_%s_bm%d_bn%d_splitk%d", fmt, c.bm, c.bn, c.splits);
    return buf;
}

}  // namespace mlq

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
//     x' (Q4_1 offset term).  Token-major ([token][block][64 halves]): each
//     workgroup of the split writes one contiguous row, and a GEMM chunk reads
//     a token's four blocks as 512 contiguous bytes (against block-major
//     storage: 4096 x 4096 Q4_0 at 512 tokens 68.3 -> 66.8 us per call).
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
#include "xsplit_device.h"

#include <hip/hip_runtime.h>

#include <algorithm>
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
// The first kXsCache of them stay in registers between the two passes (the
// max|x| of the row, then the scaled split), so rows up to 16 384 elements are
// read once; longer rows re-read the rest (L2 hits).  The split itself is
// xsplit_device.h's, which kernels producing a GEMM input also use.
template <int QT>
__global__ __launch_bounds__(256) void xsplit_kernel(const float* __restrict__ x, int N, int K,
                                                     int nb, int npad, _Float16* __restrict__ xs,
                                                     float* __restrict__ bsum,
                                                     float* __restrict__ scale) {
    (void)npad;
    const int n = blockIdx.x;
    const bool valid = n < N;
    const float* xr = x + static_cast<size_t>(valid ? n : 0) * K;
    __shared__ float red[4];
    const int nhb = 2 * nb;

    auto load16 = [&](int hb, float (&v)[16]) {
        const int k0 = hb * 16;
        if (!valid || hb >= nhb) {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = 0.0f;
        } else if (k0 + 16 <= K && (reinterpret_cast<uintptr_t>(xr + k0) & 15u) == 0) {
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
            for (int i = 0; i < 16; ++i) v[i] = (k0 + i < K) ? xr[k0 + i] : 0.0f;
        }
    };

    float cache[kXsCache][16];
#pragma unroll
    for (int c = 0; c < kXsCache; ++c) load16(threadIdx.x + 256 * c, cache[c]);
    if (nhb <= 256 * kXsCache) {
        xsplit_emit_row<QT, kXsCache>(n, nb, cache, xs, bsum, scale, red);
        return;
    }
    float mx = 0.0f;
#pragma unroll
    for (int c = 0; c < kXsCache; ++c)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(cache[c][i]));
    for (int hb = threadIdx.x + 256 * kXsCache; hb < nhb; hb += 256) {
        float v[16];
        load16(hb, v);
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(v[i]));
    }
    mx = xsplit_row_max(mx, red);
    float inv, sc;
    xsplit_scale(mx, inv, sc);
    if (threadIdx.x == 0) scale[n] = sc;
    const int iters = (nhb + 255) / 256;  // uniform across the workgroup
#pragma unroll
    for (int c = 0; c < kXsCache; ++c) xsplit_emit_half<QT>(n, nb, threadIdx.x + 256 * c, cache[c], inv, xs, bsum);
    for (int it = kXsCache; it < iters; ++it) {
        float v[16];
        const int hb = threadIdx.x + 256 * it;
        load16(hb, v);
        xsplit_emit_half<QT>(n, nb, hb, v, inv, xs, bsum);
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

// Streaming MFMA kernel.  A workgroup of four waves owns BM = 64 * RT weight
// rows x BN = 16 * TT tokens and the pairs [p0, p1) of K.  Wave w owns rows
// [16 * RT * w, 16 * RT * (w + 1)) of the tile and reads their weight pairs
// straight from global memory into registers in fragment layout (nobody else
// needs them); the x fragments of a pair (2 blocks x BN tokens x 32 hi + 32 lo
// halves) are shared by the four waves, so the workgroup copies them into LDS,
// double-buffered, one barrier per pair.  Both are requested one pair ahead;
// latency is hidden by several workgroups per CU.  Per block each wave decodes
// RT weight fragments and issues 2 * RT * TT MFMAs (x hi, x lo).
constexpr int kGemmThreads = 256;
constexpr int kGemmMaxTiles = 65536;  // split-K arrival counters in the workspace
constexpr int kXRowHalves = 72;       // 64 halves of one token's block + 8 of padding (bank spread)

template <int TT>
struct StreamLds {
    static constexpr int BN = 16 * TT;
    static constexpr int x_halves = 2 * BN * kXRowHalves;  // [block h][token][72]
    static constexpr int stage_bytes = x_halves * 2 + 2 * BN * 4;  // + Q4_1 block sums [h][token]
    static constexpr int bytes = 2 * stage_bytes;
};

template <int QT, int RT, int TT, int D>
__global__ __launch_bounds__(kGemmThreads) void gemm_stream_kernel(
    const uint8_t* __restrict__ W, const _Float16* __restrict__ xs, const float* __restrict__ bsum,
    const float* __restrict__ scale, float* __restrict__ y, float* __restrict__ part,
    unsigned* __restrict__ tile_count, int M, int N, int npad, int nb, int pairs_per_split) {
    using L = StreamLds<TT>;
    constexpr int DW = GFmt<QT>::DW;
    constexpr int BM = 64 * RT;
    constexpr int BN = 16 * TT;
    constexpr int XC = (16 * BN) / kGemmThreads;  // 16-byte x chunks per thread per pair
    static_assert((16 * BN) % kGemmThreads == 0, "x chunks must divide evenly");
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i16 = lane & 15;
    const int g = lane >> 4;
    const int m_base = blockIdx.x * BM;
    const int n_base = blockIdx.y * BN;
    const int np = nb >> 1;
    const int p0 = blockIdx.z * pairs_per_split;
    const int p1 = min(np, p0 + pairs_per_split);

    uint32_t mask = 0x000F000Fu, magic = 0x64006400u;
    asm volatile("" : "+v"(mask), "+v"(magic));

    // Weight rows of this lane (rows past M re-read row M-1; results dropped).
    const uint32_t* wrow[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int m = min(m_base + (wave * RT + r) * 16 + i16, M - 1);
        wrow[r] = reinterpret_cast<const uint32_t*>(W) + static_cast<size_t>(m) * np * DW;
    }
    // x chunks this thread copies: global offset = p * xstride + xoff[j],
    // LDS offset = loff[j] (both in halves).
    constexpr size_t xstride = 2 * 64;  // a pair's two blocks, token-major split x
    size_t xoff[XC];
    int loff[XC];
#pragma unroll
    for (int j = 0; j < XC; ++j) {
        const int c = threadIdx.x + j * kGemmThreads;  // [h][token][chunk of 8]
        const int h = c / (8 * BN);
        const int rem = c % (8 * BN);
        const int t = rem >> 3;
        const int q = rem & 7;
        xoff[j] = (static_cast<size_t>(n_base + t) * nb + h) * 64 + 8 * q;
        loff[j] = (h * BN + t) * kXRowHalves + 8 * q;
    }
    const bool sum_lane = QT == 3 && threadIdx.x < 2 * BN;
    const size_t soff = QT == 3 ? static_cast<size_t>(n_base + threadIdx.x % BN) * nb + threadIdx.x / BN : 0;

    f32x4 acc[RT][TT];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[r][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const f32x4 zero{0.0f, 0.0f, 0.0f, 0.0f};

    // Load pipeline, D pairs deep: register set d holds pair q = q0 + d (weights
    // in fragment layout, x chunks).  Step q: x chunks of set d -> LDS buffer
    // q & 1; barrier; compute pair q (weights of set d, x from LDS); request
    // pair q + D into set d.  The buffer written at step q was last read at step
    // q - 2, before the barrier of step q - 1.  Requests past the split's last
    // pair re-read that pair, so every load is unconditional.
    uint32_t wr[D][RT][7];
    u32x4 xr[D][XC];
    float sr[D];
    auto request = [&](int p, uint32_t (&w)[RT][7], u32x4 (&x)[XC], float& sv) {
#pragma unroll
        for (int r = 0; r < RT; ++r) load_pair<QT>(wrow[r] + static_cast<size_t>(p) * DW, g, w[r]);
#pragma unroll
        for (int j = 0; j < XC; ++j) x[j] = *reinterpret_cast<const u32x4*>(xs + p * xstride + xoff[j]);
        if (QT == 3) sv = bsum[static_cast<size_t>(2 * p) + soff];
    };
    const int plast = max(p0, p1 - 1);
#pragma unroll
    for (int d = 0; d < D; ++d) request(min(p0 + d, plast), wr[d], xr[d], sr[d]);

    auto step = [&](int q, uint32_t (&wrd)[RT][7], u32x4 (&xrd)[XC], float& srd) {
            char* cur = smem + ((q - p0) & 1) * L::stage_bytes;
        {
            _Float16* xl = reinterpret_cast<_Float16*>(cur);
#pragma unroll
            for (int j = 0; j < XC; ++j) *reinterpret_cast<u32x4*>(xl + loff[j]) = xrd[j];
            if (sum_lane) reinterpret_cast<float*>(cur + L::x_halves * 2)[threadIdx.x] = srd;
        }
        __syncthreads();
        const _Float16* xl = reinterpret_cast<const _Float16*>(cur);
        const float* sl = reinterpret_cast<const float*>(cur + L::x_halves * 2);
        // Per block: all x fragments, all weight fragments, then every MFMA of
        // the block (independent accumulator tiles, so they pipeline), then
        // the scale epilogue.
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            f16x8 ahi[TT], alo[TT];
            f32x4 sv[TT];
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const _Float16* src = xl + (h * BN + t * 16 + i16) * kXRowHalves + 8 * g;
                ahi[t] = *reinterpret_cast<const f16x8*>(src);
                alo[t] = *reinterpret_cast<const f16x8*>(src + 32);
                if (QT == 3) sv[t] = *reinterpret_cast<const f32x4*>(sl + h * BN + t * 16 + 4 * g);
            }
            WFrag f[RT];
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                WFrag f0, f1;
                decode_pair<QT>(wrd[r], f0, f1, mask, magic);
                f[r] = h ? f1 : f0;
            }
            f32x4 blk[RT][TT];
#pragma unroll
            for (int r = 0; r < RT; ++r)
#pragma unroll
                for (int t = 0; t < TT; ++t) blk[r][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[t], f[r].b, zero, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < RT; ++r)
#pragma unroll
                for (int t = 0; t < TT; ++t)
                    blk[r][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[t], f[r].b, blk[r][t], 0, 0, 0);
#pragma unroll
            for (int r = 0; r < RT; ++r)
#pragma unroll
                for (int t = 0; t < TT; ++t)
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) {
                        acc[r][t][qq] = __builtin_fmaf(f[r].d, blk[r][t][qq], acc[r][t][qq]);
                        if (QT == 3) acc[r][t][qq] = __builtin_fmaf(f[r].m, sv[t][qq], acc[r][t][qq]);
                    }
        }
        request(min(q + D, plast), wrd, xrd, srd);
    };
    // Full groups of D pairs without branches (so the compiler counts the
    // in-flight loads exactly), then the remaining pairs.
    int q0 = p0;
    for (; q0 + D <= p1; q0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) step(q0 + d, wr[d], xr[d], sr[d]);
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (q0 + d < p1) step(q0 + d, wr[d], xr[d], sr[d]);
    }
    __syncthreads();

    if (part == nullptr) {
#pragma unroll
        for (int t = 0; t < TT; ++t) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n_base + t * 16 + 4 * g + q;
                if (n >= N) continue;
                const float sn = scale[n];
#pragma unroll
                for (int r = 0; r < RT; ++r) {
                    const int m = m_base + (wave * RT + r) * 16 + i16;
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
            const int n = n_base + t * 16 + 4 * g + q;
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const int m = m_base + (wave * RT + r) * 16 + i16;
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
    // Every thread sums its tile elements over the splits in split order, eight
    // elements at a time with the loads of four splits in flight (each load is
    // a round trip to the point of coherence).
    constexpr int E = (BM * BN) / kGemmThreads;
    constexpr int EC = E < 8 ? E : 8;
    static_assert((BM * BN) % kGemmThreads == 0 && E % EC == 0, "tile must divide the workgroup");
    const size_t zstride = static_cast<size_t>(npad) * M;
    const unsigned S = gridDim.z;
    for (int i0 = 0; i0 < E; i0 += EC) {
        float sum[EC];
        size_t off[EC];
#pragma unroll
        for (int i = 0; i < EC; ++i) {
            const int e = threadIdx.x + (i0 + i) * kGemmThreads;
            const int n = min(n_base + e / BM, N - 1);  // clamped; out-of-range results are not stored
            const int m = min(m_base + e % BM, M - 1);
            off[i] = static_cast<size_t>(n) * M + m;
            sum[i] = 0.0f;
        }
        unsigned k = 0;
        for (; k + 4 <= S; k += 4) {
            float v[4][EC];
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int i = 0; i < EC; ++i)
                    v[u][i] = __hip_atomic_load(part + (k + u) * zstride + off[i], __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int i = 0; i < EC; ++i) sum[i] += v[u][i];
        }
        for (; k < S; ++k) {
#pragma unroll
            for (int i = 0; i < EC; ++i)
                sum[i] += __hip_atomic_load(part + k * zstride + off[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int i = 0; i < EC; ++i) {
            const int e = threadIdx.x + (i0 + i) * kGemmThreads;
            const int n = n_base + e / BM;
            const int m = m_base + e % BM;
            if (n < N && m < M) y[static_cast<size_t>(n) * M + m] = sum[i] * scale[n];
        }
    }
    if (threadIdx.x == 0) __hip_atomic_store(tile_count + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Chunked MFMA kernel.
//
// A workgroup of four waves owns BM = 64 * RW weight rows x BN = 16 * TT
// tokens and a contiguous range of K chunks (4 blocks = 128 k each); the grid
// is about one wave of workgroups (two per CU), so each workgroup streams a
// long run of chunks through a pipeline instead of paying a memory latency per
// step.  Per chunk:
//  * weights: each wave reads its own rows' chunk (RW * 16 rows x 4 blocks)
//    with coalesced 8-byte loads, P chunks ahead, into registers, and parks it
//    in a wave-private LDS buffer; MFMA B fragments are read back from there.
//  * x, one chunk ahead, into a shared LDS buffer of A fragments (slot order
//    of the weight codes), from one of two sources:
//    XS: the x split by xsplit_kernel (per-token power-of-two scale, fp16 hi +
//        lo in fragment order, Q4_1 block sums): a plain copy;
//    !XS: the f32 x itself (small batches, where a second launch would cost
//        more than the split): the workgroup picks a power-of-two scale per
//        (token, chunk) that puts the chunk's max|x| in [2^13, 2^14) and
//        splits every scaled element into fp16 hi + lo.
//  * MFMAs: per block, hi then lo into a zeroed tile, then the block scale
//    d (+ m * sum(x') for Q4_1) times the tile into the accumulator (!XS: into
//    a chunk accumulator that is scaled back by the chunk's inverse scale).
// K is split across workgroups only when the tiles alone would not fill the
// CUs; the splits of a tile are adjacent in launch order.  Each split stores
// its partial tile with write-through stores and counts in; the workgroup
// that completes the count adds the partials in split order (deterministic),
// applies the token scale and writes y.  Needs nb % 4 == 0 (8-byte aligned
// chunk rows), K == 32 nb and (!XS) a 16-byte aligned x.
constexpr int kChunkBlocks = 4;

template <int QT> struct ChunkFmt;
template <> struct ChunkFmt<1> { static constexpr int BB = 34, U = 17, WROW = 136; };  // U: 8-byte units per row
template <> struct ChunkFmt<2> { static constexpr int BB = 18, U = 9, WROW = 72; };
template <> struct ChunkFmt<3> { static constexpr int BB = 20, U = 10, WROW = 80; };

template <int QT, int RW, int TT, bool XS>
struct ChunkLds {
    static constexpr int BN = 16 * TT;
    static constexpr int w_wave = RW * 16 * ChunkFmt<QT>::WROW;  // one buffer of one wave
    static constexpr int w_bytes = 2 * 4 * w_wave;                 // [buffer][wave][row][WROW]
    static constexpr int x_halves = kChunkBlocks * BN * kXRowHalves;  // [block][token][72]
    // + (!XS) inverse scales [BN] + (Q4_1) block sums [block][BN]
    static constexpr int sums_off = x_halves * 2 + (XS ? 0 : BN * 4);
    static constexpr int x_buf = sums_off + (QT == 3 ? kChunkBlocks * BN * 4 : 0);
    static constexpr int bytes = w_bytes + 2 * x_buf;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                             0x00020000);
}
constexpr int kCoherent = 16;  // sc1: write through / read from the point of coherence (agent scope)

struct ChunkArgs {
    const uint8_t* W;
    const float* x;         // !XS: f32 x [N][K]
    const _Float16* xs;     // XS: split x [npad][nb][64] (token-major)
    const float* bsum;      // XS, Q4_1: [npad][nb]
    const float* xscale;    // XS: [npad]
    float* y;
    float* part;
    uint32_t part_bytes;
    unsigned* tile_count;
    int M, N, K, nb, npad, row_tiles, splits, chunks_per_split;
    // Grouped call (up to three weights reading the same x, e.g. q / k / v):
    // weight g owns row tiles [tile_g, tile_{g+1}) with tile_0 = 0 and writes
    // its own y [N][M_g]; W / y / M above are group 0.  A single weight has
    // tile1 = tile2 = row_tiles.
    const uint8_t* W1;
    const uint8_t* W2;
    float* y1;
    float* y2;
    int M1, M2, tile1, tile2;
    // XCD-blocked tile order (one K split, grid a multiple of 8; xcd_br = 0: off):
    // workgroup i runs on XCD i % 8, which owns the block of xcd_br-th of the row
    // tiles x (8 / xcd_br)-th of the token tiles; inside it the row tiles vary
    // fastest (token tiles if xcd_row_outer), so the block's x (or its weights)
    // stays in that XCD's L2 while the other operand streams.
    int xcd_br, xcd_row_outer;
};

template <int QT, int RW, int TT, int P, bool XS>
__global__ __launch_bounds__(kGemmThreads) void gemm_chunk_kernel(const ChunkArgs a) {
    using L = ChunkLds<QT, RW, TT, XS>;
    using F = ChunkFmt<QT>;
    constexpr int BN = L::BN;
    constexpr int TPT = kGemmThreads / BN;  // !XS: x-split threads per token
    constexpr int EPT = 128 / TPT;          // !XS: elements per thread per chunk (8, 16 or 32)
    constexpr int XU = kChunkBlocks * BN * 8 / kGemmThreads;  // XS: 16-byte x units per thread per chunk
    constexpr int XR = XS ? XU : EPT / 4;   // x registers (float4 / 16-byte units) per thread
    constexpr int WU = RW * 16 * F::U;      // weight units per wave per chunk
    constexpr int NWL = (WU + 63) / 64;     // weight loads per lane per chunk
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i16 = lane & 15;
    const int g = lane >> 4;
    const int wg = blockIdx.x;
    const int split = wg % a.splits;
    int tile = wg / a.splits;
    if (a.xcd_br > 0) {
        const int tok_tiles = a.npad / BN;
        const int bt_n = 8 / a.xcd_br;
        const int rows_b = a.row_tiles / a.xcd_br, toks_b = tok_tiles / bt_n;
        const int xcd = wg % 8, j = wg / 8;
        const int rl = a.xcd_row_outer ? j / toks_b : j % rows_b;
        const int tl = a.xcd_row_outer ? j % toks_b : j / rows_b;
        tile = ((xcd % bt_n) * toks_b + tl) * a.row_tiles + (xcd / bt_n) * rows_b + rl;
    }
    const int rt = tile % a.row_tiles;
    const int gi = (rt >= a.tile1 ? 1 : 0) + (rt >= a.tile2 ? 1 : 0);  // this tile's weight of the group
    const uint8_t* const Wg = gi == 0 ? a.W : gi == 1 ? a.W1 : a.W2;
    float* const yg = gi == 0 ? a.y : gi == 1 ? a.y1 : a.y2;
    const int m_base = (rt - (gi == 0 ? 0 : gi == 1 ? a.tile1 : a.tile2)) * (64 * RW);
    const int n_base = (tile / a.row_tiles) * BN;
    const int M = gi == 0 ? a.M : gi == 1 ? a.M1 : a.M2, N = a.N, nb = a.nb;
    const int nchunk_all = nb / kChunkBlocks;
    const int c0 = split * a.chunks_per_split;
    const int nchunk = min(nchunk_all, c0 + a.chunks_per_split) - c0;

    uint32_t mask = 0x000F000Fu, magic = 0x64006400u;
    asm volatile("" : "+v"(mask), "+v"(magic));

    // Weight units of this lane: unit u = lane + 64 i -> (row u / U, 8-byte
    // column u % U); 32-bit offsets from the split's first chunk (the host
    // keeps a weight below 4 GiB on this path).  Loads are unconditional
    // (lanes past the wave's units re-read its last unit, tokens past N read
    // token 0 and are zeroed) so that no branch forces an early wait; only
    // the LDS store is predicated.
    const uint8_t* wsplit = Wg + static_cast<size_t>(c0) * kChunkBlocks * F::BB;
    uint32_t goff[NWL];
    int loff[NWL];
#pragma unroll
    for (int i = 0; i < NWL; ++i) {
        const int u = min(lane + 64 * i, WU - 1);
        const int rl = u / F::U;
        const int col = u % F::U;
        const int row = min(m_base + wave * RW * 16 + rl, M - 1);
        goff[i] = static_cast<uint32_t>(row) * static_cast<uint32_t>(nb * F::BB) + col * 8;
        loff[i] = rl * F::WROW + col * 8;
    }
    const bool last_ok = lane + 64 * (NWL - 1) < WU;  // the last load is partial when 64 does not divide WU
    constexpr size_t kChunkBytes = static_cast<size_t>(kChunkBlocks) * F::BB;

    // !XS: x slice of this thread: token tok, elements e0 .. e0 + EPT - 1 of the chunk.
    const int tok = tid / TPT;
    const int e0 = (tid % TPT) * EPT;
    const bool tok_ok = n_base + tok < N;
    const float* xrow = XS ? nullptr
                           : a.x + static_cast<size_t>(tok_ok ? n_base + tok : 0) * a.K +
                                 static_cast<size_t>(c0) * 128 + e0;
    // XS: unit v = tid + 256 i -> (token, block j, 16-byte column q) of the
    // chunk: a token's four blocks are 512 contiguous bytes of the split x.
    uint32_t xoff[XS ? XU : 1];
    int xl_off[XS ? XU : 1];
    if (XS) {
#pragma unroll
        for (int i = 0; i < XU; ++i) {
            const int v = tid + kGemmThreads * i;
            const int q = v % 8;
            const int j = (v / 8) % kChunkBlocks;
            const int tk = v / (8 * kChunkBlocks);
            xoff[i] = (static_cast<uint32_t>(n_base + tk) * a.nb + j) * 64 + 8 * q;  // halves, from the chunk's block 0
            xl_off[i] = ((j * BN + tk) * kXRowHalves + 8 * q) * 2;                      // bytes
        }
    }
    const bool sum_lane = XS && QT == 3 && tid < kChunkBlocks * BN;

    uint2 wreg[P][NWL];
    u32x4 xreg[XR];
    float sreg = 0.0f;
    auto load_w = [&](int c, uint2 (&wr)[NWL]) {
        const uint8_t* wc = wsplit + static_cast<size_t>(c) * kChunkBytes;
#pragma unroll
        for (int i = 0; i < NWL; ++i) wr[i] = *reinterpret_cast<const uint2*>(wc + goff[i]);
    };
    auto store_w = [&](const uint2 (&wr)[NWL], int buf) {
        char* base = smem + (buf * 4 + wave) * L::w_wave;
#pragma unroll
        for (int i = 0; i < NWL; ++i) {
            if (i < NWL - 1 || last_ok) *reinterpret_cast<uint2*>(base + loff[i]) = wr[i];
        }
    };
    auto load_x = [&](int c) {
        if (XS) {
            const int b = (c0 + c) * kChunkBlocks;
            const _Float16* src = a.xs + static_cast<size_t>(b) * 64;
#pragma unroll
            for (int i = 0; i < XU; ++i) xreg[i] = *reinterpret_cast<const u32x4*>(src + xoff[i]);
            if (QT == 3) {
                const int t = sum_lane ? tid : 0;
                sreg = a.bsum[static_cast<size_t>(n_base + t % BN) * a.nb + b + t / BN];
            }
        } else {
            const u32x4* src = reinterpret_cast<const u32x4*>(xrow + static_cast<size_t>(c) * 128);
#pragma unroll
            for (int i = 0; i < XR; ++i) xreg[i] = src[i];
        }
    };
    auto put_x = [&](int buf) {
        char* xb = smem + L::w_bytes + buf * L::x_buf;
        if (XS) {
#pragma unroll
            for (int i = 0; i < XU; ++i) *reinterpret_cast<u32x4*>(xb + xl_off[i]) = xreg[i];
            if (sum_lane) reinterpret_cast<float*>(xb + L::sums_off)[tid] = sreg;
            return;
        }
        _Float16* xl = reinterpret_cast<_Float16*>(xb);
        float* sl = reinterpret_cast<float*>(xb + L::x_halves * 2);
        float v[EPT];
#pragma unroll
        for (int i = 0; i < XR; ++i) {
            const f32x4 f = __builtin_bit_cast(f32x4, xreg[i]);
#pragma unroll
            for (int k = 0; k < 4; ++k) v[4 * i + k] = tok_ok ? f[k] : 0.0f;
        }
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < EPT; ++i) mx = fmaxf(mx, fabsf(v[i]));
#pragma unroll
        for (int o = 1; o < TPT; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        float inv = 1.0f, sinv = 1.0f;
        if (mx > 0.0f && mx <= 3.0e38f) {
            int ex = 0;
            (void)frexpf(mx, &ex);  // mx in [2^(ex-1), 2^ex)
            const int e = min(126, max(-126, 14 - ex));
            inv = ldexpf(1.0f, e);
            sinv = ldexpf(1.0f, -e);
        }
        if (tid % TPT == 0) sl[tok] = sinv;
#pragma unroll
        for (int i = 0; i < EPT; ++i) v[i] *= inv;
        const int j = e0 >> 5;  // block within the chunk
        const int o = e0 & 31;  // first element within the block
        if (QT == 3) {
            float sum = 0.0f;
#pragma unroll
            for (int q = 0; q < EPT / 4; ++q) sum += (v[4 * q] + v[4 * q + 1]) + (v[4 * q + 2] + v[4 * q + 3]);
#pragma unroll
            for (int w = 1; w < 32 / EPT; w <<= 1) sum += __shfl_xor(sum, w, 64);
            if (o == 0) reinterpret_cast<float*>(xb + L::sums_off)[j * BN + tok] = sum;
        }
        _Float16* row = xl + (j * BN + tok) * kXRowHalves;
        typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int q = 0; q < EPT / 4; ++q) {
            const int e = o + 4 * q;
            float a0, a1, a2, a3;
            int slot;
            if (QT == 1) {
                slot = e;
                a0 = v[4 * q], a1 = v[4 * q + 1], a2 = v[4 * q + 2], a3 = v[4 * q + 3];
            } else {
                slot = 8 * ((e & 15) >> 2) + 4 * (e >> 4);
                a0 = v[4 * q], a1 = v[4 * q + 2], a2 = v[4 * q + 1], a3 = v[4 * q + 3];
            }
            const _Float16 h0 = static_cast<_Float16>(a0), h1 = static_cast<_Float16>(a1);
            const _Float16 h2 = static_cast<_Float16>(a2), h3 = static_cast<_Float16>(a3);
            *reinterpret_cast<f16x4*>(row + slot) = f16x4{h0, h1, h2, h3};
            *reinterpret_cast<f16x4*>(row + 32 + slot) =
                f16x4{static_cast<_Float16>(a0 - static_cast<float>(h0)), static_cast<_Float16>(a1 - static_cast<float>(h1)),
                      static_cast<_Float16>(a2 - static_cast<float>(h2)), static_cast<_Float16>(a3 - static_cast<float>(h3))};
        }
    };

    f32x4 acc[RW][TT];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[r][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const f32x4 zero{0.0f, 0.0f, 0.0f, 0.0f};

    // Per block: all RW x TT tiles get their two MFMAs (hi, lo) from zero;
    // the scale epilogue of a block runs while the next block's MFMAs are in
    // flight, so no VALU op waits on a fresh MFMA result.
    auto compute = [&](int buf) {
        const char* wb = smem + (buf * 4 + wave) * L::w_wave;
        const char* xb = smem + L::w_bytes + buf * L::x_buf;
        const _Float16* xl = reinterpret_cast<const _Float16*>(xb);
        const float* ssum = reinterpret_cast<const float*>(xb + L::sums_off);
        f32x4 cacc[XS ? 1 : RW][XS ? 1 : TT];
        f32x4 bprev[RW][TT];
        float dprev[RW], mprev[RW];
        f32x4 svprev[TT];
        auto epilogue = [&](int jb) {
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int t = 0; t < TT; ++t)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if (XS) {
                            float v = __builtin_fmaf(dprev[r], bprev[r][t][q], acc[r][t][q]);
                            if (QT == 3) v = __builtin_fmaf(mprev[r], svprev[t][q], v);
                            acc[r][t][q] = v;
                        } else {
                            float v = jb == 0 ? dprev[r] * bprev[r][t][q]
                                              : __builtin_fmaf(dprev[r], bprev[r][t][q], cacc[r][t][q]);
                            if (QT == 3) v = __builtin_fmaf(mprev[r], svprev[t][q], v);
                            cacc[r][t][q] = v;
                        }
                    }
        };
#pragma unroll
        for (int p = 0; p < kChunkBlocks / 2; ++p) {
            uint32_t wr[RW][7];
#pragma unroll
            for (int r = 0; r < RW; ++r)
                load_pair<QT>(reinterpret_cast<const uint32_t*>(wb + (r * 16 + i16) * F::WROW + p * 2 * F::BB), g, wr[r]);
            WFrag f0[RW], f1[RW];
#pragma unroll
            for (int r = 0; r < RW; ++r) decode_pair<QT>(wr[r], f0[r], f1[r], mask, magic);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int j = 2 * p + h;
                f16x8 ahi[TT], alo[TT];
                f32x4 sv[TT];
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    const _Float16* src = xl + (j * BN + t * 16 + i16) * kXRowHalves + 8 * g;
                    ahi[t] = *reinterpret_cast<const f16x8*>(src);
                    alo[t] = *reinterpret_cast<const f16x8*>(src + 32);
                    if (QT == 3) sv[t] = *reinterpret_cast<const f32x4*>(ssum + j * BN + t * 16 + 4 * g);
                }
                f32x4 bcur[RW][TT];
#pragma unroll
                for (int r = 0; r < RW; ++r)
#pragma unroll
                    for (int t = 0; t < TT; ++t)
                        bcur[r][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[t], (h ? f1[r] : f0[r]).b, zero, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < RW; ++r)
#pragma unroll
                    for (int t = 0; t < TT; ++t)
                        bcur[r][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[t], (h ? f1[r] : f0[r]).b, bcur[r][t], 0, 0, 0);
                if (j > 0) epilogue(j - 1);
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    const WFrag& f = h ? f1[r] : f0[r];
                    dprev[r] = f.d;
                    mprev[r] = f.m;
#pragma unroll
                    for (int t = 0; t < TT; ++t) bprev[r][t] = bcur[r][t];
                }
#pragma unroll
                for (int t = 0; t < TT; ++t) svprev[t] = sv[t];
            }
        }
        epilogue(kChunkBlocks - 1);
        if (!XS) {
            const float* sl = reinterpret_cast<const float*>(xb + L::x_halves * 2);
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const f32x4 s4 = *reinterpret_cast<const f32x4*>(sl + t * 16 + 4 * g);
#pragma unroll
                for (int r = 0; r < RW; ++r)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        acc[r][t][q] = __builtin_fmaf(s4[q], cacc[XS ? 0 : r][XS ? 0 : t][q], acc[r][t][q]);
            }
        }
    };

    // Pipeline.  Register set k % P holds weight chunk k; at step c the set of
    // chunk c + 1 goes to LDS buffer (c + 1) & 1 and is refilled with chunk
    // c + 1 + P; x chunk c + 1 (loaded one step earlier) goes to its buffer
    // and chunk c + 2 is requested; then chunk c is computed.  The barrier at
    // the end of step c publishes buffer (c + 1) & 1 and frees buffer c & 1.
    // Memory counters drain in issue order, so each step requests x (needed
    // next step) before the weights (needed P steps later), with a scheduling
    // barrier between them: waiting for x then leaves the weight prefetch in
    // flight.  Requests past the last chunk re-read the last chunk (L2 hits),
    // so that every load is unconditional and can be counted exactly.
    const int clast = nchunk - 1;
    // x first: every wave requests the first x chunk before any wave requests
    // weights (a bare barrier, no memory wait), so the CU's memory queue serves
    // x ahead of the weight misses and x is split while the weights arrive
    // (4096 x 4096 Q4_0: N = 16 13.0 -> 12.0 us, N = 64 20.4 -> 19.9 us).
    load_x(0);
    __builtin_amdgcn_s_barrier();
    load_w(0, wreg[0]);
#pragma unroll
    for (int k = 1; k < P; ++k) load_w(min(k, clast), wreg[k]);
    put_x(0);
    load_x(min(1, clast));
    store_w(wreg[0], 0);
    __builtin_amdgcn_sched_barrier(0);
    load_w(min(P, clast), wreg[0]);
    __syncthreads();
    // Full groups of P steps without branches, then the last steps, which
    // request nothing new except x.
    int cb = 0;
    for (; cb + P < nchunk; cb += P) {
#pragma unroll
        for (int u = 0; u < P; ++u) {
            const int c = cb + u;
            store_w(wreg[(u + 1) % P], (c + 1) & 1);
            put_x((c + 1) & 1);
            load_x(min(c + 2, clast));
            __builtin_amdgcn_sched_barrier(0);
            load_w(min(c + 1 + P, clast), wreg[(u + 1) % P]);
            compute(c & 1);
            __syncthreads();
        }
    }
#pragma unroll
    for (int u = 0; u < P; ++u) {
        const int c = cb + u;
        if (c < nchunk) {
            if (c + 1 < nchunk) {
                store_w(wreg[(u + 1) % P], (c + 1) & 1);
                put_x((c + 1) & 1);
                if (c + 2 < nchunk) load_x(c + 2);
            }
            compute(c & 1);
            __syncthreads();
        }
    }

    // Token scale of output element q of token tile t (XS: the x split's
    // per-token scale; !XS: already applied per chunk).
    auto tok_scale = [&](int t, int q) {
        if (!XS) return 1.0f;
        return a.xscale[n_base + t * 16 + 4 * g + q];
    };
    if (a.splits == 1) {
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n_base + t * 16 + 4 * g + q;
                if (n >= N) continue;
                const float sn = tok_scale(t, q);
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    const int m = m_base + (wave * RW + r) * 16 + i16;
                    if (m < M) yg[static_cast<size_t>(n) * M + m] = acc[r][t][q] * sn;
                }
            }
        return;
    }

    // Split K: partial tile [tile][split][r][t][thread] as float4, write-through.
    const __amdgpu_buffer_rsrc_t prs = make_rsrc(a.part, a.part_bytes);
    const uint32_t tile_base = static_cast<uint32_t>(tile) * a.splits * (RW * TT * kGemmThreads * 16);
    constexpr uint32_t split_stride = RW * TT * kGemmThreads * 16;
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t)
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(u32x4, acc[r][t]), prs,
                tile_base + split * split_stride + ((r * TT + t) * kGemmThreads + tid) * 16, 0, kCoherent);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __shared__ unsigned last;
    __syncthreads();
    if (tid == 0) {
        const unsigned done = __hip_atomic_fetch_add(a.tile_count + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = done == static_cast<unsigned>(a.splits) - 1 ? 1u : 0u;
    }
    __syncthreads();
    if (last == 0u) return;
    // Sum the splits in order: every (r, t) tile of up to kBatch splits is
    // requested before any is added, so the sum costs about one round trip
    // to the point of coherence per batch.
    constexpr int RT4 = RW * TT;
    constexpr int kBatch = RT4 <= 2 ? 16 : RT4 <= 4 ? 8 : 4;
    f32x4 sum[RT4];
#pragma unroll
    for (int k = 0; k < RT4; ++k) sum[k] = zero;
    for (int s0 = 0; s0 < a.splits; s0 += kBatch) {
        f32x4 v[kBatch][RT4];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int s = min(s0 + b, a.splits - 1);
#pragma unroll
            for (int k = 0; k < RT4; ++k)
                v[b][k] = __builtin_bit_cast(
                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                               prs, tile_base + s * split_stride + (k * kGemmThreads + tid) * 16, 0, kCoherent));
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b)
            if (s0 + b < a.splits) {
#pragma unroll
                for (int k = 0; k < RT4; ++k) sum[k] += v[b][k];
            }
    }
#pragma unroll
    for (int k = 0; k < RT4; ++k) {
        const int r = k / TT;
        const int t = k % TT;
        const int m = m_base + (wave * RW + r) * 16 + i16;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n = n_base + t * 16 + 4 * g + q;
            if (n < N && m < M) yg[static_cast<size_t>(n) * M + m] = sum[k][q] * tok_scale(t, q);
        }
    }
    if (tid == 0) __hip_atomic_store(a.tile_count + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Configurations: rows per wave (RT) and token tiles (TT) by batch size.  K is
// split across workgroups until the grid gives every CU a few workgroups,
// keeping at least eight pairs per split.
struct GemmCfg {
    int rt, tt, bm, bn, splits, pairs_per_split, npad, lds;
};

GemmCfg choose(const LinearShape& s) {
    GemmCfg c;
    if (s.rows <= 16) {
        c.rt = 1, c.tt = 1;
    } else if (s.rows <= 32) {
        c.rt = 1, c.tt = 2;
    } else if (s.rows <= 64) {
        c.rt = 1, c.tt = 4;
    } else {
        c.rt = 2, c.tt = 4;
    }
    c.bm = 64 * c.rt;
    c.bn = 16 * c.tt;
    c.lds = c.tt == 1 ? StreamLds<1>::bytes : c.tt == 2 ? StreamLds<2>::bytes : StreamLds<4>::bytes;
    c.npad = (s.rows + c.bn - 1) / c.bn * c.bn;
    const int np = s.nb / 2;
    const long long tiles = static_cast<long long>((s.M + c.bm - 1) / c.bm) * (c.npad / c.bn);
    const long long target = c.rt == 1 ? 1024 : 512;
    int splits = static_cast<int>((target + tiles - 1) / tiles);
    splits = max(1, min(splits, np / 8));
    if (tiles > kGemmMaxTiles) splits = 1;
    c.pairs_per_split = (np + splits - 1) / splits;
    c.splits = (np + c.pairs_per_split - 1) / c.pairs_per_split;
    return c;
}

struct WsLayout {
    size_t count, xs, bsum, scale, part, total;
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

template <int QT, int RT, int TT>
hipError_t launch_t(const LinearShape& s, const GemmCfg& c, const WsLayout& l, const void* w,
                    const float* x, float* y, char* ws, hipStream_t stream) {
    _Float16* xs = reinterpret_cast<_Float16*>(ws + l.xs);
    float* bsum = reinterpret_cast<float*>(ws + l.bsum);
    float* scale = reinterpret_cast<float*>(ws + l.scale);
    float* part = c.splits > 1 ? reinterpret_cast<float*>(ws + l.part) : nullptr;
    unsigned* count = reinterpret_cast<unsigned*>(ws + l.count);
    hipLaunchKernelGGL((xsplit_kernel<QT>), dim3(c.npad), dim3(256), 0, stream, x, s.rows, s.K, s.nb,
                       c.npad, xs, bsum, scale);
    dim3 grid((s.M + 64 * RT - 1) / (64 * RT), c.npad / (16 * TT), c.splits);
    constexpr int lds = StreamLds<TT>::bytes;
    hipLaunchKernelGGL((gemm_stream_kernel<QT, RT, TT, (RT == 1 ? 4 : 2)>), grid, dim3(kGemmThreads), lds, stream,
                       static_cast<const uint8_t*>(w), xs, bsum, scale, y, part, count, s.M, s.rows, c.npad,
                       s.nb, c.pairs_per_split);
    return hipGetLastError();
}

template <int QT>
hipError_t launch_q(const LinearShape& s, const GemmCfg& c, const WsLayout& l, const void* w,
                    const float* x, float* y, char* ws, hipStream_t stream) {
    if (c.rt == 2) return launch_t<QT, 2, 4>(s, c, l, w, x, y, ws, stream);
    switch (c.tt) {
        case 1: return launch_t<QT, 1, 1>(s, c, l, w, x, y, ws, stream);
        case 2: return launch_t<QT, 1, 2>(s, c, l, w, x, y, ws, stream);
        default: return launch_t<QT, 1, 4>(s, c, l, w, x, y, ws, stream);
    }
}

// Chunked-kernel configuration (rules from an MI355X sweep of rows per wave,
// token tile, x split, prefetch depth and K splits at 4096x4096 and
// 11008x4096, Q4_0 and Q8_0, N = 16 / 64 / 512):
//  * up to 16 tokens: 64 rows (one row tile per wave) x 16 tokens per
//    workgroup, K split until the grid is about 640 workgroups with at least
//    4 chunks per split (fewer, longer splits beat a larger grid: the split
//    reduction is a serial tail; short rows keep 2 chunks per split);
//  * up to 128 tokens: 128 rows x 32 tokens, x split in the kernel;
//  * more tokens: x split once by xsplit_kernel (the in-kernel split would be
//    repeated by every row tile), 128 rows x 32 tokens, or x 64 tokens for
//    Q8_0 from 512 tokens (its 34-byte blocks gain most from fewer weight
//    passes there; at 256 tokens, and for Q4 throughout, the larger tile's
//    single workgroup per CU measured slower: 11008 x 4096 Q8_0 N = 256
//    124.2 against 110.4 us);
//  * from 32 tokens on, 8 chunks per split unless the tiles alone give every
//    CU a workgroup (then no K split; with x split once, two splits until
//    there are two workgroups per CU).
struct ChunkCfg {
    int rw, tt, row_tiles, tok_tiles, splits, cps, npad;
    bool xs;
};

bool chunk_supported(const LinearShape& s) {
    return s.rows > 1 && s.nb >= 8 && s.nb % kChunkBlocks == 0 && s.K == s.nb * kQK && s.qtype >= 1 && s.qtype <= 3;
}

ChunkCfg choose_chunk(const LinearShape& s) {
    ChunkCfg c;
    c.rw = s.rows <= 16 ? 1 : 2;
    c.tt = s.rows <= 16 ? 1 : (s.rows >= 512 && s.qtype == 1) ? 4 : 2;
    c.xs = s.rows > 128;
    c.row_tiles = (s.M + 64 * c.rw - 1) / (64 * c.rw);
    c.tok_tiles = (s.rows + 16 * c.tt - 1) / (16 * c.tt);
    c.npad = c.tok_tiles * 16 * c.tt;
    const long long tiles = static_cast<long long>(c.row_tiles) * c.tok_tiles;
    const int nchunks = s.nb / kChunkBlocks;
    int splits;
    if (c.tt == 1) {
        splits = static_cast<int>((640 + tiles - 1) / tiles);
        splits = std::min(splits, nchunks >= 16 ? nchunks / 4 : nchunks / 2);
    } else if (!c.xs) {
        splits = tiles >= 256 ? 1 : nchunks / 8;
    } else {
        // N = 256: two splits for 256 tiles (4096 x 4096 Q4_0: 45.2 -> 40.1 us)
        const bool fill = c.tt == 4 ? tiles >= 256 : tiles >= 512;
        splits = fill ? 1 : tiles >= 256 ? 2 : nchunks / 8;
    }
    splits = std::max(1, splits);
    if (tiles > kGemmMaxTiles) splits = 1;
    c.cps = (nchunks + splits - 1) / splits;
    c.splits = (nchunks + c.cps - 1) / c.cps;
    return c;
}

// Workspace: [split-K counters][split x][block sums][token scales][partials].
struct ChunkWs {
    size_t xs, bsum, scale, part, part_bytes, total;
};

ChunkWs chunk_layout(const LinearShape& s, const ChunkCfg& c) {
    auto up = [](size_t v) { return (v + 255) & ~static_cast<size_t>(255); };
    ChunkWs l;
    l.xs = up(static_cast<size_t>(kGemmMaxTiles) * sizeof(unsigned));
    l.bsum = l.xs + (c.xs ? up(static_cast<size_t>(s.nb) * c.npad * 64 * sizeof(_Float16)) : 0);
    l.scale = l.bsum + (c.xs ? up(static_cast<size_t>(s.nb) * c.npad * sizeof(float)) : 0);
    l.part = l.scale + (c.xs ? up(static_cast<size_t>(c.npad) * sizeof(float)) : 0);
    l.part_bytes = c.splits == 1 ? 0
                                 : static_cast<size_t>(c.row_tiles) * c.tok_tiles * c.splits *
                                       (c.rw * c.tt * kGemmThreads * 16);
    l.total = l.part + l.part_bytes;
    return l;
}

size_t chunk_workspace_bytes(const LinearShape& s) { return chunk_layout(s, choose_chunk(s)).total; }

// Two weight chunks in flight per wave at every tile shape: at 16 tokens, four
// (the earlier default) cost 2.5-15 % (4096 x 4096 Q4_0 12.1 -> 11.8 us,
// 11008 x 4096 Q8_0 26.6 -> 22.5 us): the ring's VGPRs halve the waves per SIMD,
// and the loop is not waiting on the weights.
// Weights of a grouped call: n <= 3 linears with the same qtype, K and rows.
struct ChunkGroup {
    int n;
    const void* w[3];
    float* y[3];
    int M[3];
};

template <int QT, int RW, int TT, bool XS, int P = 2>
hipError_t launch_chunk_t(const LinearShape& s, const ChunkCfg& c, const void* w, const float* x, float* y,
                          char* ws, hipStream_t stream, const ChunkGroup* grp = nullptr, bool presplit = false) {
    constexpr int lds = ChunkLds<QT, RW, TT, XS>::bytes;
    auto kern = gemm_chunk_kernel<QT, RW, TT, P, XS>;
    static bool attr = [&] {
        return hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                   lds) == hipSuccess;
    }();
    if (!attr) return hipErrorInvalidConfiguration;
    const ChunkWs l = chunk_layout(s, c);
    ChunkArgs a;
    a.W = static_cast<const uint8_t*>(w);
    a.x = x;
    a.xs = XS ? reinterpret_cast<const _Float16*>(ws + l.xs) : nullptr;
    a.bsum = XS ? reinterpret_cast<const float*>(ws + l.bsum) : nullptr;
    a.xscale = XS ? reinterpret_cast<const float*>(ws + l.scale) : nullptr;
    a.y = y;
    a.part = reinterpret_cast<float*>(ws + l.part);
    a.part_bytes = static_cast<uint32_t>(l.part_bytes);
    a.tile_count = reinterpret_cast<unsigned*>(ws);
    a.M = s.M, a.N = s.rows, a.K = s.K, a.nb = s.nb, a.npad = c.npad;
    a.row_tiles = c.row_tiles, a.splits = c.splits, a.chunks_per_split = c.cps;
    a.W1 = a.W2 = nullptr;
    a.y1 = a.y2 = nullptr;
    a.M1 = a.M2 = 0;
    a.tile1 = a.tile2 = c.row_tiles;
    a.xcd_br = 0;
    a.xcd_row_outer = 0;
    // One K split: block the tiles by XCD (4096 x 4096 Q4_0 at 512 tokens: fabric reads
    // 76.8 -> 52.7 MB per call, the time unchanged within 1 %).
    if (c.splits == 1 && (c.row_tiles * c.tok_tiles) % 8 == 0) {
        for (int br : {4, 2, 8, 1}) {
            const int bt = 8 / br;
            if (c.row_tiles % br == 0 && c.tok_tiles % bt == 0) {
                a.xcd_br = br;
                // Keep the smaller operand of the block resident: its weights (rows x K)
                // or its x (tokens x K, split: 4 bytes per element).
                const double wb = static_cast<double>(c.row_tiles / br) * 64 * RW * s.nb * block_bytes(s.qtype);
                const double xb = static_cast<double>(c.tok_tiles / bt) * 16 * TT * s.K * 4.0;
                a.xcd_row_outer = wb > xb ? 1 : 0;
                break;
            }
        }
    }
    if (grp != nullptr) {
        const int bm = 64 * RW;
        a.W = static_cast<const uint8_t*>(grp->w[0]);
        a.y = grp->y[0];
        a.M = grp->M[0];
        if (grp->n >= 2) {
            a.W1 = static_cast<const uint8_t*>(grp->w[1]), a.y1 = grp->y[1], a.M1 = grp->M[1];
            a.tile1 = grp->M[0] / bm;
        }
        if (grp->n >= 3) {
            a.W2 = static_cast<const uint8_t*>(grp->w[2]), a.y2 = grp->y[2], a.M2 = grp->M[2];
            a.tile2 = a.tile1 + grp->M[1] / bm;
        }
    }
    if (XS && !presplit) {
        hipLaunchKernelGGL((xsplit_kernel<QT>), dim3(c.npad), dim3(256), 0, stream, x, s.rows, s.K, s.nb, c.npad,
                           reinterpret_cast<_Float16*>(ws + l.xs), reinterpret_cast<float*>(ws + l.bsum),
                           reinterpret_cast<float*>(ws + l.scale));
    }
    const int grid = c.row_tiles * c.tok_tiles * c.splits;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kGemmThreads), lds, stream, a);
    return hipGetLastError();
}

template <int QT>
hipError_t launch_chunk_q(const LinearShape& s, const ChunkCfg& c, const void* w, const float* x, float* y,
                          char* ws, hipStream_t stream, const ChunkGroup* grp = nullptr, bool presplit = false) {
    if (c.tt == 1) return launch_chunk_t<QT, 1, 1, false>(s, c, w, x, y, ws, stream, grp);
    if (c.tt == 2 && !c.xs) return launch_chunk_t<QT, 2, 2, false>(s, c, w, x, y, ws, stream, grp);
    if (c.tt == 2) return launch_chunk_t<QT, 2, 2, true>(s, c, w, x, y, ws, stream, grp, presplit);
    return launch_chunk_t<QT, 2, 4, true>(s, c, w, x, y, ws, stream, grp, presplit);
}

bool use_chunk(const LinearShape& s, const float* x) {
    if (!chunk_supported(s)) return false;
    const ChunkCfg c = choose_chunk(s);
    const size_t wbytes = static_cast<size_t>(s.M) * s.nb * block_bytes(s.qtype);
    return (c.xs || (reinterpret_cast<uintptr_t>(x) & 15u) == 0) && wbytes < (static_cast<size_t>(1) << 32) &&
           chunk_layout(s, c).part_bytes < (static_cast<size_t>(1) << 31);
}

}  // namespace

bool gemm_supported(const LinearShape& s) {
    return s.rows > 1 && s.nb % 2 == 0 && s.nb >= 2 && (s.qtype >= 1 && s.qtype <= 3);
}

size_t gemm_workspace_bytes(const LinearShape& s) {
    if (!gemm_supported(s)) return 0;
    size_t b = layout(s, choose(s)).total;
    if (chunk_supported(s)) b = std::max(b, chunk_workspace_bytes(s));
    return b;
}

hipError_t launch_gemm(const LinearShape& s, const void* w, const float* x, float* y, void* ws,
                       size_t ws_bytes, hipStream_t stream) {
    if (!gemm_supported(s)) return hipErrorNotSupported;
    if (ws == nullptr) return hipErrorInvalidValue;
    char* base = static_cast<char*>(ws);
    if (use_chunk(s, x)) {
        if (ws_bytes < chunk_workspace_bytes(s)) return hipErrorInvalidValue;
        const ChunkCfg c = choose_chunk(s);
        switch (s.qtype) {
            case 1: return launch_chunk_q<1>(s, c, w, x, y, base, stream);
            case 2: return launch_chunk_q<2>(s, c, w, x, y, base, stream);
            default: return launch_chunk_q<3>(s, c, w, x, y, base, stream);
        }
    }
    const GemmCfg c = choose(s);
    const WsLayout l = layout(s, c);
    if (ws_bytes < l.total) return hipErrorInvalidValue;
    switch (s.qtype) {
        case 1: return launch_q<1>(s, c, l, w, x, y, base, stream);
        case 2: return launch_q<2>(s, c, l, w, x, y, base, stream);
        default: return launch_q<3>(s, c, l, w, x, y, base, stream);
    }
}

GemmSplitX gemm_split_x(const LinearShape& s, int n, const int* M) {
    GemmSplitX r{};
    if (n < 1 || n > 3 || M == nullptr) return r;
    LinearShape st = s;
    st.M = 0;
    for (int g = 0; g < n; ++g) {
        if (M[g] <= 0) return r;
        st.M += M[g];
    }
    if (!chunk_supported(st)) return r;
    const ChunkCfg c = choose_chunk(st);
    if (!c.xs || !use_chunk(st, nullptr)) return r;
    for (int g = 0; g + 1 < n; ++g)
        if (M[g] % (64 * c.rw) != 0) return r;
    const ChunkWs l = chunk_layout(st, c);
    r.ok = true;
    r.npad = c.npad;
    r.xs = l.xs;
    r.bsum = l.bsum;
    r.scale = l.scale;
    r.ws_bytes = l.total;
    return r;
}

bool gemm_group_supported(const LinearShape& s, int n, const int* M, const float* x) {
    if (n < 1 || n > 3 || M == nullptr) return false;
    LinearShape st = s;
    st.M = 0;
    for (int g = 0; g < n; ++g) {
        if (M[g] <= 0) return false;
        st.M += M[g];
    }
    if (!use_chunk(st, x)) return false;
    const int bm = 64 * choose_chunk(st).rw;
    for (int g = 0; g + 1 < n; ++g)
        if (M[g] % bm != 0) return false;  // a row tile may not straddle two weights
    return true;
}

hipError_t launch_gemm_group(const LinearShape& s, int n, const void* const* w, float* const* y, const int* M,
                             const float* x, void* ws, size_t ws_bytes, hipStream_t stream, bool x_split) {
    if (n < 1 || n > 3 || w == nullptr || y == nullptr || M == nullptr) return hipErrorInvalidValue;
    LinearShape st = s;
    st.M = 0;
    for (int g = 0; g < n; ++g) {
        if (M[g] <= 0) return hipErrorInvalidValue;
        st.M += M[g];
    }
    if (!gemm_group_supported(s, n, M, x)) return hipErrorNotSupported;
    const ChunkCfg c = choose_chunk(st);
    if (x_split && !c.xs) return hipErrorInvalidValue;  // gemm_split_x said no
    if (ws == nullptr) return hipErrorInvalidValue;
    if (ws_bytes < chunk_workspace_bytes(st)) return hipErrorInvalidValue;
    ChunkGroup grp{};
    grp.n = n;
    for (int g = 0; g < n; ++g) grp.w[g] = w[g], grp.y[g] = y[g], grp.M[g] = M[g];
    char* base = static_cast<char*>(ws);
    switch (st.qtype) {
        case 1: return launch_chunk_q<1>(st, c, w[0], x, y[0], base, stream, &grp, x_split);
        case 2: return launch_chunk_q<2>(st, c, w[0], x, y[0], base, stream, &grp, x_split);
        default: return launch_chunk_q<3>(st, c, w[0], x, y[0], base, stream, &grp, x_split);
    }
}

const char* gemm_kernel_name(const LinearShape& s) {
    static thread_local char buf[96];
    const char* fmt = s.qtype == 1 ? "q8_0" : s.qtype == 2 ? "q4_0" : "q4_1";
    if (chunk_supported(s)) {
        const ChunkCfg c = choose_chunk(s);
        snprintf(buf, sizeof buf, "gemm_mfma_%s_chunk%s_bm%d_bn%d_splitk%d", fmt, c.xs ? "_xs" : "", 64 * c.rw,
                 16 * c.tt, c.splits);
        return buf;
    }
    const GemmCfg c = choose(s);
    snprintf(buf, sizeof buf, "gemm_mfma_%s_bm%d_bn%d_splitk%d", fmt, c.bm, c.bn, c.splits);
    return buf;
}

}  // namespace mlq

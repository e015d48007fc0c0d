// Device helpers shared by the decode GEMV kernels (gemv.hip) and the
// persistent sequence kernel (sequence.hip): block formats, x staging into
// LDS as block-scaled integer limbs, the per-pair integer dot product and the
// DPP row reduction.  Both translation units include this file so a row is
// summed in exactly the same order by either kernel.
//
// Arithmetic.  Per 32-element block b of x, with m_b = max |x_k| over the
// block, x is written as x_k = s_b * X_k + e_k with s_b = m_b / R and the
// integer X_k = rint(x_k / s_b), |X_k| <= R, |e_k| <= s_b / 2:
//   Q4_0 / Q4_1: R = 32639 (two int8 limbs, X = 256 hi + lo),
//   Q8_0:        R = 4160000 (three limbs, X = 65536 hi + 256 mid + lo).
// The weights' integers (Q4 nibbles 0..15, Q8 bytes -128..127) meet the limbs
// in v_dot4 (four int8 products summed into an int32, exact), so per block
// and row the kernel gets the exact integer T = sum_k q_k X_k and then
//   Q4_0: y += d * (s_b * (T - 8 sum_k X_k))     (the -8 folded into the start)
//   Q4_1: y += d * (s_b * T) + m * sum_k x_k
//   Q8_0: y += d * (s_b * T)
// (src/quant.cpp:421-447 computes the same sums over d * q (+ m) in f32).
// Only x's representation (2^-16 or 2^-23 of the block maximum) and the f32
// steps after T round.  Against the CPU reference's f32 sums this is
// ~2e-5 (Q4) / ~1e-7 (Q8) relative to |y| on N(0, 1) inputs, and the error on
// outputs near zero stays ~20x below the 1e-3 * ||x|| * max|d| floor of the
// tolerance (Q4; Q8's third limb puts it ~5000x below).  A block holding an
// Inf or NaN gets s_b = NaN, so the rows it feeds come out NaN as in f32.
#pragma once

#include "mlq_kernels.h"

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mlq {
namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float h_lo(uint32_t v) { return (float)__builtin_bit_cast(h2_t, v).x; }
__device__ __forceinline__ float h_hi(uint32_t v) { return (float)__builtin_bit_cast(h2_t, v).y; }

template <int QT> struct Fmt;
template <> struct Fmt<1> { static constexpr int BB = 34, DW = 17; };  // Q8_0
template <> struct Fmt<2> { static constexpr int BB = 18, DW = 9; };   // Q4_0
template <> struct Fmt<3> { static constexpr int BB = 20, DW = 10; };  // Q4_1

// x limbs per format: L int8 limbs per element; a pair's x is 16 L dwords
// (per block 8 dwords of 4 elements per limb).
template <int QT> struct XLimbs {
    static constexpr int L = QT == 1 ? 3 : 2;
    static constexpr int PAIR_DW = 16 * L;
    // Largest |X|: balanced digits of X + 128 (+ 32768) must fit a signed
    // byte each, and 1.5 * 2^23 + X + 32896 must stay below 2^24.
    static constexpr float RANGE = QT == 1 ? 4160000.0f : 32639.0f;
};

// Device pointers that the compiler cannot trace to a kernel argument (loaded
// from a descriptor table) are generic; generic accesses become FLAT
// instructions, which count against the LDS counter as well and make every
// wait conservative.  These casts state that the memory is global.
typedef __attribute__((address_space(1))) const uint32_t g_u32;
typedef __attribute__((address_space(1))) const float g_f32;
__device__ __forceinline__ g_u32* as_global(const uint32_t* p) { return (g_u32*)p; }
__device__ __forceinline__ g_f32* as_global(const float* p) { return (g_f32*)p; }

constexpr int kMaxPairLdsBytes = 64 * 1024;
constexpr int kWaves = 8;             // waves per workgroup
constexpr int kPersistentWgs = 256;   // one workgroup per CU on a 256-CU MI355X

// LDS of the pair kernels: the x limbs (64 L bytes per pair) and 16 bytes of
// constants per block.
inline int pair_lds_bytes(int qtype, int nb) { return (nb / 2) * 64 * (qtype == 1 ? 3 : 2) + nb * 16; }

#define MLQ_DPP_F32(x, ctrl, rmask) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (x)), (ctrl), (rmask), 0xF, false))

__device__ __forceinline__ float quad_sum(float v) {
    v += MLQ_DPP_F32(v, 0xB1, 0xF);  // quad_perm [1,0,3,2]
    v += MLQ_DPP_F32(v, 0x4E, 0xF);  // quad_perm [2,3,0,1]
    return v;
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// Sum over the workgroup (every thread calls it; the result in every thread).
__device__ __forceinline__ float workgroup_sum(float v) {
    __shared__ float part[16];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = part[0];
    for (int i = 1; i < static_cast<int>(blockDim.x >> 6); ++i) t += part[i];
    return t;
}

// ---------------------------------------------------------------------------
// x staging.  Four threads per block, each taking two of the block's eight
// x dwords (four elements each).  The elements of x dword d are those the
// kernel's weight dword d of the same block holds, in byte order (PairDot
// below): Q4 x dword d = 2j + h pairs with qs dword j, low nibbles (h = 0,
// elements E_j) or high nibbles (h = 1, E_j + 16); Q8_0 x dword j pairs with
// qs dword j.  E_j, as two runs of two elements, is {4j, 4j+2} except in the
// first block of a pair of the formats whose qs start 2 bytes into a dword
// (Q4_0 / Q8_0): there the dwords are {qs[0,1], qs[last 2]} (one byte
// permute) and then the stored dwords, {4j-2, 4j}.
template <int QT>
__device__ __forceinline__ int2 x_runs(int blk, int d) {
    if (QT == 1) {
        if (blk == 0) return d == 0 ? make_int2(0, 30) : make_int2(4 * d - 2, 4 * d);
        return make_int2(4 * d, 4 * d + 2);
    }
    const int j = d >> 1, h = (d & 1) * 16;
    if (QT == 2 && blk == 0) return j == 0 ? make_int2(h, 14 + h) : make_int2(4 * j - 2 + h, 4 * j + h);
    return make_int2(4 * j + h, 4 * j + 2 + h);
}

// LDS placement of x dword idx (0 .. 16 L - 1) of pair p: 16-byte quads
// XOR-swizzled by pair so a wave's reads spread over the banks.
template <int QT>
__device__ __forceinline__ int x_slot(int p, int idx) {
    constexpr int L = XLimbs<QT>::L;
    const int swz = L == 2 ? (p & 7) : (p & 3);
    return p * (16 * L) + ((((idx >> 2) ^ swz)) << 2) + (idx & 3);
}

// The eight elements of thread `sub`'s two x dwords of block g; elements past
// K read as 0 (buffer range check), so a partial last block contributes
// nothing (the reference loops only k < K, src/quant.cpp:421-426).
// COHERENT loads with agent scope (sc1): they return what another workgroup
// of the same launch stored with agent-scope stores even when this XCD's L2
// holds an older copy of the line.
template <int QT, bool COHERENT>
__device__ __forceinline__ void load8(__amdgpu_buffer_rsrc_t rs, int g, int sub, float (&v)[8]) {
    constexpr int kPolicy = COHERENT ? 16 : 0;
    const int blk = g & 1;
#pragma unroll
    for (int dd = 0; dd < 2; ++dd) {
        const int2 r = x_runs<QT>(blk, 2 * sub + dd);
        const int e0 = (g * kQK + r.x) * 4, e1 = (g * kQK + r.y) * 4;
        v[4 * dd] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, e0, 0, kPolicy));
        v[4 * dd + 1] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, e0 + 4, 0, kPolicy));
        v[4 * dd + 2] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, e1, 0, kPolicy));
        v[4 * dd + 3] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, e1 + 4, 0, kPolicy));
    }
}

// Quantizes thread `sub`'s eight elements of block g (the four threads of the
// block are one aligned lane quad) and stores their limbs and, from sub 0,
// the block constants {s_b, -8 sum X (Q4_0, as int bits), sum x, 0}.
// X = rint(x / s_b) comes out of one fma as the low mantissa bits of
// x * (1 / s_b) + 1.5 * 2^23 (exact: |X| < 2^22, so the sum stays in the
// binade whose ulp is 1; the pattern is 0x4B400000 + X).  The balanced
// base-256 digits are then bytes of that integer offset by 128 (and 32896):
// lo = byte 0 of X, mid (Q8_0) or hi (Q4) = byte 1 of X + 128, hi (Q8_0) =
// byte 2 of X + 32896, each read as a signed byte; byte permutes gather four
// elements' digits into a dword.
template <int QT>
__device__ __forceinline__ void emit_block(int g, int sub, const float (&v)[8], uint32_t* __restrict__ xl,
                                           float4* __restrict__ xc) {
    constexpr int L = XLimbs<QT>::L;
    constexpr float RANGE = XLimbs<QT>::RANGE;
    constexpr float kMagic = 12582912.0f;  // 1.5 * 2^23
    // Largest |x| of the block, NaN if any element is NaN (Inf stays Inf).
    float m = __builtin_elementwise_maximum(__builtin_fabsf(v[0]), __builtin_fabsf(v[1]));
#pragma unroll
    for (int i = 2; i < 8; i += 2)
        m = __builtin_elementwise_maximum(m, __builtin_elementwise_maximum(__builtin_fabsf(v[i]), __builtin_fabsf(v[i + 1])));
    m = __builtin_elementwise_maximum(m, MLQ_DPP_F32(m, 0xB1, 0xF));
    m = __builtin_elementwise_maximum(m, MLQ_DPP_F32(m, 0x4E, 0xF));
    // Blocks below 2^-100 are scaled by 2^64 first, so RANGE / m stays finite;
    // m = Inf or NaN gives inv = 0 and s_b = Inf or NaN: the rows come out
    // non-finite.
    const float k = m < 0x1p-100f ? 0x1p64f : 1.0f;
    const float mk = m * k;
    // 1 / s_b to within an ulp or two: s_b * inv = 1 + O(2^-22), far below
    // x's own representation error (2^-16 of the block maximum).
    const float inv = mk > 0.0f && mk <= 3.4e38f ? RANGE * __builtin_amdgcn_rcpf(mk) : 0.0f;
    const float s = mk * (1.0f / RANGE) * (m < 0x1p-100f ? 0x1p-64f : 1.0f);
    uint32_t out[L][2];
    float xs = 0.0f;
#pragma unroll
    for (int dd = 0; dd < 2; ++dd) {
        uint32_t a[4], b[4], c[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float xv = v[4 * dd + e];
            if (QT == 3) xs += xv;
            const float f = __builtin_fmaf(xv * k, inv, kMagic);
            a[e] = __builtin_bit_cast(uint32_t, f);
            b[e] = __builtin_bit_cast(uint32_t, f + 128.0f);
            // (byte 2 of 1.5 * 2^23 is 0x40: taken out of the integer first)
            if (L == 3) c[e] = __builtin_bit_cast(uint32_t, f + 32896.0f) - 0x00400000u;
        }
        // perm(hi, lo, sel): result byte i = byte sel_i of {hi:lo} (lo = 0..3).
        auto gather = [](const uint32_t (&r)[4], uint32_t byte_sel) -> uint32_t {
            const uint32_t s01 = byte_sel | ((byte_sel + 4) << 8) | 0x0C0C0000u;  // {r0.b, r1.b, 0, 0}
            const uint32_t s23 = 0x0C0Cu | (byte_sel << 16) | ((byte_sel + 4) << 24);  // {0, 0, r2.b, r3.b}
            return __builtin_amdgcn_perm(r[1], r[0], s01) | __builtin_amdgcn_perm(r[3], r[2], s23);
        };
        if (L == 2) {
            out[0][dd] = gather(b, 1);
            out[1][dd] = gather(a, 0);
        } else {
            out[0][dd] = gather(c, 2);
            out[1][dd] = gather(b, 1);
            out[2][dd] = gather(a, 0);
        }
    }
    const int p = g >> 1, blk = g & 1;
#pragma unroll
    for (int l = 0; l < L; ++l) {
        const int idx = blk * (8 * L) + l * 8 + 2 * sub;
        *reinterpret_cast<uint2*>(xl + x_slot<QT>(p, idx)) = make_uint2(out[l][0], out[l][1]);
    }
    int sx = 0;
    if (QT == 2) {  // sum X = 256 sum hi + sum lo over the thread's elements
        const int ones = 0x01010101;
        sx = 256 * (dot4(out[0][0], ones, 0) + dot4(out[0][1], ones, 0)) + dot4(out[1][0], ones, 0) +
             dot4(out[1][1], ones, 0);
        sx += __builtin_amdgcn_update_dpp(0, sx, 0xB1, 0xF, 0xF, false);
        sx += __builtin_amdgcn_update_dpp(0, sx, 0x4E, 0xF, 0xF, false);
    }
    if (QT == 3) xs = quad_sum(xs);
    if (sub == 0) xc[g] = make_float4(s, __builtin_bit_cast(float, -8 * sx), xs, 0.0f);
}

// Stages x (or, NORM, rmsnorm(x) * norm_w: src/ops.cpp:18-41, mean of squares
// over the K elements, scale = 1 / sqrt(ms + eps), x * scale * w; every
// workgroup normalises its own copy) into LDS as limbs plus block constants.
// Loads are issued kBatch rounds (of blockDim / 4 blocks) at a time, so a long
// x pays the load latency once per batch.  Ends with the workgroup barrier
// that makes the limbs visible.
constexpr int kBatch = 3;

// Rounds past the last block re-read the last block (unused): a load under a
// branch makes the compiler wait for it at the branch's end, which would
// serialise the x loads with the weight requests that follow them.
template <int QT, bool COHERENT, int B>
__device__ __forceinline__ void load_batch(__amdgpu_buffer_rsrc_t rs, int g, int per, int nb, int sub,
                                           float (&v)[B][8]) {
#pragma unroll
    for (int r = 0; r < B; ++r) load8<QT, COHERENT>(rs, min(g + r * per, nb - 1), sub, v[r]);
}

struct NoRequests {
    __device__ __forceinline__ void operator()() const {}
};

// The first batch's x (and norm_w) loads are issued before `after_loads()`
// runs, so a kernel can request its weights there: the x loads, older in the
// in-order load counter, are then waited for without waiting for the weights.
// B: rounds per batch (1 when the caller knows nb <= blockDim / 4).
// ONE: the caller guarantees nb <= B * blockDim / 4 (one batch): the code has
// no loop and no load under a branch, so nothing makes the compiler wait for
// the weight requests issued in `after_loads` before quantizing.
template <int QT, bool COHERENT = false, bool NORM = false, int B = kBatch, bool ONE = false,
          typename F = NoRequests>
__device__ __forceinline__ void stage_x(const float* __restrict__ x, int K, int nb, uint32_t* __restrict__ xl,
                                        float4* __restrict__ xc, const float* __restrict__ norm_w = nullptr,
                                        float norm_eps = 0.0f, F&& after_loads = F{}) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(x), static_cast<short>(0), K * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(NORM ? norm_w : x), static_cast<short>(0), K * 4, 0x00020000);
    const int per = static_cast<int>(blockDim.x >> 2);
    const int sub = threadIdx.x & 3;
    const int g0 = static_cast<int>(threadIdx.x >> 2);
    const int step = B * per;
    float v[B][8];
    float w[B][8];
    if (ONE) {
        load_batch<QT, COHERENT, B>(rs, g0, per, nb, sub, v);
        if (NORM) load_batch<QT, false, B>(rw, g0, per, nb, sub, w);
        after_loads();
        if (NORM) {
            float ss = 0.0f;
#pragma unroll
            for (int r = 0; r < B; ++r) {
                float t = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) t += v[r][i] * v[r][i];
                ss += g0 + r * per < nb ? t : 0.0f;  // rounds past the last block re-read it
            }
            const float scale = 1.0f / sqrtf(workgroup_sum(ss) / static_cast<float>(K) + norm_eps);
#pragma unroll
            for (int r = 0; r < B; ++r)
#pragma unroll
                for (int i = 0; i < 8; ++i) v[r][i] = v[r][i] * scale * w[r][i];
        }
#pragma unroll
        for (int r = 0; r < B; ++r)
            if (g0 + r * per < nb) emit_block<QT>(g0 + r * per, sub, v[r], xl, xc);
        __syncthreads();
        return;
    }
    if (!NORM && __is_same(F, NoRequests)) {  // nothing to interleave: one loop over the batches
        for (int g = g0; g < nb; g += step) {
            load_batch<QT, COHERENT, B>(rs, g, per, nb, sub, v);
#pragma unroll
            for (int r = 0; r < B; ++r)
                if (g + r * per < nb) emit_block<QT>(g + r * per, sub, v[r], xl, xc);
        }
        __syncthreads();
        return;
    }
    load_batch<QT, COHERENT, B>(rs, g0, per, nb, sub, v);
    if (NORM) load_batch<QT, false, B>(rw, g0, per, nb, sub, w);
    after_loads();
    float scale = 1.0f;
    if (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int r = 0; r < B; ++r)
            if (g0 + r * per < nb)
#pragma unroll
                for (int i = 0; i < 8; ++i) ss += v[r][i] * v[r][i];
        for (int g = g0 + step; g < nb; g += step) {
            float t[B][8];
            load_batch<QT, COHERENT, B>(rs, g, per, nb, sub, t);
#pragma unroll
            for (int r = 0; r < B; ++r)
                if (g + r * per < nb)
#pragma unroll
                    for (int i = 0; i < 8; ++i) ss += t[r][i] * t[r][i];
        }
        scale = 1.0f / sqrtf(workgroup_sum(ss) / static_cast<float>(K) + norm_eps);
    }
    for (int g = g0; g < nb; g += step) {
        if (g != g0) {
            load_batch<QT, COHERENT, B>(rs, g, per, nb, sub, v);
            if (NORM) load_batch<QT, false, B>(rw, g, per, nb, sub, w);
        }
        if (NORM) {
#pragma unroll
            for (int r = 0; r < B; ++r)
#pragma unroll
                for (int i = 0; i < 8; ++i) v[r][i] = v[r][i] * scale * w[r][i];
        }
#pragma unroll
        for (int r = 0; r < B; ++r)
            if (g + r * per < nb) emit_block<QT>(g + r * per, sub, v[r], xl, xc);
    }
    __syncthreads();
}

// stage_x with as many load rounds per batch as the row needs (up to
// kBatch): a round past the last block only re-reads it.
template <int QT, bool COHERENT = false, bool NORM = false, typename F = NoRequests>
__device__ __forceinline__ void stage_x_fit(const float* __restrict__ x, int K, int nb, uint32_t* __restrict__ xl,
                                            float4* __restrict__ xc, const float* __restrict__ norm_w = nullptr,
                                            float norm_eps = 0.0f, F&& after_loads = F{}) {
    const int per = static_cast<int>(blockDim.x >> 2);
    if (nb <= per) {
        stage_x<QT, COHERENT, NORM, 1, true>(x, K, nb, xl, xc, norm_w, norm_eps, after_loads);
    } else if (nb <= 2 * per) {
        stage_x<QT, COHERENT, NORM, 2, true>(x, K, nb, xl, xc, norm_w, norm_eps, after_loads);
    } else if (nb <= kBatch * per) {
        stage_x<QT, COHERENT, NORM, kBatch, true>(x, K, nb, xl, xc, norm_w, norm_eps, after_loads);
    } else {
        stage_x<QT, COHERENT, NORM, kBatch, false>(x, K, nb, xl, xc, norm_w, norm_eps, after_loads);
    }
}

// A lane's x for pair p: its 16 L limb dwords and the two blocks' constants.
template <int QT>
__device__ __forceinline__ void load_xq(const uint32_t* __restrict__ xl, const float4* __restrict__ xc, int p,
                                        uint32_t (&xq)[XLimbs<QT>::PAIR_DW], float4& c0, float4& c1) {
    constexpr int Q = XLimbs<QT>::PAIR_DW / 4;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const uint4 v = *reinterpret_cast<const uint4*>(xl + x_slot<QT>(p, 4 * q));
        xq[4 * q] = v.x;
        xq[4 * q + 1] = v.y;
        xq[4 * q + 2] = v.z;
        xq[4 * q + 3] = v.w;
    }
    c0 = xc[2 * p];
    c1 = xc[2 * p + 1];
}

__device__ __forceinline__ int block_c(const float4& c) { return __builtin_bit_cast(int, c.y); }

// acc += contribution of one pair (two blocks) of one row.
template <int QT> struct PairDot;

// One Q4 block: qs dwords q[0..3], x dwords xb[0..15] (limb 0 then limb 1,
// each low / high nibble alternating); returns the exact 256 H + L.
__device__ __forceinline__ int q4_block(const uint32_t (&q)[4], const uint32_t* xb, int start) {
    int h = 0, l = start;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t a = q[j] & 0x0F0F0F0Fu;
        const uint32_t b = (q[j] >> 4) & 0x0F0F0F0Fu;
        h = dot4(a, xb[2 * j], h);
        l = dot4(a, xb[8 + 2 * j], l);
        h = dot4(b, xb[2 * j + 1], h);
        l = dot4(b, xb[8 + 2 * j + 1], l);
    }
    return h * 256 + l;
}

template <> struct PairDot<2> {  // Q4_0: w0 = {d0, qs0[0..1]}, w4 = {qs0[14..15], d1}
    __device__ __forceinline__ static float run(const uint32_t* w, const uint32_t (&xq)[32], const float4& c0,
                                                const float4& c1, float acc) {
        const uint32_t q0[4] = {__builtin_amdgcn_perm(w[4], w[0], 0x05040302u), w[1], w[2], w[3]};  // qs0[0,1,14,15]
        const uint32_t q1[4] = {w[5], w[6], w[7], w[8]};
        const int t0 = q4_block(q0, xq, block_c(c0));
        const int t1 = q4_block(q1, xq + 16, block_c(c1));
        acc = __builtin_fmaf(h_lo(w[0]), c0.x * static_cast<float>(t0), acc);
        acc = __builtin_fmaf(h_hi(w[4]), c1.x * static_cast<float>(t1), acc);
        return acc;
    }
};

template <> struct PairDot<3> {  // Q4_1: w0 = {d0, m0}, w5 = {d1, m1}
    __device__ __forceinline__ static float run(const uint32_t* w, const uint32_t (&xq)[32], const float4& c0,
                                                const float4& c1, float acc) {
        const uint32_t q0[4] = {w[1], w[2], w[3], w[4]};
        const uint32_t q1[4] = {w[6], w[7], w[8], w[9]};
        const int t0 = q4_block(q0, xq, 0);
        const int t1 = q4_block(q1, xq + 16, 0);
        acc = __builtin_fmaf(h_lo(w[0]), c0.x * static_cast<float>(t0), acc);
        acc = __builtin_fmaf(h_hi(w[0]), c0.z, acc);
        acc = __builtin_fmaf(h_lo(w[5]), c1.x * static_cast<float>(t1), acc);
        acc = __builtin_fmaf(h_hi(w[5]), c1.z, acc);
        return acc;
    }
};

template <> struct PairDot<1> {  // Q8_0: w0 = {d0, qs0[0..1]}, w8 = {qs0[30..31], d1}
    // One block: qs dwords q[0..7] (signed bytes), x dwords xb[0..23]
    // (limbs hi, mid, lo); returns sum q X in f32 (|sum| < 2^34, so the
    // limbs' partial sums are combined in f32).
    __device__ __forceinline__ static float block(const uint32_t (&q)[8], const uint32_t* xb) {
        int h = 0, md = 0, l = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            h = dot4(q[j], xb[j], h);
            md = dot4(q[j], xb[8 + j], md);
            l = dot4(q[j], xb[16 + j], l);
        }
        return __builtin_fmaf(65536.0f, static_cast<float>(h), static_cast<float>(md * 256 + l));
    }
    __device__ __forceinline__ static float run(const uint32_t* w, const uint32_t (&xq)[48], const float4& c0,
                                                const float4& c1, float acc) {
        const uint32_t q0[8] = {__builtin_amdgcn_perm(w[8], w[0], 0x05040302u), w[1], w[2], w[3], w[4], w[5], w[6], w[7]};
        const uint32_t q1[8] = {w[9], w[10], w[11], w[12], w[13], w[14], w[15], w[16]};
        const float t0 = block(q0, xq);
        const float t1 = block(q1, xq + 24);
        acc = __builtin_fmaf(h_lo(w[0]), c0.x * t0, acc);
        acc = __builtin_fmaf(h_hi(w[8]), c1.x * t1, acc);
        return acc;
    }
};

// Sum over each aligned group of LPR lanes with DPP adds (VALU only).  The
// total is complete in the group's last lane (in every lane for LPR <= 16).
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
    v += MLQ_DPP_F32(v, 0xB1, 0xF);    // quad_perm [1,0,3,2]
    v += MLQ_DPP_F32(v, 0x4E, 0xF);    // quad_perm [2,3,0,1]
    v += MLQ_DPP_F32(v, 0x141, 0xF);   // row_half_mirror: 8-lane sums
    if (LPR >= 16) v += MLQ_DPP_F32(v, 0x140, 0xF);  // row_mirror: 16-lane sums
    if (LPR >= 32) v += MLQ_DPP_F32(v, 0x142, 0xA);  // row_bcast:15 into rows 1, 3
    if (LPR >= 64) v += MLQ_DPP_F32(v, 0x143, 0xC);  // row_bcast:31 into rows 2, 3
    return v;
}

}  // namespace
}  // namespace mlq

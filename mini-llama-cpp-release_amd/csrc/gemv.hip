// Decode GEMV for Q8_0 / Q4_0 / Q4_1 weights on gfx950 (MI355X).
//
// y[M] = W[M, K] . x[K], W stored as the reference's 32-element blocks
// (quantized_tensor.h:26-59), x and y f32.  This replaces the
// one-thread-per-output kernels of src/cuda_quant.cu:37-137.
//
// Layout and work split:
//  * A *pair* is two consecutive blocks of a row: 36 / 68 / 40 bytes for
//    Q4_0 / Q8_0 / Q4_1, a multiple of 4 bytes.  When a row holds an even
//    number of blocks every pair starts 4-byte aligned, so a lane reads its
//    pair with 9 / 17 / 10 dword loads and a wave reads a contiguous span of a
//    row: coalesced, with the stored format untouched.
//  * LPR lanes ("a slot") share R rows; lane l of a slot owns pairs
//    l, l + LPR, ... of those rows.  A wave holds 64 / LPR slots.
//  * x is staged once per workgroup in LDS as f32 with per-block constants
//    (one thread per block, whole-block vector loads); 16-byte LDS slots are
//    XOR-swizzled by pair so a wave's reads spread over the banks.
//  * Every lane requests its first W pair(s) before staging x, so the W
//    latency overlaps the staging and the barrier.
//  * "single" kernel (row of at most LPR pairs): each lane keeps its 64 x
//    values in VGPRs and the workgroups are persistent (at most ~2 per CU),
//    walking row groups with the next group's W requested before the current
//    one is computed.  "multi" kernel (longer rows): one row group per wave,
//    x read from LDS per pair, next pair's W requested before the current one
//    is computed.
//  * Row sums are reduced across the slot's lanes with DPP adds (quad_perm,
//    row mirrors, row_bcast), all VALU, no LDS round trip.
//
// Arithmetic (VALU, fp32 accumulate, ~1.7 VALU ops per weight):
//  * A stored nibble or biased byte becomes an exact fp16 integer with one
//    AND-OR (or one byte permute) against the fp16 pattern 0x6400 (1024.0):
//    Q4 low nibble q -> 1024 + q, Q4 high nibble (masked in place) -> 1024 + 16q,
//    Q8 byte q ^ 0x80 -> 1024 + 128 + q.  Two such values share a dword.
//  * v_fma_mix_f32 multiplies the fp16 half by the f32 x element and
//    accumulates in f32; x of high-nibble elements is pre-scaled by 1/16 so
//    16q * x/16 == q * x.
//  * Each block is summed in two chains (ILP) starting at -bias, where
//    bias = 1024 * sum(x') + 8 * sum(x) (Q4_0), 1024 * sum(x') (Q4_1),
//    1152 * sum(x) (Q8_0) is computed once per workgroup; the chains end at
//    sum(q_signed * x) for the block, then y += d * sum (+ m * sum(x) for Q4_1)
//    with d and m read as fp16 operands of the same fma_mix.
//  Products are exact; only the f32 accumulations round.  The intermediate
//  magnitude (~1024 * |partial sum of x|) costs ~10 bits of the f32 sum, i.e.
//  ~1e-4 relative error per block sum, far inside the 1e-3 tolerance.
//
// Rows with an odd block count (pairs would straddle rows) and very long rows
// go to a simple one-wave-per-row kernel with byte loads.

#include "mlq_kernels.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

namespace mlq {
namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float h_lo(uint32_t v) { return (float)__builtin_bit_cast(h2_t, v).x; }
__device__ __forceinline__ float h_hi(uint32_t v) { return (float)__builtin_bit_cast(h2_t, v).y; }

constexpr uint32_t kF16Magic2 = 0x64006400u;   // {1024.0h, 1024.0h}
constexpr uint32_t kF16MagicB = 0x64646464u;   // byte source for v_perm

template <int QT> struct Fmt;
template <> struct Fmt<1> { static constexpr int BB = 34, DW = 17; };  // Q8_0
template <> struct Fmt<2> { static constexpr int BB = 18, DW = 9; };   // Q4_0
template <> struct Fmt<3> { static constexpr int BB = 20, DW = 10; };  // Q4_1

constexpr int kMaxPairLdsBytes = 64 * 1024;
constexpr int kWaves = 8;             // waves per workgroup
constexpr int kPersistentWgs = 512;   // ~2 workgroups per CU on a 256-CU MI355X

// ---------------------------------------------------------------------------
// x staging: one thread per block.  Writes x' (f32, Q4 high halves scaled by
// 1/16) into 16-byte slots swizzled by pair, and per-block constants {c0, c1}:
//   Q8_0: c0 = 1152 * X          Q4_0: c0 = 1024 * S + 8 * X
//   Q4_1: c0 = 1024 * S, c1 = X  with X = sum(x), S = sum(x') over the block.
// Elements past K read as 0, so a partial last block contributes nothing
// (the reference loops only k < K, src/quant.cpp:421-426).
template <int QT>
__device__ __forceinline__ void stage_x(const float* __restrict__ x, int K, int nb,
                                        float4* __restrict__ xs4, float2* __restrict__ cb) {
    for (int g = threadIdx.x; g < nb; g += blockDim.x) {
        float v[32];
        const int k0 = g * kQK;
        if (k0 + kQK <= K && (reinterpret_cast<uintptr_t>(x + k0) & 15u) == 0) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 f = reinterpret_cast<const float4*>(x + k0)[i];
                v[4 * i] = f.x;
                v[4 * i + 1] = f.y;
                v[4 * i + 2] = f.z;
                v[4 * i + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i) v[i] = (k0 + i < K) ? x[k0 + i] : 0.0f;
        }
        float X = 0.0f;
        float S = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i += 4) X += (v[i] + v[i + 1]) + (v[i + 2] + v[i + 3]);
        if (QT != 1) {
#pragma unroll
            for (int i = 16; i < 32; ++i) v[i] *= 0.0625f;
#pragma unroll
            for (int i = 0; i < 32; i += 4) S += (v[i] + v[i + 1]) + (v[i + 2] + v[i + 3]);
        }
        const int p = g >> 1;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int slot = ((g & 1) << 3) + j;
            xs4[p * 16 + (slot ^ (p & 15))] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
        }
        float2 c;
        if (QT == 1) {
            c.x = 1152.0f * X;
            c.y = 0.0f;
        } else if (QT == 2) {
            c.x = 1024.0f * S + 8.0f * X;
            c.y = 0.0f;
        } else {
            c.x = 1024.0f * S;
            c.y = X;
        }
        cb[g] = c;
    }
}

__device__ __forceinline__ void load_xv(const float4* __restrict__ xs4, int p, float (&xv)[64]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float4 v = xs4[p * 16 + (i ^ (p & 15))];
        xv[4 * i] = v.x;
        xv[4 * i + 1] = v.y;
        xv[4 * i + 2] = v.z;
        xv[4 * i + 3] = v.w;
    }
}

// Bit patterns the nibble expansion needs, held in VGPRs: gfx9 VOP3 encodings
// take no literal, so only register operands let (d & mask) | magic issue as a
// single v_and_or_b32.  The empty asm makes the values opaque to the compiler,
// which would otherwise rematerialise them as literals of two VOP2 ops.
struct NibConsts {
    uint32_t lo;     // 0x000F000F: low nibbles of bytes 0 and 2
    uint32_t hi;     // 0x00F000F0: high nibbles of bytes 0 and 2, in place
    uint32_t magic;  // 0x64006400
    __device__ __forceinline__ static NibConsts make() {
        NibConsts c{0x000F000Fu, 0x00F000F0u, kF16Magic2};
        asm volatile("" : "+v"(c.lo), "+v"(c.hi), "+v"(c.magic));
        return c;
    }
};

// One dword of Q4 nibbles: bytes hold qs[j0..j3] of one block (low nibble =
// element j, high nibble = element j + 16, src/quant.cpp:259, 442-447).
template <int J0, int J1, int J2, int J3, int BASE>
__device__ __forceinline__ float nib_dot(uint32_t d, const float* xv, float a, const NibConsts& k) {
    const uint32_t lo02 = (d & k.lo) | k.magic;
    const uint32_t hi02 = (d & k.hi) | k.magic;
    const uint32_t d8 = d >> 8;
    const uint32_t lo13 = (d8 & k.lo) | k.magic;
    const uint32_t hi13 = (d8 & k.hi) | k.magic;
    a = __builtin_fmaf(h_lo(lo02), xv[BASE + J0], a);
    a = __builtin_fmaf(h_hi(lo02), xv[BASE + J2], a);
    a = __builtin_fmaf(h_lo(hi02), xv[BASE + J0 + 16], a);
    a = __builtin_fmaf(h_hi(hi02), xv[BASE + J2 + 16], a);
    a = __builtin_fmaf(h_lo(lo13), xv[BASE + J1], a);
    a = __builtin_fmaf(h_hi(lo13), xv[BASE + J3], a);
    a = __builtin_fmaf(h_lo(hi13), xv[BASE + J1 + 16], a);
    a = __builtin_fmaf(h_hi(hi13), xv[BASE + J3 + 16], a);
    return a;
}

// One dword of Q8_0 bytes qs[j0..j3].
template <int J0, int J1, int J2, int J3, int BASE>
__device__ __forceinline__ float byte_dot(uint32_t d, const float* xv, float a) {
    const uint32_t dx = d ^ 0x80808080u;
    const uint32_t p01 = __builtin_amdgcn_perm(kF16MagicB, dx, 0x04010400u);
    const uint32_t p23 = __builtin_amdgcn_perm(kF16MagicB, dx, 0x04030402u);
    a = __builtin_fmaf(h_lo(p01), xv[BASE + J0], a);
    a = __builtin_fmaf(h_hi(p01), xv[BASE + J1], a);
    a = __builtin_fmaf(h_lo(p23), xv[BASE + J2], a);
    a = __builtin_fmaf(h_hi(p23), xv[BASE + J3], a);
    return a;
}

// acc += contribution of one pair (two blocks) of one row; each block is
// summed as two interleaved chains.
template <int QT> struct PairDot;

template <> struct PairDot<2> {  // Q4_0: w0 = {d0, qs0[0..1]}, w4 = {qs0[14..15], d1}
    __device__ __forceinline__ static float run(const uint32_t* w, const float* xv, float2 c0,
                                                float2 c1, float acc, const NibConsts& k) {
        const uint32_t t = __builtin_amdgcn_perm(w[4], w[0], 0x05040302u);  // qs0[0,1,14,15]
        float a0 = -c0.x, a1 = 0.0f, b0 = -c1.x, b1 = 0.0f;
        a0 = nib_dot<0, 1, 14, 15, 0>(t, xv, a0, k);
        a1 = nib_dot<2, 3, 4, 5, 0>(w[1], xv, a1, k);
        b0 = nib_dot<0, 1, 2, 3, 32>(w[5], xv, b0, k);
        b1 = nib_dot<4, 5, 6, 7, 32>(w[6], xv, b1, k);
        a0 = nib_dot<6, 7, 8, 9, 0>(w[2], xv, a0, k);
        a1 = nib_dot<10, 11, 12, 13, 0>(w[3], xv, a1, k);
        b0 = nib_dot<8, 9, 10, 11, 32>(w[7], xv, b0, k);
        b1 = nib_dot<12, 13, 14, 15, 32>(w[8], xv, b1, k);
        acc = __builtin_fmaf(h_lo(w[0]), a0 + a1, acc);
        acc = __builtin_fmaf(h_hi(w[4]), b0 + b1, acc);
        return acc;
    }
};

template <> struct PairDot<3> {  // Q4_1: w0 = {d0, m0}, w5 = {d1, m1}
    __device__ __forceinline__ static float run(const uint32_t* w, const float* xv, float2 c0,
                                                float2 c1, float acc, const NibConsts& k) {
        float a0 = -c0.x, a1 = 0.0f, b0 = -c1.x, b1 = 0.0f;
        a0 = nib_dot<0, 1, 2, 3, 0>(w[1], xv, a0, k);
        a1 = nib_dot<4, 5, 6, 7, 0>(w[2], xv, a1, k);
        b0 = nib_dot<0, 1, 2, 3, 32>(w[6], xv, b0, k);
        b1 = nib_dot<4, 5, 6, 7, 32>(w[7], xv, b1, k);
        a0 = nib_dot<8, 9, 10, 11, 0>(w[3], xv, a0, k);
        a1 = nib_dot<12, 13, 14, 15, 0>(w[4], xv, a1, k);
        b0 = nib_dot<8, 9, 10, 11, 32>(w[8], xv, b0, k);
        b1 = nib_dot<12, 13, 14, 15, 32>(w[9], xv, b1, k);
        acc = __builtin_fmaf(h_lo(w[0]), a0 + a1, acc);
        acc = __builtin_fmaf(h_hi(w[0]), c0.y, acc);
        acc = __builtin_fmaf(h_lo(w[5]), b0 + b1, acc);
        acc = __builtin_fmaf(h_hi(w[5]), c1.y, acc);
        return acc;
    }
};

template <> struct PairDot<1> {  // Q8_0: w0 = {d0, qs0[0..1]}, w8 = {qs0[30..31], d1}
    __device__ __forceinline__ static float run(const uint32_t* w, const float* xv, float2 c0,
                                                float2 c1, float acc, const NibConsts&) {
        const uint32_t t = __builtin_amdgcn_perm(w[8], w[0], 0x05040302u);  // qs0[0,1,30,31]
        float a0 = -c0.x, a1 = 0.0f, b0 = -c1.x, b1 = 0.0f;
        a0 = byte_dot<0, 1, 30, 31, 0>(t, xv, a0);
        a1 = byte_dot<2, 3, 4, 5, 0>(w[1], xv, a1);
        b0 = byte_dot<0, 1, 2, 3, 32>(w[9], xv, b0);
        b1 = byte_dot<4, 5, 6, 7, 32>(w[10], xv, b1);
        a0 = byte_dot<6, 7, 8, 9, 0>(w[2], xv, a0);
        a1 = byte_dot<10, 11, 12, 13, 0>(w[3], xv, a1);
        b0 = byte_dot<8, 9, 10, 11, 32>(w[11], xv, b0);
        b1 = byte_dot<12, 13, 14, 15, 32>(w[12], xv, b1);
        a0 = byte_dot<14, 15, 16, 17, 0>(w[4], xv, a0);
        a1 = byte_dot<18, 19, 20, 21, 0>(w[5], xv, a1);
        b0 = byte_dot<16, 17, 18, 19, 32>(w[13], xv, b0);
        b1 = byte_dot<20, 21, 22, 23, 32>(w[14], xv, b1);
        a0 = byte_dot<22, 23, 24, 25, 0>(w[6], xv, a0);
        a1 = byte_dot<26, 27, 28, 29, 0>(w[7], xv, a1);
        b0 = byte_dot<24, 25, 26, 27, 32>(w[15], xv, b0);
        b1 = byte_dot<28, 29, 30, 31, 32>(w[16], xv, b1);
        acc = __builtin_fmaf(h_lo(w[0]), a0 + a1, acc);
        acc = __builtin_fmaf(h_hi(w[8]), b0 + b1, acc);
        return acc;
    }
};

// Sum over each aligned group of LPR lanes with DPP adds (VALU only).  The
// total is complete in the group's last lane (in every lane for LPR <= 16).
#define MLQ_DPP_F32(x, ctrl, rmask) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (x)), (ctrl), (rmask), 0xF, false))
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

template <int R, int DW>
__device__ __forceinline__ void load_rows(const uint32_t* __restrict__ W, size_t row_dw, int row0, int M,
                                          int p, uint32_t (&w)[R][DW]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r, M - 1);  // rows past M compute on row M-1 and are dropped
        const uint32_t* src = W + static_cast<size_t>(row) * row_dw + static_cast<size_t>(p) * DW;
#pragma unroll
        for (int i = 0; i < DW; ++i) w[r][i] = src[i];
    }
}

// Rows of at most LPR pairs: x in VGPRs, persistent over row groups.
template <int QT, int LPR, int R, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemv_single_kernel(
    const uint8_t* __restrict__ Wb, const float* __restrict__ x, float* __restrict__ y, int M, int K,
    int nb, int groups) {
    constexpr int DW = Fmt<QT>::DW;
    constexpr int SUB = 64 / LPR;
    extern __shared__ float4 lds4[];
    const int np = nb >> 1;
    float4* xs4 = lds4;
    float2* cb = reinterpret_cast<float2*>(lds4 + np * 16);
    x += static_cast<size_t>(blockIdx.y) * K;
    y += static_cast<size_t>(blockIdx.y) * M;
    const uint32_t* W = reinterpret_cast<const uint32_t*>(Wb);

    const int lane = threadIdx.x & 63;
    const int slot = lane / LPR;
    const int pl = lane % LPR;
    const bool active = pl < np;
    const int p = active ? pl : 0;
    const size_t row_dw = static_cast<size_t>(np) * DW;
    const int gstride = gridDim.x * WAVES;
    int gi = blockIdx.x * WAVES + (threadIdx.x >> 6);

    uint32_t wc[R][DW];
    if (gi < groups) load_rows<R, DW>(W, row_dw, gi * (SUB * R) + slot * R, M, p, wc);
    stage_x<QT>(x, K, nb, xs4, cb);
    __syncthreads();
    float xv[64];
    load_xv(xs4, p, xv);
    const float2 c0 = cb[2 * p];
    const float2 c1 = cb[2 * p + 1];
    const NibConsts nk = NibConsts::make();

    for (; gi < groups; gi += gstride) {
        uint32_t wn[R][DW];
        const int gn = gi + gstride;
        if (gn < groups) load_rows<R, DW>(W, row_dw, gn * (SUB * R) + slot * R, M, p, wn);
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = active ? PairDot<QT>::run(wc[r], xv, c0, c1, 0.0f, nk) : 0.0f;
            acc[r] = group_sum<LPR>(acc[r]);
        }
        if (pl == LPR - 1) {
            const int row0 = gi * (SUB * R) + slot * R;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (row0 + r < M) y[row0 + r] = acc[r];
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < DW; ++i) wc[r][i] = wn[r][i];
    }
}

// Rows of more than LPR pairs: one row group per wave, x from LDS per pair.
template <int QT, int LPR, int R, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemv_multi_kernel(
    const uint8_t* __restrict__ Wb, const float* __restrict__ x, float* __restrict__ y, int M, int K,
    int nb) {
    constexpr int DW = Fmt<QT>::DW;
    constexpr int SUB = 64 / LPR;
    extern __shared__ float4 lds4[];
    const int np = nb >> 1;
    float4* xs4 = lds4;
    float2* cb = reinterpret_cast<float2*>(lds4 + np * 16);
    x += static_cast<size_t>(blockIdx.y) * K;
    y += static_cast<size_t>(blockIdx.y) * M;
    const uint32_t* W = reinterpret_cast<const uint32_t*>(Wb);

    const int lane = threadIdx.x & 63;
    const int slot = lane / LPR;
    const int pl = lane % LPR;
    const int row0 = (blockIdx.x * WAVES + (threadIdx.x >> 6)) * (SUB * R) + slot * R;
    const size_t row_dw = static_cast<size_t>(np) * DW;

    uint32_t wc[R][DW];
    if (pl < np) load_rows<R, DW>(W, row_dw, row0, M, pl, wc);
    stage_x<QT>(x, K, nb, xs4, cb);
    __syncthreads();
    const NibConsts nk = NibConsts::make();
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    for (int p = pl; p < np; p += LPR) {
        uint32_t wn[R][DW];
        if (p + LPR < np) load_rows<R, DW>(W, row_dw, row0, M, p + LPR, wn);
        float xv[64];
        load_xv(xs4, p, xv);
        const float2 c0 = cb[2 * p];
        const float2 c1 = cb[2 * p + 1];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = PairDot<QT>::run(wc[r], xv, c0, c1, acc[r], nk);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < DW; ++i) wc[r][i] = wn[r][i];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = group_sum<LPR>(acc[r]);
    if (pl == LPR - 1) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (row0 + r < M) y[row0 + r] = acc[r];
        }
    }
}

// ---------------------------------------------------------------------------
// Generic kernel: one wave per output row, lanes over blocks, byte loads.
// Handles every shape (odd block counts, K beyond the LDS budget).
template <int QT>
__global__ __launch_bounds__(256) void gemv_generic_kernel(const uint8_t* __restrict__ W,
                                                           const float* __restrict__ x,
                                                           float* __restrict__ y, int M, int K,
                                                           int nb) {
    constexpr int BB = Fmt<QT>::BB;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    x += static_cast<size_t>(blockIdx.y) * K;
    y += static_cast<size_t>(blockIdx.y) * M;
    float acc = 0.0f;
    for (int b = lane; b < nb; b += 64) {
        const uint8_t* blk = W + (static_cast<size_t>(row) * nb + b) * BB;
        const uint16_t dbits = static_cast<uint16_t>(blk[0] | (blk[1] << 8));
        const float d = (float)__builtin_bit_cast(_Float16, dbits);
        const int k0 = b * kQK;
        const int len = min(kQK, K - k0);
        float s = 0.0f;
        float sx = 0.0f;
        for (int i = 0; i < len; ++i) {
            float q;
            if (QT == 1) {
                q = static_cast<float>(static_cast<int8_t>(blk[2 + i]));
            } else {
                const int off = (QT == 2) ? 2 : 4;
                const uint8_t byte = blk[off + (i & 15)];
                const int nib = (i < 16) ? (byte & 15) : (byte >> 4);
                q = static_cast<float>(QT == 2 ? nib - 8 : nib);
            }
            s = __builtin_fmaf(q, x[k0 + i], s);
            sx += x[k0 + i];
        }
        acc = __builtin_fmaf(d, s, acc);
        if (QT == 3) {
            const uint16_t mbits = static_cast<uint16_t>(blk[2] | (blk[3] << 8));
            acc = __builtin_fmaf((float)__builtin_bit_cast(_Float16, mbits), sx, acc);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (lane == 0) y[row] = acc;
}

// ---------------------------------------------------------------------------
// Host-side selection (rules from MI355X measurements of every variant at the
// benchmark shapes).

enum class Kind { Single, Multi, Generic };

struct PairCfg {
    Kind kind;
    int lpr;
    int r;
};

int pair_lds_bytes(int nb) { return (nb / 2) * 256 + nb * 8; }

PairCfg choose_pair(const LinearShape& s) {
    if (s.nb % 2 != 0 || pair_lds_bytes(s.nb) > kMaxPairLdsBytes) return PairCfg{Kind::Generic, 64, 1};
    const int np = s.nb / 2;
    if (np <= 16) return PairCfg{Kind::Single, 16, 1};
    if (np <= 64) return PairCfg{Kind::Single, 64, s.M <= 8192 ? 2 : 1};
    // Longer rows: the widest lane group whose last sweep leaves <= 12.5% idle.
    for (int lpr : {64, 32, 16}) {
        const int iters = (np + lpr - 1) / lpr;
        if (static_cast<double>(np) / (static_cast<double>(lpr) * iters) >= 0.875) return PairCfg{Kind::Multi, lpr, 1};
    }
    return PairCfg{Kind::Multi, 16, 1};
}

template <int QT, int LPR, int R>
hipError_t launch_single_t(const LinearShape& s, const void* w, const float* x, float* y,
                           hipStream_t stream) {
    constexpr int rows_per_group = (64 / LPR) * R;
    const int groups = (s.M + rows_per_group - 1) / rows_per_group;
    int grid = (groups + kWaves - 1) / kWaves;
    if (grid > kPersistentWgs) grid = kPersistentWgs;
    hipLaunchKernelGGL((gemv_single_kernel<QT, LPR, R, kWaves>), dim3(grid, s.rows), dim3(kWaves * 64),
                       pair_lds_bytes(s.nb), stream, static_cast<const uint8_t*>(w), x, y, s.M, s.K, s.nb,
                       groups);
    return hipGetLastError();
}

template <int QT, int LPR>
hipError_t launch_multi_t(const LinearShape& s, const void* w, const float* x, float* y,
                          hipStream_t stream) {
    constexpr int rows_per_wg = kWaves * (64 / LPR);
    dim3 grid((s.M + rows_per_wg - 1) / rows_per_wg, s.rows);
    hipLaunchKernelGGL((gemv_multi_kernel<QT, LPR, 1, kWaves>), grid, dim3(kWaves * 64), pair_lds_bytes(s.nb),
                       stream, static_cast<const uint8_t*>(w), x, y, s.M, s.K, s.nb);
    return hipGetLastError();
}

template <int QT>
hipError_t launch_q(const LinearShape& s, const PairCfg& c, const void* w, const float* x, float* y,
                    hipStream_t stream) {
    if (c.kind == Kind::Single) {
        if (c.lpr == 16) return launch_single_t<QT, 16, 1>(s, w, x, y, stream);
        if (c.r == 2) return launch_single_t<QT, 64, 2>(s, w, x, y, stream);
        return launch_single_t<QT, 64, 1>(s, w, x, y, stream);
    }
    if (c.kind == Kind::Multi) {
        if (c.lpr == 64) return launch_multi_t<QT, 64>(s, w, x, y, stream);
        if (c.lpr == 32) return launch_multi_t<QT, 32>(s, w, x, y, stream);
        return launch_multi_t<QT, 16>(s, w, x, y, stream);
    }
    dim3 grid((s.M + 3) / 4, s.rows);
    hipLaunchKernelGGL((gemv_generic_kernel<QT>), grid, dim3(256), 0, stream, static_cast<const uint8_t*>(w), x,
                       y, s.M, s.K, s.nb);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv(const LinearShape& s, const void* w, const float* x, float* y,
                       hipStream_t stream) {
    const PairCfg c = choose_pair(s);
    switch (s.qtype) {
        case 1: return launch_q<1>(s, c, w, x, y, stream);
        case 2: return launch_q<2>(s, c, w, x, y, stream);
        case 3: return launch_q<3>(s, c, w, x, y, stream);
        default: return hipErrorInvalidValue;
    }
}

const char* gemv_kernel_name(const LinearShape& s) {
    static thread_local char buf[96];
    const char* fmt = s.qtype == 1 ? "q8_0" : s.qtype == 2 ? "q4_0" : "q4_1";
    const PairCfg c = choose_pair(s);
    if (c.kind == Kind::Single) {
        snprintf(buf, sizeof buf, "gemv_single_%s_lpr%d_r%d", fmt, c.lpr, c.r);
    } else if (c.kind == Kind::Multi) {
        snprintf(buf, sizeof buf, "gemv_multi_%s_lpr%d", fmt, c.lpr);
    } else {
        snprintf(buf, sizeof buf, "gemv_generic_%s", fmt);
    }
    return buf;
}

}  // namespace mlq

// Device helpers shared by the decode GEMV kernels (gemv.hip) and the
// persistent sequence kernel (sequence.hip): block formats, x staging into
// LDS, the nibble / byte expansion to exact fp16 integers, the per-pair dot
// product and the DPP row reduction.  Both translation units include this
// file so a row is summed in exactly the same order by either kernel.
#pragma once

#include "mlq_kernels.h"

#include <hip/hip_runtime.h>

#include <cstdint>

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

// Device pointers that the compiler cannot trace to a kernel argument (loaded
// from a descriptor table) are generic; generic accesses become FLAT
// instructions, which count against the LDS counter as well and make every
// wait conservative.  These casts state that the memory is global.
typedef __attribute__((address_space(1))) const uint32_t g_u32;
typedef __attribute__((address_space(1))) const float g_f32;
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const f32x4_t g_f4;
__device__ __forceinline__ g_u32* as_global(const uint32_t* p) { return (g_u32*)p; }
__device__ __forceinline__ g_f32* as_global(const float* p) { return (g_f32*)p; }

constexpr int kMaxPairLdsBytes = 64 * 1024;
constexpr int kWaves = 8;             // waves per workgroup
constexpr int kPersistentWgs = 512;   // ~2 workgroups per CU on a 256-CU MI355X

// LDS of the pair kernels: 256 B of x per pair plus 8 B of constants per block.
inline int pair_lds_bytes(int nb) { return (nb / 2) * 256 + nb * 8; }

// ---------------------------------------------------------------------------
// x staging: one thread per block.  Writes x' (f32, Q4 high halves scaled by
// 1/16) into 16-byte slots swizzled by pair, and per-block constants {c0, c1}:
//   Q8_0: c0 = 1152 * X          Q4_0: c0 = 1024 * S + 8 * X
//   Q4_1: c0 = 1024 * S, c1 = X  with X = sum(x), S = sum(x') over the block.
// Elements past K read as 0, so a partial last block contributes nothing
// (the reference loops only k < K, src/quant.cpp:421-426).
// COHERENT reads x with agent-scope (sc1) loads, which return what another
// workgroup of the same launch stored with agent-scope stores even when this
// XCD's L2 holds an older copy of the line.  Those loads are not cached, so
// they are issued as coalesced 16-byte buffer loads (the buffer's range check
// returns 0 past K) into the pair region of LDS first; each thread then takes
// its block from LDS.  A block's two pair partners (g, g ^ 1) are neighbouring
// lanes of one wave, so every read of the region happens before any write
// that permutes it.
// NORM stages rmsnorm(x) * w instead of x (src/ops.cpp:18-41: mean of
// squares over the K elements, scale = 1 / sqrt(ms + eps), x * scale * w):
// every workgroup normalises its own copy.  Each thread loads its block's x
// and w together, the squares are reduced over the workgroup once (every
// thread of the block takes part; NORM needs nb <= blockDim, one block per
// thread), and the values are scaled from registers -- x is read once.
template <int QT, bool COHERENT = false, bool NORM = false>
__device__ __forceinline__ void stage_x(const float* __restrict__ x, int K, int nb,
                                        float4* __restrict__ xs4, float2* __restrict__ cb,
                                        const float* __restrict__ norm_w = nullptr, float norm_eps = 0.0f) {
    if (COHERENT) {
        constexpr int kAgentScope = 16;  // sc1 cache policy
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(x), static_cast<short>(0), K * 4, 0x00020000);
        const int n4 = nb * (kQK / 4);
        const int k4 = K / 4;
        for (int i = threadIdx.x; i < n4; i += blockDim.x) {
            float4 v;
            if (i < k4) {
                v = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, i * 16, 0, kAgentScope));
            } else {
                v.x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, i * 16, 0, kAgentScope));
                v.y = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, i * 16 + 4, 0, kAgentScope));
                v.z = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, i * 16 + 8, 0, kAgentScope));
                v.w = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, i * 16 + 12, 0, kAgentScope));
            }
            xs4[i] = v;
        }
        __syncthreads();
    }
    for (int g0 = 0; g0 < nb; g0 += blockDim.x) {
        const int g = NORM ? min(static_cast<int>(threadIdx.x), nb - 1) : g0 + static_cast<int>(threadIdx.x);
        if (!NORM && g >= nb) break;
        float v[32];
        const int k0 = g * kQK;
        if (COHERENT) {
            const float4* rb = xs4 + g * 8;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 f = rb[i];
                v[4 * i] = f.x;
                v[4 * i + 1] = f.y;
                v[4 * i + 2] = f.z;
                v[4 * i + 3] = f.w;
            }
        } else if (k0 + kQK <= K && (reinterpret_cast<uintptr_t>(x + k0) & 15u) == 0) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const f32x4_t fv = ((g_f4*)(x + k0))[i];
                const float4 f = make_float4(fv.x, fv.y, fv.z, fv.w);
                v[4 * i] = f.x;
                v[4 * i + 1] = f.y;
                v[4 * i + 2] = f.z;
                v[4 * i + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i) v[i] = (k0 + i < K) ? as_global(x)[k0 + i] : 0.0f;
        }
        if (NORM) {
            float w[32];
            if (k0 + kQK <= K && (reinterpret_cast<uintptr_t>(norm_w + k0) & 15u) == 0) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const f32x4_t fv = ((g_f4*)(norm_w + k0))[i];
                    w[4 * i] = fv.x;
                    w[4 * i + 1] = fv.y;
                    w[4 * i + 2] = fv.z;
                    w[4 * i + 3] = fv.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 32; ++i) w[i] = (k0 + i < K) ? as_global(norm_w)[k0 + i] : 0.0f;
            }
            // Squares of this thread's block (a repeated last block counts 0).
            float ss = 0.0f;
            if (static_cast<int>(threadIdx.x) < nb) {
#pragma unroll
                for (int i = 0; i < 32; ++i) ss += v[i] * v[i];
            }
            __shared__ float part[16];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
            if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
            __syncthreads();
            float t = part[0];
            for (int i = 1; i < static_cast<int>(blockDim.x >> 6); ++i) t += part[i];
            const float scale = 1.0f / sqrtf(t / static_cast<float>(K) + norm_eps);
#pragma unroll
            for (int i = 0; i < 32; ++i) v[i] = v[i] * scale * w[i];
            if (static_cast<int>(threadIdx.x) >= nb) break;
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

}  // namespace
}  // namespace mlq

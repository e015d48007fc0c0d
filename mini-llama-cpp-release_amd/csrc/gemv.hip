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
//  * x is staged once per workgroup in LDS as block-scaled integer limbs
//    with per-block constants (four threads per block, buffer loads whose
//    range check reads elements past K as 0); 16-byte LDS slots are
//    XOR-swizzled by pair so a wave's reads spread over the banks.
//  * Every lane requests its first W pair(s) before staging x, so the W
//    latency overlaps the staging and the barrier.
//  * "single" kernel (row of at most LPR pairs): each lane keeps its pair's
//    x limbs in VGPRs and the workgroups are persistent (one per CU), each
//    wave walking its row groups with a ring of the next 2-3 groups' W
//    requests in flight.  "multi" kernel (longer rows): one row group per wave,
//    x read from LDS per pair, next pair's W requested before the current one
//    is computed.
//  * Row sums are reduced across the slot's lanes with DPP adds (quad_perm,
//    row mirrors, row_bcast), all VALU, no LDS round trip.
//
// Arithmetic (integer dot products, exact per block; gemv_device.h): x is
// written per block as s_b * X with X a 16-bit (Q4) or 23-bit (Q8_0) integer
// in int8 limbs, the stored nibbles / bytes meet the limbs in v_dot4 (4
// products per instruction, ~1.0 VALU op per Q4 weight and ~0.8 per Q8_0
// weight including the unpacking), and each block's exact integer sum is
// scaled by d * s_b into the f32 row sum.

// Rows with an odd block count (pairs would straddle rows) and very long rows
// go to a simple one-wave-per-row kernel with byte loads.

#include "gemv_device.h"
#include "pick_key.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

namespace mlq {
namespace {

// Call of a group that owns launch row `row` (calls are in row order).
__device__ __forceinline__ int group_call(const GemvGroup& g, int row) {
    int k = 0;
#pragma unroll
    for (int j = 1; j < kGroupMaxCalls; ++j) k = (j < g.ncalls && row >= g.row_begin[j]) ? j : k;
    return k;
}

__device__ __forceinline__ const uint32_t* group_row(const GemvGroup& g, int row, size_t row_dw) {
    const void* w = g.W[0];
    int rb = 0;
#pragma unroll
    for (int j = 1; j < kGroupMaxCalls; ++j) {
        if (j < g.ncalls && row >= g.row_begin[j]) {
            w = g.W[j];
            rb = g.row_begin[j];
        }
    }
    return static_cast<const uint32_t*>(w) + static_cast<size_t>(row - rb) * row_dw;
}

// y of launch row `row` for batch row `b` (each call's y is [rows][M_j]).
__device__ __forceinline__ float* group_y(const GemvGroup& g, int row, int M, int b) {
    float* y = g.y[0];
    int rb = 0;
    int re = g.ncalls > 1 ? g.row_begin[1] : M;
#pragma unroll
    for (int j = 1; j < kGroupMaxCalls; ++j) {
        if (j < g.ncalls && row >= g.row_begin[j]) {
            y = g.y[j];
            rb = g.row_begin[j];
            re = j + 1 < g.ncalls ? g.row_begin[j + 1] : M;
        }
    }
    return y + static_cast<size_t>(b) * (re - rb) + (row - rb);
}

// The call of a group that holds row `row`, kept in scalar registers by a
// wave that visits rows in increasing order: the lookup runs only when a row
// passes the current call's end.  y is the call's y of batch row b.
struct CallCursor {
    const uint32_t* w;
    float* y;
    int rb, re;  // the call's launch rows [rb, re)
    __device__ __forceinline__ void seek(const GemvGroup& g, int M, int b, int row) {
        const void* W = g.W[0];
        float* Y = g.y[0];
        int r0 = 0;
        int r1 = g.ncalls > 1 ? g.row_begin[1] : M;
#pragma unroll
        for (int j = 1; j < kGroupMaxCalls; ++j) {
            if (j < g.ncalls && row >= g.row_begin[j]) {
                W = g.W[j];
                Y = g.y[j];
                r0 = g.row_begin[j];
                r1 = j + 1 < g.ncalls ? g.row_begin[j + 1] : M;
            }
        }
        w = static_cast<const uint32_t*>(W);
        y = Y + static_cast<size_t>(b) * (r1 - r0);
        rb = r0;
        re = r1;
    }
};

// Folds every lane's key into the launch's result; called once by every
// thread of every workgroup.  The workgroup's best key goes to its group slot
// with one atomic max, then the workgroup arrives; the last arrival of the
// last group swaps the slots back to zero and writes the token.  Atomics are
// agent-scope and each returns before the next is issued, so every max is
// performed before the arrival that counts it.  Nothing waits on another
// workgroup: the launch always drains.
template <int WAVES>
__device__ __forceinline__ void pick_finish(PickState* ps, int32_t* token, unsigned long long best) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long other = __shfl_xor(best, o, 64);
        best = other > best ? other : best;
    }
    __shared__ unsigned long long wave_best[WAVES];
    if ((threadIdx.x & 63) == 0) wave_best[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x != 0) return;
    unsigned long long b = wave_best[0];
#pragma unroll
    for (int i = 1; i < WAVES; ++i) b = wave_best[i] > b ? wave_best[i] : b;
    const unsigned j = blockIdx.x % kPickGroups;
    const unsigned in_group = (gridDim.x - j + kPickGroups - 1) / kPickGroups;
    const unsigned groups = gridDim.x < kPickGroups ? gridDim.x : kPickGroups;
    const unsigned long long before =
        __hip_atomic_fetch_max(&ps->key[j][0], b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::"v"(before) : "memory");
    if (__hip_atomic_fetch_add(&ps->sub[j][0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != in_group - 1) return;
    __hip_atomic_store(&ps->sub[j][0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (__hip_atomic_fetch_add(&ps->top[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != groups - 1) return;
    __hip_atomic_store(&ps->top[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Every slot, unrolled: slots past `groups` are never written and hold 0,
    // and issuing all exchanges before using any costs one round trip.
    unsigned long long v[kPickGroups];
#pragma unroll
    for (int i = 0; i < kPickGroups; ++i)
        v[i] = __hip_atomic_exchange(&ps->key[i][0], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned long long k = 0;
#pragma unroll
    for (int i = 0; i < kPickGroups; ++i) k = v[i] > k ? v[i] : k;
    *token = pick_token(k);
}

// Launch modes of the GEMV kernels.  The plain mode stores y = W x; the pick
// modes also fold the greedy pick over y (y may be null); the norm modes
// stage rmsnorm(x) * norm_w instead of x (the decode step's RMSNorm, done by
// each workgroup on its own copy of x); the accumulate mode adds the rows into
// y (the decode step's residual add: y is the residual stream, x another
// buffer); the GLU mode (single kernel only) takes the gate and up weights as
// the group's two calls of equal rows, computes row i of both in the same
// lanes and stores silu(gate_i) * up_i into y[0] (the SwiGLU of the decode
// step, with the FFN RMSNorm staged).
constexpr int kModePlain = 0;
constexpr int kModePick = 1;
constexpr int kModeNorm = 2;
constexpr int kModeNormPick = 3;
constexpr int kModeAcc = 4;
constexpr int kModeNormGlu = 5;
template <int MODE> struct Mode {
    static constexpr bool pick = MODE == kModePick || MODE == kModeNormPick;
    static constexpr bool norm = MODE == kModeNorm || MODE == kModeNormPick || MODE == kModeNormGlu;
    static constexpr bool acc = MODE == kModeAcc;
    static constexpr bool glu = MODE == kModeNormGlu;
};

// Row groups in flight per wave in the single kernel (its register ring).
// One workgroup of 8 waves per CU (2 waves per SIMD, up to 256 VGPRs) with a
// deep ring measured faster on MI355X than two workgroups per CU with one
// group in flight: x is staged half as often and more weight bytes are in
// flight per CU.
template <int QT> struct SingleDepth { static constexpr int D = QT == 1 ? 2 : 3; };

// Rows of at most LPR pairs: x in VGPRs, persistent over row groups.  Wave w
// takes groups w, w + W, ... (W waves in the grid), group i being rows
// i * SUB + slot; its ring slot k holds groups k, k + D, k + 2D, ... of the
// wave: a slot is computed, then refilled in place with the group D ahead.
// The first PRE ring slots are requested with x, before x is quantized; the
// rest right after (issuing requests stalls once the memory system is
// saturated, and x's quantization waits behind them).
template <int QT, int LPR, int WAVES, int D, int MODE, int PRE = D>
__global__ __launch_bounds__(WAVES * 64, 2) void gemv_single_kernel(const GemvGroup g, const float* __restrict__ x,
                                                                   int M, int K, int nb, int groups) {
    constexpr int DW = Fmt<QT>::DW;
    constexpr int SUB = 64 / LPR;
    extern __shared__ float4 lds4[];
    const int np = nb >> 1;
    uint32_t* xl = reinterpret_cast<uint32_t*>(lds4);
    float4* xc = reinterpret_cast<float4*>(xl + np * XLimbs<QT>::PAIR_DW);
    x += static_cast<size_t>(blockIdx.y) * K;

    const int lane = threadIdx.x & 63;
    const int slot = lane / LPR;
    const int pl = lane % LPR;
    const bool active = pl < np;
    const int p = active ? pl : 0;
    const size_t row_dw = static_cast<size_t>(np) * DW;
    const int gstride = gridDim.x * WAVES;
    const int g0 = blockIdx.x * WAVES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nu = g0 < groups ? (groups - g0 + gstride - 1) / gstride : 0;  // groups of this wave

    // Every weight request is unconditional (a group past the end re-reads the
    // last one; its result is dropped): a guarded request makes the compiler
    // wait for it right away, which serialises the prefetch.
    constexpr bool PICK = Mode<MODE>::pick;
    constexpr bool ACC = Mode<MODE>::acc;
    constexpr bool GLU = Mode<MODE>::glu;
    uint32_t wq[D][DW];
    uint32_t uq[GLU ? D : 1][DW];  // GLU mode: the up rows of the ring's units
    float rq[D];  // accumulate mode: the residual of the slot's row, requested with its weights
    // Units are requested (rq_cur) and stored (st_cur) in increasing row order.
    CallCursor rq_cur, st_cur;
    rq_cur.seek(g, M, blockIdx.y, 0);
    st_cur = rq_cur;
    auto request_glu = [&](int gi, int k) {
        const size_t row = static_cast<size_t>(min(min(gi, groups - 1) * SUB + slot, M - 1));
        const uint32_t* gs = static_cast<const uint32_t*>(g.W[0]) + row * row_dw + static_cast<size_t>(p) * DW;
        const uint32_t* us = static_cast<const uint32_t*>(g.W[1]) + row * row_dw + static_cast<size_t>(p) * DW;
#pragma unroll
        for (int i = 0; i < DW; ++i) wq[k][i] = gs[i];
#pragma unroll
        for (int i = 0; i < DW; ++i) uq[GLU ? k : 0][i] = us[i];
    };
    auto request = [&](int gi, uint32_t (&w)[DW], float& r) {
        const int r0 = min(gi, groups - 1) * SUB;
        if (r0 >= rq_cur.re) rq_cur.seek(g, M, blockIdx.y, r0);
        const uint32_t* src;
        const float* res;
        if (r0 + SUB <= rq_cur.re) {  // the unit's rows lie in one call
            src = rq_cur.w + static_cast<size_t>(r0 + slot - rq_cur.rb) * row_dw;
            res = rq_cur.y + (r0 + slot - rq_cur.rb);
        } else {
            const int row = min(r0 + slot, M - 1);
            src = group_row(g, row, row_dw);
            res = group_y(g, row, M, blockIdx.y);
        }
        src += static_cast<size_t>(p) * DW;
#pragma unroll
        for (int i = 0; i < DW; ++i) w[i] = src[i];
        if (ACC) r = *res;
    };
    // nb <= 2 * 64 pairs <= blockDim / 4: one round of x loads
    static_assert(PRE >= 1 && PRE <= D, "ring slots requested before staging");
    auto request_slot = [&](int k) {
        if (GLU) {
            request_glu(g0 + k * gstride, k);
        } else {
            request(g0 + k * gstride, wq[k], rq[k]);
        }
    };
    // x first: every wave of the workgroup has issued its x loads before any
    // wave requests weights (a bare barrier, no memory wait), so the CU's
    // memory queue serves x ahead of the weight misses.  With the weights
    // first, x came back only after ~3 us at the start of a launch on MI355X
    // (queued behind other waves' misses); x first: the 7B sweep 1028 -> 1000 us.
    stage_x<QT, false, Mode<MODE>::norm, 1, true>(x, K, nb, xl, xc, g.norm_w, g.norm_eps, [&] {
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int k = 0; k < PRE; ++k) request_slot(k);
    });
#pragma unroll
    for (int k = PRE; k < D; ++k) request_slot(k);
    uint32_t xq[XLimbs<QT>::PAIR_DW];
    float4 c0, c1;
    load_xq<QT>(xl, xc, p, xq, c0, c1);
    const bool store_y = !PICK || g.y[0] != nullptr;
    unsigned long long best = 0;

    int gi = g0;
    auto step_glu = [&](int k) {
        const float vg = PairDot<QT>::run(wq[k], xq, c0, c1, 0.0f);
        const float vu = PairDot<QT>::run(uq[GLU ? k : 0], xq, c0, c1, 0.0f);
        request_glu(gi + D * gstride, k);
        const float a = group_sum<LPR>(active ? vg : 0.0f);
        const float b = group_sum<LPR>(active ? vu : 0.0f);
        const int row = gi * SUB + slot;
        if (pl == LPR - 1 && row < M) {
            const float sig = 1.0f / (1.0f + expf(-a));  // src/ops.cpp:72-107
            g.y[0][static_cast<size_t>(blockIdx.y) * M + row] = a * sig * b;
        }
        gi += gstride;
    };
    auto step = [&](uint32_t (&w)[DW], float& r) {
        const float v = PairDot<QT>::run(w, xq, c0, c1, 0.0f);  // inactive lanes hold pair 0: dropped
        const float res = r;
        request(gi + D * gstride, w, r);
        const float acc = group_sum<LPR>(active ? v : 0.0f);
        const int r0 = gi * SUB;
        const int row = r0 + slot;
        if (r0 >= st_cur.re && r0 < M) st_cur.seek(g, M, blockIdx.y, r0);
        if (pl == LPR - 1 && row < M) {
            if (store_y) {
                float* yp = r0 + SUB <= st_cur.re ? st_cur.y + (row - st_cur.rb) : group_y(g, row, M, blockIdx.y);
                *yp = ACC ? res + acc : acc;
            }
            if (PICK) {
                const unsigned long long k = pick_key(acc, row);
                best = k > best ? k : best;
            }
        }
        gi += gstride;
    };
    int u = 0;
    if (GLU) {
        for (; u + D <= nu; u += D) {
#pragma unroll
            for (int k = 0; k < D; ++k) step_glu(k);
        }
#pragma unroll
        for (int k = 0; k < D; ++k)
            if (u + k < nu) step_glu(k);
        return;
    }
    for (; u + D <= nu; u += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) step(wq[k], rq[k]);
    }
#pragma unroll
    for (int k = 0; k < D; ++k)
        if (u + k < nu) step(wq[k], rq[k]);
    if (PICK) pick_finish<WAVES>(g.pick, g.token, best);
}

// Rows of more than LPR pairs: x from LDS per pair.  Wave w takes row items
// w, w + W, ... (W waves in the grid; item i being rows i * SUB + slot), each
// walked in chunks c = 0 .. nch-1 (pair c * LPR + pl of every lane; lanes past
// the row keep their sum).  A ring of D units (item, chunk) of weight requests
// is in flight per wave, refilled in place; the first PRE of them are
// requested with x, the rest once x is staged.  Workgroup size, grid cap, D
// and PRE come from MI355X measurements (launch_multi_t).

template <int QT, int LPR, int WAVES, int D, int MODE, int PRE = D>
__global__ __launch_bounds__(WAVES * 64) void gemv_multi_kernel(const GemvGroup g, const float* __restrict__ x,
                                                               int M, int K, int nb, int items) {
    constexpr int DW = Fmt<QT>::DW;
    constexpr int SUB = 64 / LPR;
    extern __shared__ float4 lds4[];
    const int np = nb >> 1;
    uint32_t* xl = reinterpret_cast<uint32_t*>(lds4);
    float4* xc = reinterpret_cast<float4*>(xl + np * XLimbs<QT>::PAIR_DW);
    x += static_cast<size_t>(blockIdx.y) * K;

    const int lane = threadIdx.x & 63;
    const int slot = lane / LPR;
    const int pl = lane % LPR;
    const size_t row_dw = static_cast<size_t>(np) * DW;
    const int GW = gridDim.x * WAVES;
    const int gw = blockIdx.x * WAVES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nch = (np + LPR - 1) / LPR;
    const int nit = gw < items ? (items - gw + GW - 1) / GW : 0;
    const int nu = nit * nch;

    // Requests are unconditional (past the row: the last pair; past the
    // items: the last item) so the prefetch is never waited for early.
    constexpr bool PICK = Mode<MODE>::pick;
    constexpr bool ACC = Mode<MODE>::acc;
    uint32_t wq[D][DW];
    float rq[D];  // accumulate mode: the residual of the unit's row
    CallCursor rq_cur, st_cur;
    rq_cur.seek(g, M, blockIdx.y, 0);
    st_cur = rq_cur;
    int pit = gw, pc = 0;  // the next unit to request
    auto request = [&](uint32_t (&w)[DW], float& r) {
        const int r0 = min(pit, items - 1) * SUB;
        if (r0 >= rq_cur.re) rq_cur.seek(g, M, blockIdx.y, r0);
        const uint32_t* src;
        const float* res;
        if (r0 + SUB <= rq_cur.re) {
            src = rq_cur.w + static_cast<size_t>(r0 + slot - rq_cur.rb) * row_dw;
            res = rq_cur.y + (r0 + slot - rq_cur.rb);
        } else {
            const int row = min(r0 + slot, M - 1);
            src = group_row(g, row, row_dw);
            res = group_y(g, row, M, blockIdx.y);
        }
        src += static_cast<size_t>(min(pc * LPR + pl, np - 1)) * DW;
#pragma unroll
        for (int i = 0; i < DW; ++i) w[i] = src[i];
        if (ACC) r = *res;
        if (++pc == nch) {
            pc = 0;
            pit += GW;
        }
    };
    static_assert(PRE >= 1 && PRE <= D, "ring units requested before staging");
    // x first (see the single kernel): every thread reaches this callback once.
    stage_x_fit<QT, false, Mode<MODE>::norm>(x, K, nb, xl, xc, g.norm_w, g.norm_eps, [&] {
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int k = 0; k < PRE; ++k) request(wq[k], rq[k]);
    });
#pragma unroll
    for (int k = PRE; k < D; ++k) request(wq[k], rq[k]);
    const bool store_y = !PICK || g.y[0] != nullptr;
    unsigned long long best = 0;
    int it = gw, c = 0;
    float acc = 0.0f;
    auto step = [&](uint32_t (&w)[DW], float& r) {
        const int p = c * LPR + pl;
        uint32_t xq[XLimbs<QT>::PAIR_DW];
        float4 c0, c1;
        load_xq<QT>(xl, xc, min(p, np - 1), xq, c0, c1);
        const float a = PairDot<QT>::run(w, xq, c0, c1, acc);
        acc = p < np ? a : acc;
        const float res = r;
        request(w, r);
        if (++c == nch) {
            const float t = group_sum<LPR>(acc);
            const int r0 = it * SUB;
            const int row = r0 + slot;
            if (r0 >= st_cur.re && r0 < M) st_cur.seek(g, M, blockIdx.y, r0);
            if (pl == LPR - 1 && row < M) {
                if (store_y) {
                    float* yp = r0 + SUB <= st_cur.re ? st_cur.y + (row - st_cur.rb) : group_y(g, row, M, blockIdx.y);
                    *yp = ACC ? res + t : t;
                }
                if (PICK) {
                    const unsigned long long k = pick_key(t, row);
                    best = k > best ? k : best;
                }
            }
            acc = 0.0f;
            c = 0;
            it += GW;
        }
    };
    int u = 0;
    for (; u + D <= nu; u += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) step(wq[k], rq[k]);
    }
#pragma unroll
    for (int k = 0; k < D; ++k)
        if (u + k < nu) step(wq[k], rq[k]);
    if (PICK) pick_finish<WAVES>(g.pick, g.token, best);
}

// ---------------------------------------------------------------------------
// Generic kernel: one wave per output row, lanes over blocks, byte loads.
// Handles every shape (odd block counts, K beyond the LDS budget).
template <int QT, int MODE>
__global__ __launch_bounds__(256) void gemv_generic_kernel(const GemvGroup g, const float* __restrict__ x,
                                                           int M, int K, int nb) {
    constexpr bool PICK = Mode<MODE>::pick;
    constexpr bool NORM = Mode<MODE>::norm;
    constexpr bool ACC = Mode<MODE>::acc;
    constexpr int BB = Fmt<QT>::BB;
    const int lane = threadIdx.x & 63;
    const int wave_row = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // A wave past the last row computes row M-1 again and drops it (every
    // wave of a picking workgroup has to reach the final fold).
    const bool live = wave_row < M;
    const int row = live ? wave_row : M - 1;
    x += static_cast<size_t>(blockIdx.y) * K;
    const int k = group_call(g, row);
    const uint8_t* W = static_cast<const uint8_t*>(g.W[k]) +
                       static_cast<size_t>(row - g.row_begin[k]) * nb * BB;
    const float res = ACC ? *group_y(g, row, M, blockIdx.y) : 0.0f;
    // Norm mode: each wave reduces the squares of x itself and reads
    // x * scale * w on the fly.
    float scale = 1.0f;
    if (NORM) {
        float ss = 0.0f;
        for (int i = lane; i < K; i += 64) ss += x[i] * x[i];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        scale = 1.0f / sqrtf(ss / static_cast<float>(K) + g.norm_eps);
    }
    auto xat = [&](int i) { return NORM ? x[i] * scale * g.norm_w[i] : x[i]; };
    float acc = 0.0f;
    for (int b = lane; b < nb; b += 64) {
        const uint8_t* blk = W + static_cast<size_t>(b) * BB;
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
            const float xi = xat(k0 + i);
            s = __builtin_fmaf(q, xi, s);
            sx += xi;
        }
        acc = __builtin_fmaf(d, s, acc);
        if (QT == 3) {
            const uint16_t mbits = static_cast<uint16_t>(blk[2] | (blk[3] << 8));
            acc = __builtin_fmaf((float)__builtin_bit_cast(_Float16, mbits), sx, acc);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (lane == 0 && live && (!PICK || g.y[0] != nullptr)) *group_y(g, row, M, blockIdx.y) = ACC ? res + acc : acc;
    if (PICK) pick_finish<4>(g.pick, g.token, lane == 0 && live ? pick_key(acc, row) : 0ull);
}

// ---------------------------------------------------------------------------
// Host-side selection (rules from MI355X measurements of every variant at the
// benchmark shapes).

enum class Kind { Single, Multi, Generic };

struct PairCfg {
    Kind kind;
    int lpr;
};

PairCfg choose_pair(const LinearShape& s) {
    if (s.nb % 2 != 0 || pair_lds_bytes(s.qtype, s.nb) > kMaxPairLdsBytes) return PairCfg{Kind::Generic, 64};
    const int np = s.nb / 2;
    if (np <= 16) return PairCfg{Kind::Single, 16};
    if (np <= 64) return PairCfg{Kind::Single, 64};
    // Longer rows: the widest lane group whose last sweep leaves <= 12.5% idle.
    for (int lpr : {64, 32, 16}) {
        const int iters = (np + lpr - 1) / lpr;
        if (static_cast<double>(np) / (static_cast<double>(lpr) * iters) >= 0.875) return PairCfg{Kind::Multi, lpr};
    }
    return PairCfg{Kind::Multi, 16};
}

template <int QT, int LPR, int MODE>
hipError_t launch_single_t(const LinearShape& s, const GemvGroup& g, const float* x, hipStream_t stream) {
    constexpr int rows_per_group = 64 / LPR;
    constexpr int D = SingleDepth<QT>::D;
    const int groups = (s.M + rows_per_group - 1) / rows_per_group;
    int grid = (groups + kWaves - 1) / kWaves;
    if (grid > kPersistentWgs) grid = kPersistentWgs;
    // Ring slots requested before x is quantized (MI355X, Q4_0 x 4096, cold
    // weights): one when a wave has at most two groups (4096 rows: 5.55 ->
    // 5.30 us), all but one for longer runs (12288 rows: 8.39 -> 8.26 us).
    // Q8_0's two-slot ring: one ahead of x (since x is loaded ahead of the
    // weights: 4864 x 896 3.96 -> 3.81 us, the 4096-row shapes unchanged).
    const int per_wave = (groups + grid * kWaves - 1) / (grid * kWaves);
    auto kern = D < 3 ? gemv_single_kernel<QT, LPR, kWaves, D, MODE, 1>
                      : per_wave <= 2 ? gemv_single_kernel<QT, LPR, kWaves, D, MODE, 1>
                                      : gemv_single_kernel<QT, LPR, kWaves, D, MODE, (D > 1 ? D - 1 : 1)>;
    hipLaunchKernelGGL(kern, dim3(grid, s.rows), dim3(kWaves * 64), pair_lds_bytes(QT, s.nb), stream, g, x, s.M, s.K,
                       s.nb, groups);
    return hipGetLastError();
}

template <int QT, int LPR, int MODE>
hipError_t launch_multi_t(const LinearShape& s, const GemvGroup& g, const float* x, hipStream_t stream) {
    constexpr int sub = 64 / LPR;
    const int items = (s.M + sub - 1) / sub;
    auto go = [&](auto kernel, int waves, int cap) {
        int grid = (items + waves - 1) / waves;
        if (grid > cap) grid = cap;
        hipLaunchKernelGGL(kernel, dim3(grid, s.rows), dim3(waves * 64), pair_lds_bytes(QT, s.nb), stream, g, x, s.M,
                           s.K, s.nb, items);
        return hipGetLastError();
    };
    // Few rows: small workgroups spread over more CUs, three units in flight.
    // Many rows: Q4 one persistent 16-wave workgroup per CU (x staged once
    // per CU) with two units in flight, Q8_0 8-wave workgroups with one item
    // per wave.
    if (items < 2048) return go(gemv_multi_kernel<QT, LPR, 4, 3, MODE>, 4, 1 << 20);
    if (QT == 1) return go(gemv_multi_kernel<QT, LPR, 8, 1, MODE>, 8, 1 << 20);
    // One of the two units requested with x, the other once x is staged
    // (4096 x 11008 Q4_0, cold weights: 9.50 -> 9.34 us).
    return go(gemv_multi_kernel<QT, LPR, 16, 2, MODE, 1>, 16, kPersistentWgs);
}

template <int QT, int MODE>
hipError_t launch_q(const LinearShape& s, const PairCfg& c, const GemvGroup& g, const float* x,
                    hipStream_t stream) {
    if (c.kind == Kind::Single) {
        if (c.lpr == 16) return launch_single_t<QT, 16, MODE>(s, g, x, stream);
        return launch_single_t<QT, 64, MODE>(s, g, x, stream);
    }
    if (c.kind == Kind::Multi) {
        if (c.lpr == 64) return launch_multi_t<QT, 64, MODE>(s, g, x, stream);
        if (c.lpr == 32) return launch_multi_t<QT, 32, MODE>(s, g, x, stream);
        return launch_multi_t<QT, 16, MODE>(s, g, x, stream);
    }
    dim3 grid((s.M + 3) / 4, s.rows);
    hipLaunchKernelGGL((gemv_generic_kernel<QT, MODE>), grid, dim3(256), 0, stream, g, x, s.M, s.K, s.nb);
    return hipGetLastError();
}

template <int MODE>
hipError_t launch_mode(const LinearShape& s, const GemvGroup& g, const float* x, hipStream_t stream) {
    const PairCfg c = choose_pair(s);
    switch (s.qtype) {
        case 1: return launch_q<1, MODE>(s, c, g, x, stream);
        case 2: return launch_q<2, MODE>(s, c, g, x, stream);
        case 3: return launch_q<3, MODE>(s, c, g, x, stream);
        default: return hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------------------
// Measurement kernel (not a GEMV): the weight stream of a grouped decode GEMV
// launch with no arithmetic.  The grid (one persistent workgroup of 8 waves
// per CU), the work units (row item x chunk of LPR pairs, each lane one pair
// of 9 / 17 / 10 dwords), the dealing of items to waves and the ring of D
// units requested ahead are those of the GEMV kernels; each lane folds the
// dwords it loads into one XOR, stored at the end so no load is dropped.  Its
// time is the floor a GEMV launch of that shape pays for launching and for
// streaming its weights.
template <int QT, int LPR, int D>
__global__ __launch_bounds__(kWaves * 64, 2) void stream_floor_kernel(const GemvGroup g, int M, int nb, int items,
                                                                      uint32_t* __restrict__ sink) {
    constexpr int DW = Fmt<QT>::DW;
    constexpr int SUB = 64 / LPR;
    const int np = nb >> 1;
    const int nch = (np + LPR - 1) / LPR;
    const int lane = threadIdx.x & 63;
    const int slot = lane / LPR;
    const int pl = lane % LPR;
    const size_t row_dw = static_cast<size_t>(np) * DW;
    const int GW = gridDim.x * kWaves;
    const int gw = blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nu = gw < items ? (items - gw + GW - 1) / GW * nch : 0;
    int pit = gw, pc = 0;  // the next unit to request (past the end: the last one again)
    auto request = [&](uint32_t (&w)[DW]) {
        const int row = min(min(pit, items - 1) * SUB + slot, M - 1);
        const uint32_t* src = group_row(g, row, row_dw) + static_cast<size_t>(min(pc * LPR + pl, np - 1)) * DW;
#pragma unroll
        for (int i = 0; i < DW; ++i) w[i] = src[i];
        if (++pc == nch) {
            pc = 0;
            pit += GW;
        }
    };
    uint32_t wq[D][DW];
#pragma unroll
    for (int k = 0; k < D; ++k) request(wq[k]);
    uint32_t acc = 0;
    auto step = [&](uint32_t (&w)[DW]) {
#pragma unroll
        for (int i = 0; i < DW; ++i) acc ^= w[i];
        request(w);
    };
    int u = 0;
    for (; u + D <= nu; u += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) step(wq[k]);
    }
#pragma unroll
    for (int k = 0; k < D; ++k)
        if (u + k < nu) step(wq[k]);
    sink[(static_cast<size_t>(gw) * 64 + lane) & (kFloorSinkWords - 1)] = acc;
}

// Measurement kernels (not GEMVs) that take a GEMV launch's floor apart:
// probe_empty_kernel is the launch alone (the floor's grid, no work);
// probe_load_kernel streams the same weights with the plainest pattern: each
// call's weight bytes as 16-byte units, thread t of T reading units t, t + T,
// ... eight at a time, folded into one XOR (a tail of under 16 bytes per call
// is not read).
__global__ __launch_bounds__(kWaves * 64) void probe_empty_kernel(uint32_t* __restrict__ sink) {
    (void)sink;
}

typedef uint32_t probe_u4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kWaves * 64) void probe_load_kernel(const GemvGroup g, int M, size_t row_bytes,
                                                                 uint32_t* __restrict__ sink) {
    const size_t T = static_cast<size_t>(gridDim.x) * blockDim.x;
    const size_t t = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    probe_u4 acc{0u, 0u, 0u, 0u};
    for (int j = 0; j < g.ncalls; ++j) {
        const int r0 = g.row_begin[j];
        const int r1 = j + 1 < g.ncalls ? g.row_begin[j + 1] : M;
        const size_t units = static_cast<size_t>(r1 - r0) * row_bytes / 16;
        const probe_u4* w = static_cast<const probe_u4*>(g.W[j]);
        for (size_t u = t; u < units; u += 8 * T) {
            probe_u4 v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = u + k * T < units ? w[u + k * T] : probe_u4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int k = 0; k < 8; ++k) acc ^= v[k];
        }
    }
    sink[t & (kFloorSinkWords - 1)] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

// f32 GEMV: the reference's arithmetic (src/quant.cpp:413-429: each weight
// dequantized to f32, w = d * (q - 8), d * q or d * q + m, then an f32
// multiply-add with x), for pricing the integer path against it.  Work units
// as in the multi kernel: a wave takes row r and chunk c of 64 pairs, lane l
// pair 64 c + l, and rows w, w + W, ...; D units' weights are requested ahead.
// x is staged in LDS as f32 with its 16-byte slots XOR-swizzled by pair, so
// that the 64 lanes, each reading its own pair's 64 elements, spread over the
// banks.  Each lane sums its elements in k order with fused multiply-adds; the
// row sum is the lanes' sums added by a butterfly.
typedef float gf32x4 __attribute__((ext_vector_type(4)));

template <int QT, int D>
__global__ __launch_bounds__(512) void gemv_f32_kernel(const GemvGroup g, const float* __restrict__ x, int M, int K,
                                                       int nb) {
    constexpr int DW = Fmt<QT>::DW;
    extern __shared__ gf32x4 xs4[];  // [np][16] slots
    const int np = nb >> 1;
    for (int v = threadIdx.x; v < np * 16; v += blockDim.x) {
        const int p = v >> 4, sl = v & 15;
        const int k0 = 64 * p + 4 * sl;
        gf32x4 f;
        for (int i = 0; i < 4; ++i) f[i] = k0 + i < K ? x[k0 + i] : 0.0f;
        xs4[16 * p + (sl ^ (p & 15))] = f;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int W = gridDim.x * 8;
    const int gw = blockIdx.x * 8 + (threadIdx.x >> 6);
    const int nch = (np + 63) >> 6;
    const int rows_w = gw < M ? (M - gw + W - 1) / W : 0;
    const int nu = rows_w * nch;
    if (nu == 0) return;
    const size_t row_dw = static_cast<size_t>(np) * DW;
    int pr = 0, pc = 0;  // the next unit to request (past the end: the last one again)
    auto request = [&](uint32_t (&w)[DW]) {
        const int row = gw + W * min(pr, rows_w - 1);
        const int p = min(min(pc, nch - 1) * 64 + lane, np - 1);
        const uint32_t* src = group_row(g, row, row_dw) + static_cast<size_t>(p) * DW;
#pragma unroll
        for (int i = 0; i < DW; ++i) w[i] = src[i];
        if (++pc == nch) {
            pc = 0;
            ++pr;
        }
    };
    uint32_t ring[D][DW];
#pragma unroll
    for (int k = 0; k < D; ++k) request(ring[k]);
    float acc = 0.0f;
    int cr = 0, cc = 0;  // the unit being computed
    // One block: the 32 codes (nibbles or bytes) of qs[0..7] (dwords) with
    // scale d (and offset m), against x slots 8h .. 8h + 7 of pair p.
    auto block = [&](const uint32_t (&q)[8], float d, float m, int p, int h) {
        float xv[32];
#pragma unroll
        for (int sl = 0; sl < 8; ++sl) {
            const gf32x4 f = xs4[16 * p + ((8 * h + sl) ^ (p & 15))];
#pragma unroll
            for (int i = 0; i < 4; ++i) xv[4 * sl + i] = f[i];
        }
        if (QT == 1) {
#pragma unroll
            for (int k = 0; k < 32; ++k) {
                const int8_t b = static_cast<int8_t>(q[k >> 2] >> (8 * (k & 3)));
                acc = __builtin_fmaf(d * static_cast<float>(b), xv[k], acc);
            }
        } else {
            const float off = QT == 2 ? -8.0f * d : m;
#pragma unroll
            for (int k = 0; k < 32; ++k) {
                const uint32_t byte = q[(k & 15) >> 2] >> (8 * (k & 3));
                const uint32_t nib = k < 16 ? (byte & 15u) : ((byte >> 4) & 15u);
                acc = __builtin_fmaf(__builtin_fmaf(static_cast<float>(nib), d, off), xv[k], acc);
            }
        }
    };
    auto step = [&](uint32_t (&w)[DW]) {
        const int p = cc * 64 + lane;
        if (p < np) {
            uint32_t q0[8], q1[8];
            float d0, d1, m0 = 0.0f, m1 = 0.0f;
            if (QT == 2) {  // 9 dwords: d0 | qs0 (bytes 2..17) | d1 (bytes 18..19) | qs1 (dwords 5..8)
#pragma unroll
                for (int i = 0; i < 4; ++i) q0[i] = __builtin_amdgcn_alignbit(w[i + 1], w[i], 16);
#pragma unroll
                for (int i = 0; i < 4; ++i) q1[i] = w[5 + i];
                d0 = h_lo(w[0]);
                d1 = h_hi(w[4]);
            } else if (QT == 1) {  // 17 dwords: d0 | qs0 (bytes 2..33) | d1 (bytes 34..35) | qs1 (dwords 9..16)
#pragma unroll
                for (int i = 0; i < 8; ++i) q0[i] = __builtin_amdgcn_alignbit(w[i + 1], w[i], 16);
#pragma unroll
                for (int i = 0; i < 8; ++i) q1[i] = w[9 + i];
                d0 = h_lo(w[0]);
                d1 = h_hi(w[8]);
            } else {  // 10 dwords: d0 m0 | qs0 (dwords 1..4) | d1 m1 | qs1 (dwords 6..9)
#pragma unroll
                for (int i = 0; i < 4; ++i) q0[i] = w[1 + i], q1[i] = w[6 + i];
                d0 = h_lo(w[0]);
                m0 = h_hi(w[0]);
                d1 = h_lo(w[5]);
                m1 = h_hi(w[5]);
            }
            block(q0, d0, m0, p, 0);
            block(q1, d1, m1, p, 1);
        }
        request(w);
        if (++cc == nch) {
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
            if (lane == 0) {
                const int row = gw + W * cr;
                *group_y(g, row, M, 0) = acc;
            }
            acc = 0.0f;
            cc = 0;
            ++cr;
        }
    };
    int u = 0;
    for (; u + D <= nu; u += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) step(ring[k]);
    }
#pragma unroll
    for (int k = 0; k < D; ++k)
        if (u + k < nu) step(ring[k]);
}

}  // namespace

hipError_t launch_gemv_f32(const LinearShape& s, const GemvGroup& g, const float* x, hipStream_t stream) {
    if (g.ncalls < 1 || g.ncalls > kGroupMaxCalls || s.rows != 1 || s.nb % 2 != 0) return hipErrorInvalidValue;
    const size_t lds = static_cast<size_t>(s.nb / 2) * 16 * sizeof(float) * 4;
    if (lds > 160 * 1024) return hipErrorNotSupported;
    int grid = (s.M + 7) / 8;
    if (grid > 2 * kPersistentWgs) grid = 2 * kPersistentWgs;
    auto go = [&](auto kernel) {
        if (lds > 64 * 1024 &&
            hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(lds)) != hipSuccess)
            return hipErrorInvalidConfiguration;
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(512), lds, stream, g, x, s.M, s.K, s.nb);
        return hipGetLastError();
    };
    switch (s.qtype) {
        case 1: return go(gemv_f32_kernel<1, 2>);
        case 2: return go(gemv_f32_kernel<2, 3>);
        default: return go(gemv_f32_kernel<3, 3>);
    }
}

hipError_t launch_gemv_group(const LinearShape& s, const GemvGroup& g, const float* x, hipStream_t stream) {
    if (g.ncalls < 1 || g.ncalls > kGroupMaxCalls) return hipErrorInvalidValue;
    return launch_mode<kModePlain>(s, g, x, stream);
}

hipError_t launch_gemv_glu(const LinearShape& s, const GemvGroup& g, const float* x, hipStream_t stream) {
    if (g.ncalls != 2 || g.norm_w == nullptr || g.y[0] == nullptr || g.row_begin[1] != s.M)
        return hipErrorInvalidValue;
    const PairCfg c = choose_pair(s);
    if (c.kind != Kind::Single) return hipErrorNotSupported;
    // A unit is two rows (gate and up).  Q4: two units in flight per wave and
    // one workgroup per CU measured fastest (LLaMA-7B-shaped Q4_0 greedy decode
    // 727 -> 737 tokens/s; one unit and two workgroups per CU had been best
    // before x was loaded ahead of the weights; three units: 717).  Q8_0 keeps
    // one unit (its 17-dword pairs would not fit two units in 128 VGPRs).
    // Rows of 64 pairs: one of the two units requested with x, the other once
    // x is staged (741 -> 752 tokens/s; both with x, as before: 741; three
    // units with one ahead: 736; one unit, two workgroups per CU: 731).
    auto go = [&](auto kernel, int lpr, int wgs_per_cu) {
        const int groups = (s.M + (64 / lpr) - 1) / (64 / lpr);
        int grid = (groups + kWaves - 1) / kWaves;
        if (grid > wgs_per_cu * kPersistentWgs) grid = wgs_per_cu * kPersistentWgs;
        hipLaunchKernelGGL(kernel, dim3(grid, s.rows), dim3(kWaves * 64), pair_lds_bytes(s.qtype, s.nb), stream, g, x,
                           s.M, s.K, s.nb, groups);
        return hipGetLastError();
    };
    switch (s.qtype * 100 + c.lpr) {
        case 116: return go(gemv_single_kernel<1, 16, kWaves, 1, kModeNormGlu>, 16, 2);
        case 164: return go(gemv_single_kernel<1, 64, kWaves, 1, kModeNormGlu>, 64, 2);
        case 216: return go(gemv_single_kernel<2, 16, kWaves, 2, kModeNormGlu>, 16, 1);
        case 264: return go(gemv_single_kernel<2, 64, kWaves, 2, kModeNormGlu, 1>, 64, 1);
        case 316: return go(gemv_single_kernel<3, 16, kWaves, 2, kModeNormGlu>, 16, 1);
        case 364: return go(gemv_single_kernel<3, 64, kWaves, 2, kModeNormGlu, 1>, 64, 1);
        default: return hipErrorInvalidValue;
    }
}

bool gemv_glu_supported(const LinearShape& s) { return choose_pair(s).kind == Kind::Single; }

hipError_t launch_gemv_decode(const LinearShape& s, const GemvGroup& g, const float* x, bool norm, bool accumulate,
                              hipStream_t stream) {
    if (g.ncalls < 1 || g.ncalls > kGroupMaxCalls || (norm && accumulate)) return hipErrorInvalidValue;
    if (norm && g.norm_w == nullptr) return hipErrorInvalidValue;
    if (accumulate) return launch_mode<kModeAcc>(s, g, x, stream);
    if (norm) return launch_mode<kModeNorm>(s, g, x, stream);
    return launch_mode<kModePlain>(s, g, x, stream);
}

hipError_t launch_gemv_pick(const LinearShape& s, const void* w, const float* x, float* y, PickState* ps,
                            int32_t* token, hipStream_t stream) {
    if (s.rows != 1 || ps == nullptr || token == nullptr) return hipErrorInvalidValue;
    GemvGroup g{};
    g.W[0] = w;
    g.y[0] = y;
    g.ncalls = 1;
    g.pick = ps;
    g.token = token;
    return launch_mode<kModePick>(s, g, x, stream);
}

hipError_t launch_gemv_pick_norm(const LinearShape& s, const void* w, const float* x, const float* norm_w,
                                 float norm_eps, float* y, PickState* ps, int32_t* token, hipStream_t stream) {
    if (s.rows != 1 || ps == nullptr || token == nullptr || norm_w == nullptr) return hipErrorInvalidValue;
    GemvGroup g{};
    g.W[0] = w;
    g.y[0] = y;
    g.ncalls = 1;
    g.pick = ps;
    g.token = token;
    g.norm_w = norm_w;
    g.norm_eps = norm_eps;
    return launch_mode<kModeNormPick>(s, g, x, stream);
}

hipError_t launch_gemv(const LinearShape& s, const void* w, const float* x, float* y,
                       hipStream_t stream) {
    GemvGroup g{};
    g.W[0] = w;
    g.y[0] = y;
    g.ncalls = 1;
    return launch_gemv_group(s, g, x, stream);
}

hipError_t launch_stream_floor(const LinearShape& s, const GemvGroup& g, uint32_t* sink, hipStream_t stream) {
    if (g.ncalls < 1 || g.ncalls > kGroupMaxCalls || s.nb % 2 != 0 || sink == nullptr) return hipErrorInvalidValue;
    const int np = s.nb / 2;
    int lpr = 16;
    if (np > 16) lpr = 64;
    if (np > 64) {
        lpr = 16;
        for (int l : {64, 32, 16}) {
            const int iters = (np + l - 1) / l;
            if (static_cast<double>(np) / (static_cast<double>(l) * iters) >= 0.875) {
                lpr = l;
                break;
            }
        }
    }
    const int items = (s.M + (64 / lpr) - 1) / (64 / lpr);
    int grid = (items + kWaves - 1) / kWaves;
    if (grid > kPersistentWgs) grid = kPersistentWgs;
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(kWaves * 64), 0, stream, g, s.M, s.nb, items, sink);
        return hipGetLastError();
    };
    switch (s.qtype * 100 + lpr) {
        case 116: return go(stream_floor_kernel<1, 16, 2>);
        case 132: return go(stream_floor_kernel<1, 32, 2>);
        case 164: return go(stream_floor_kernel<1, 64, 2>);
        case 216: return go(stream_floor_kernel<2, 16, 3>);
        case 232: return go(stream_floor_kernel<2, 32, 3>);
        case 264: return go(stream_floor_kernel<2, 64, 3>);
        case 316: return go(stream_floor_kernel<3, 16, 3>);
        case 332: return go(stream_floor_kernel<3, 32, 3>);
        case 364: return go(stream_floor_kernel<3, 64, 3>);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_stream_probe(const LinearShape& s, const GemvGroup& g, int mode, uint32_t* sink,
                               hipStream_t stream) {
    if (g.ncalls < 1 || g.ncalls > kGroupMaxCalls || sink == nullptr) return hipErrorInvalidValue;
    // The floor's grid: one persistent workgroup of kWaves waves per CU at most.
    const int np = s.nb / 2;
    const int rows_per_item = np > 16 ? 1 : 4;
    const int items = (s.M + rows_per_item - 1) / rows_per_item;
    int grid = (items + kWaves - 1) / kWaves;
    if (grid > kPersistentWgs) grid = kPersistentWgs;
    if (mode == kProbeEmpty) {
        hipLaunchKernelGGL(probe_empty_kernel, dim3(grid), dim3(kWaves * 64), 0, stream, sink);
    } else if (mode == kProbeLoad) {
        const size_t row_bytes = static_cast<size_t>(s.nb) * block_bytes(s.qtype);
        hipLaunchKernelGGL(probe_load_kernel, dim3(grid), dim3(kWaves * 64), 0, stream, g, s.M, row_bytes, sink);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

const char* gemv_kernel_name(const LinearShape& s) {
    static thread_local char buf[96];
    const char* fmt = s.qtype == 1 ? "q8_0" : s.qtype == 2 ? "q4_0" : "q4_1";
    const PairCfg c = choose_pair(s);
    if (c.kind == Kind::Single) {
        snprintf(buf, sizeof buf, "gemv_single_%s_lpr%d", fmt, c.lpr);
    } else if (c.kind == Kind::Multi) {
        snprintf(buf, sizeof buf, "gemv_multi_%s_lpr%d", fmt, c.lpr);
    } else {
        snprintf(buf, sizeof buf, "gemv_generic_%s", fmt);
    }
    return buf;
}

}  // namespace mlq

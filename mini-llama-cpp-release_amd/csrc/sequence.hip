// Persistent decode GEMV over a whole sequence of linears (one launch).
//
// A decode step issues a fixed chain of GEMVs (LLaMA: q, k, v -> o ->
// gate, up -> down per layer, then lm_head).  Launched one kernel at a time,
// every call pays the launch, the first-byte latency of its weights and the
// drain of its last wave (about 4.5 us per launch on MI355X, against 1.5 us of
// HBM time for a 4096x4096 Q4_0 matrix).  This kernel runs the chain in one
// launch and keeps the weights streaming across stage boundaries:
//  * The chain is split into *stages*: up to kSeqMaxCalls GEMVs that read the
//    same x (q, k, v or gate, up) and write disjoint outputs.  A stage's rows
//    are concatenated into row items and dealt to all waves of the grid (wave
//    w takes items w, w + GW, ...), so a fused q/k/v stage is one balanced
//    pass.
//  * Each wave walks its work units (row item x chunk of LPR pairs) with a
//    D-deep register ring of weight requests.  Inside a stage the ring runs D
//    units ahead; at a stage's end the wave arrives at the barrier first and
//    then requests the next stage's first D units at once, so they stream
//    from HBM while the grid synchronises and stages x (weights never depend
//    on earlier outputs).
//  * Between stages a grid-wide barrier makes every output of the earlier
//    stages visible before any wave stages the next x, so a call may consume
//    any earlier call's y, exactly as with one launch per call in stream order.
//  * Per row the arithmetic is that of the GEMV kernels in gemv.hip (same pair
//    dot, same lane-group width and chunk order, same DPP reduction), so
//    outputs are bit-identical to one launch per call.
//
// Barrier protocol (device memory, agent scope, no cache-maintenance fences):
//  * outputs are written with agent-scope stores (write-through to the point
//    of coherence); a stage whose x an earlier stage of the launch wrote reads
//    it with agent-scope loads, so no L2 writeback or invalidate is needed -
//    those cost ~20-40 us per grid barrier on MI355X when every workgroup
//    issues them;
//  * arrival: each wave waits for its stores to complete (its ring holds no
//    request then: the next stage's are issued after arriving), the
//    workgroup synchronises, and thread 0 adds 1 to sub[b % 8]; the last
//    arrival of a group adds 1 to `top` (a two-level tree: one hot address
//    would serialise all arrivals, ~90 ns each);
//  * thread 0 polls `top`; the poll is bounded by `spin_limit`: a workgroup
//    that gives up sets `error` and stops waiting, so every wave always
//    reaches the end of the kernel (the launch's outputs are then void and the
//    host reports it);
//  * the workgroups count themselves out through `exit`; the last one resets
//    all counters, so the next launch starts from zero without a host reset.
// All workgroups must be resident together: the host sizes the grid from the
// occupancy of this kernel (at most two workgroups per CU).

#include "gemv_device.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

namespace mlq {
namespace {

// First stage at or after `s` in which wave `gw` has a row item.
__device__ __forceinline__ int seq_next_stage(const SeqStageDesc* __restrict__ st, int nstages, int s, int gw) {
    while (s < nstages && gw >= st[s].items) ++s;
    return s;
}

// Unit i of wave gw in stage S: row item gw + (i / nch) * GW, chunk i % nch.
template <int QT, int LPR>
__device__ __forceinline__ void seq_load(const SeqStageDesc& S, int it, int c, int slot, int pl,
                                         uint32_t (&w)[Fmt<QT>::DW]) {
    constexpr int DW = Fmt<QT>::DW;
    constexpr int SUB = 64 / LPR;
    // Rows / pairs past the end re-read the last one; their results are dropped.
    const int row = min(it * SUB + slot, S.rows - 1);
    const int p = min(c * LPR + pl, S.np - 1);
    const void* W = S.call[0].W;
    int rb = 0;
#pragma unroll
    for (int j = 1; j < kSeqMaxCalls; ++j) {
        if (j < S.ncalls && row >= S.call[j].row_begin) {
            W = S.call[j].W;
            rb = S.call[j].row_begin;
        }
    }
    g_u32* src = as_global(static_cast<const uint32_t*>(W)) + static_cast<size_t>(row - rb) * (static_cast<size_t>(S.np) * DW) +
                 static_cast<size_t>(p) * DW;
#pragma unroll
    for (int i = 0; i < DW; ++i) w[i] = src[i];
}

// The row sum of lane group `slot` (held by its last lane after group_sum)
// in every lane of the group.
template <int LPR>
__device__ __forceinline__ float seq_bcast(float v) {
    const int src = (threadIdx.x & 63) | (LPR - 1);
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src << 2, __builtin_bit_cast(int, v)));
}

// Every lane stores: the lanes of a row group store the same value, and a
// group past the stage's rows recomputed the last row (its requests are
// clamped to it), so it stores that row's own value again.  No store is
// predicated, which keeps the weight requests' waits exact.
__device__ __forceinline__ void seq_store_row(const SeqStageDesc& S, int row, float v) {
    float* y = S.call[0].y;
    int rb = 0;
#pragma unroll
    for (int j = 1; j < kSeqMaxCalls; ++j) {
        if (j < S.ncalls && row >= S.call[j].row_begin) {
            y = S.call[j].y;
            rb = S.call[j].row_begin;
        }
    }
    __hip_atomic_store((__attribute__((address_space(1))) float*)(y + (row - rb)), v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned seq_load_word(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void seq_store_word(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned seq_groups() { return gridDim.x < kSeqGroups ? gridDim.x : kSeqGroups; }

// Barrier number n (1-based within the launch), arrival half.
__device__ __forceinline__ void seq_arrive(SeqSync* sync, unsigned n) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's y stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned C = seq_groups();
        const unsigned g = blockIdx.x % C;
        const unsigned members = (gridDim.x - g + C - 1) / C;
        const unsigned old = __hip_atomic_fetch_add(&sync->sub[g][0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == n * members - 1) {
            __hip_atomic_fetch_add(&sync->top[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Barrier number n, waiting half (thread 0 polls, then the workgroup syncs).
__device__ __forceinline__ void seq_wait(SeqSync* sync, unsigned n, unsigned spin_limit, bool& gave_up) {
    if (threadIdx.x == 0 && !gave_up) {
        const unsigned target = n * seq_groups();
        unsigned polls = 0;
        while (seq_load_word(&sync->top[0]) < target) {
            if (++polls > spin_limit) {
                seq_store_word(&sync->error[0], 1u);
                gave_up = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
}

// Register budget: 128 VGPRs (the x pair, the weight ring and the cursors),
// so that two workgroups fit per CU: every wave of the grid is needed to
// give the 4096-row stages one row per wave.
template <int QT> struct SeqOcc { static constexpr int waves_per_simd = 4; };
// Weight ring depth (work units in flight per wave).
template <int QT> struct SeqDepth { static constexpr int D = QT == 1 ? 1 : 2; };

template <int QT, int LPR>
__global__ __launch_bounds__(kWaves * 64, SeqOcc<QT>::waves_per_simd) void gemv_sequence_kernel(
    const SeqStageDesc* __restrict__ st, int nstages, SeqSync* __restrict__ sync, unsigned spin_limit) {
    constexpr int DW = Fmt<QT>::DW;
    constexpr int SUB = 64 / LPR;
    constexpr int D = SeqDepth<QT>::D;
    extern __shared__ float4 lds4[];
    const int lane = threadIdx.x & 63;
    const int slot = lane / LPR;
    const int pl = lane % LPR;
    const int gw = blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int GW = gridDim.x * kWaves;
    bool gave_up = false;

    // The ring holds units 0 .. D-1 of stage `ws` (the next stage with items
    // for this wave) or, inside a stage, the next D units.
    uint32_t wq[D][DW];
    auto fill = [&](int s) {
        const SeqStageDesc& S = st[s];
        int it = gw, c = 0;
#pragma unroll
        for (int i = 0; i < D; ++i) {
            seq_load<QT, LPR>(S, it, c, slot, pl, wq[i]);
            if (++c == S.nch) {
                c = 0;
                if (it + GW < S.items) it += GW;  // past the wave's last item: re-read it
            }
        }
    };
    int ws = seq_next_stage(st, nstages, 0, gw);
    if (ws < nstages) fill(ws);

    unsigned barriers = 0;
    for (int s = 0; s < nstages; ++s) {
        const SeqStageDesc& S = st[s];
        if (s > 0) {
            if (S.barrier) {
                seq_wait(sync, barriers, spin_limit, gave_up);
            } else {
                __syncthreads();  // LDS of the previous stage is no longer read
            }
        }
        const int np = S.np;
        uint32_t* xl = reinterpret_cast<uint32_t*>(lds4);
        float4* xc = reinterpret_cast<float4*>(xl + np * XLimbs<QT>::PAIR_DW);
        if (S.coherent) {
            stage_x_fit<QT, true>(S.x, S.K, S.nb, xl, xc);
        } else {
            stage_x_fit<QT, false>(S.x, S.K, S.nb, xl, xc);
        }

        if (ws == s) {
            // Units of this wave: items gw, gw + GW, ... (< items), nch chunks each.
            const int nit = (S.items - gw + GW - 1) / GW;
            const int nu = nit * S.nch;
            int it = gw, c = 0;        // unit being computed
            int pit = gw, pc = 0;      // unit D ahead (the next request)
            for (int i = 0; i < D; ++i) {
                if (++pc == S.nch) {
                    pc = 0;
                    pit += GW;
                }
            }
            // Ring slot k holds units k, k + D, k + 2D, ...: a slot is computed,
            // then refilled in place with the unit D ahead (no register copies,
            // which would wait for a request just issued).  Full rounds of D
            // units run without branches; the last round's units are guarded.
            if (S.nch == 1) {
                // Rows of one chunk: every item of the stage uses the same x pair.
                const int pp = min(pl, np - 1);
                uint32_t xq[XLimbs<QT>::PAIR_DW];
                float4 c0, c1;
                load_xq<QT>(xl, xc, pp, xq, c0, c1);
                const bool active = pl < np;
                auto step = [&](uint32_t (&w)[DW]) {
                    const float acc = active ? PairDot<QT>::run(w, xq, c0, c1, 0.0f) : 0.0f;
                    seq_load<QT, LPR>(S, pit, 0, slot, pl, w);  // past the end: clamped, unused
                    pit += GW;
                    seq_store_row(S, min(it * SUB + slot, S.rows - 1), seq_bcast<LPR>(group_sum<LPR>(acc)));
                    it += GW;
                };
                int u = 0;
                for (; u + D <= nu; u += D) {
#pragma unroll
                    for (int k = 0; k < D; ++k) step(wq[k]);
                }
#pragma unroll
                for (int k = 0; k < D; ++k)
                    if (u + k < nu) step(wq[k]);
            } else {
                float acc = 0.0f;
                auto step = [&](uint32_t (&w)[DW]) {
                    const int p = c * LPR + pl;
                    const int pp = min(p, np - 1);
                    uint32_t xq[XLimbs<QT>::PAIR_DW];
                    float4 c0, c1;
                    load_xq<QT>(xl, xc, pp, xq, c0, c1);
                    const float a = PairDot<QT>::run(w, xq, c0, c1, acc);
                    acc = p < np ? a : acc;
                    seq_load<QT, LPR>(S, pit, pc, slot, pl, w);  // past the end: clamped, unused
                    if (++pc == S.nch) {
                        pc = 0;
                        pit += GW;
                    }
                    // The running row sum is stored after every chunk (the last
                    // chunk's store is the result; nothing reads y before the
                    // next barrier), so that no store sits in a branch.
                    seq_store_row(S, min(it * SUB + slot, S.rows - 1), seq_bcast<LPR>(group_sum<LPR>(acc)));
                    acc = c == S.nch - 1 ? 0.0f : acc;
                    if (++c == S.nch) {
                        c = 0;
                        it += GW;
                    }
                };
                int u = 0;
                for (; u + D <= nu; u += D) {
#pragma unroll
                    for (int k = 0; k < D; ++k) step(wq[k]);
                }
#pragma unroll
                for (int k = 0; k < D; ++k)
                    if (u + k < nu) step(wq[k]);
            }
        }
        // Arrive before requesting the next stage's weights, so the arrival
        // does not wait for them; then fill the ring for the next stage with
        // items for this wave.
        if (s + 1 < nstages && st[s + 1].barrier) seq_arrive(sync, ++barriers);
        if (ws == s) {
            ws = seq_next_stage(st, nstages, s + 1, gw);
            if (ws < nstages) fill(ws);
        }
    }

    // Count out; the last workgroup resets the counters for the next launch.
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned done = __hip_atomic_fetch_add(&sync->exit[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == gridDim.x - 1) {
            for (int g = 0; g < kSeqGroups; ++g) seq_store_word(&sync->sub[g][0], 0u);
            seq_store_word(&sync->top[0], 0u);
            seq_store_word(&sync->exit[0], 0u);
        }
    }
}

template <int QT, int LPR>
const void* seq_kernel_ptr() {
    return reinterpret_cast<const void*>(&gemv_sequence_kernel<QT, LPR>);
}

const void* seq_kernel(int qtype, int lpr) {
    switch (qtype * 100 + lpr) {
        case 116: return seq_kernel_ptr<1, 16>();
        case 132: return seq_kernel_ptr<1, 32>();
        case 164: return seq_kernel_ptr<1, 64>();
        case 216: return seq_kernel_ptr<2, 16>();
        case 232: return seq_kernel_ptr<2, 32>();
        case 264: return seq_kernel_ptr<2, 64>();
        case 316: return seq_kernel_ptr<3, 16>();
        case 332: return seq_kernel_ptr<3, 32>();
        case 364: return seq_kernel_ptr<3, 64>();
        default: return nullptr;
    }
}

}  // namespace

bool sequence_supported(int qtype, int K) {
    const int nb = (K + kQK - 1) / kQK;
    return (qtype >= 1 && qtype <= 3) && nb % 2 == 0 && pair_lds_bytes(qtype, nb) <= kMaxPairLdsBytes;
}

int sequence_lpr(int K) {
    // The lane-group width gemv.hip picks for a single launch of this shape,
    // so a row is summed in the same order either way.
    const int np = (K + kQK - 1) / kQK / 2;
    if (np <= 16) return 16;
    if (np <= 64) return 64;
    for (int lpr : {64, 32, 16}) {
        const int iters = (np + lpr - 1) / lpr;
        if (static_cast<double>(np) / (static_cast<double>(lpr) * iters) >= 0.875) return lpr;
    }
    return 16;
}

int sequence_stage_lds_bytes(int qtype, int K) { return pair_lds_bytes(qtype, (K + kQK - 1) / kQK); }

hipError_t sequence_grid(int qtype, int lpr, int lds_bytes, int device, int* grid) {
    const void* k = seq_kernel(qtype, lpr);
    if (k == nullptr) return hipErrorInvalidValue;
    int per_cu = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, kWaves * 64, lds_bytes);
    if (e != hipSuccess) return e;
    int cus = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess) return e;
    if (per_cu < 1 || cus < 1) return hipErrorInvalidConfiguration;
    *grid = cus * (per_cu < 2 ? per_cu : 2);
    return hipSuccess;
}

hipError_t launch_sequence(int qtype, int lpr, const SeqStageDesc* stages, int nstages, SeqSync* sync,
                           int grid, int lds_bytes, unsigned spin_limit, hipStream_t stream) {
    const void* k = seq_kernel(qtype, lpr);
    if (k == nullptr || nstages <= 0 || grid <= 0) return hipErrorInvalidValue;
    void* args[] = {&stages, &nstages, &sync, &spin_limit};
    return hipLaunchKernel(k, dim3(grid), dim3(kWaves * 64), args, static_cast<size_t>(lds_bytes), stream);
}

const char* sequence_kernel_name(int qtype, int lpr) {
    static thread_local char buf[64];
    const char* fmt = qtype == 1 ? "q8_0" : qtype == 2 ? "q4_0" : "q4_1";
    snprintf(buf, sizeof buf, "gemv_sequence_%s_lpr%d", fmt, lpr);
    return buf;
}

}  // namespace mlq

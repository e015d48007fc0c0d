// Pipelined persistent GEMV chain (MLQ_SEQ_PIPELINED): a decode step's chain
// of GEMV stages in one launch whose weight stream never drains at a stage
// boundary.
//
// Why the boundary drains in a plain persistent kernel: a wave's memory
// counter (vmcnt) covers loads and stores in issue order, so a wave that must
// see its own y stores complete before it arrives at a grid barrier, or that
// waits for the next stage's x, also waits for every weight request it issued
// earlier -- including the next stage's, which are the ones that should keep
// HBM busy while the grid synchronises.
//
// Here the work of a boundary is split by wave:
//  * Compute waves (kChainCompute per workgroup) only ever wait for their own
//    weight requests.  Each keeps a D-deep register ring of work units (row
//    item x chunk) that runs across stages: the slot a unit frees is refilled
//    with the wave's next unit, of this stage or of the next one, so at a
//    boundary the next stage's first units are already in flight.  A row's y
//    is stored by the compute wave itself when a later request of that wave
//    (which the wave waits for before the stage ends) was issued after the
//    store -- that wait proves the store complete.  The rows of the wave's
//    last D units of a stage are not covered that way; they go to LDS and the
//    control wave stores them (their own global store goes to the wave's own
//    sink words).
//  * The control wave (one per workgroup) holds no weight requests: after the
//    workgroup's compute waves finish a stage it stores the handed-over rows
//    with agent-scope stores, waits for them, arrives at the grid barrier,
//    polls it, and loads the next stage's x straight into LDS (LDS DMA,
//    16 bytes per lane, no registers).  Its waits cover only its own
//    requests.
//  * Between them, workgroup barriers on LDS only (s_barrier with LDS
//    fences): B2 "raw x in LDS", then the compute waves turn it into limbs
//    (the integer x representation of gemv_device.h) and B3 "limbs ready",
//    then the stage, then B1 "stage done, rows handed over".
// Per row the arithmetic is that of gemv.hip (same pair dot, lane-group width,
// chunk order and DPP reduction): outputs are bit-identical to one launch per
// call.
//
// Grid barrier: the two-level counter tree of sequence.hip (8 group counters
// and a top counter, agent scope, no cache-maintenance fences), arrived at and
// polled by the control waves only; waits are bounded (`spin_limit`): a
// workgroup that gives up sets `error` and carries on, so the kernel always
// ends; the last workgroup out resets the counters.  All workgroups must be
// resident together: the host sizes the grid from the kernel's occupancy.
// Rows of in_features with K % 32 == 0 only (x is loaded in 1 KB DMA rounds
// of whole 16-byte groups).

#include "gemv_device.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

namespace mlq {
namespace {

constexpr int kChainCompute = 15;                         // compute waves per workgroup
constexpr int kChainThreads = (kChainCompute + 1) * 64;   // + one control wave
constexpr int kChainMaxGrid = 1024;                       // workgroups a launch may have (sink size)
template <int QT> struct ChainDepth { static constexpr int D = QT == 1 ? 1 : 2; };

// Workgroup barrier ordering LDS only: the caller's LDS writes are complete
// and visible after it, weight requests stay in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ unsigned chain_load_word(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void chain_store_word(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void chain_store_y(float* p, float v) {
    __hip_atomic_store((__attribute__((address_space(1))) float*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Stage descriptors are read through the constant address space, so every
// field read is a scalar load (counted by lgkmcnt): a vector load of a
// descriptor field would be waited for with the in-order vmcnt, which would
// also wait for the weight ring.
typedef __attribute__((address_space(4))) const SeqStageDesc CDesc;

// Output address of stage row `row` (the call holding it).
__device__ __forceinline__ float* chain_y(CDesc& S, int row) {
    float* y = S.call[0].y;
    int rb = 0;
#pragma unroll
    for (int j = 1; j < kSeqMaxCalls; ++j) {
        if (j < S.ncalls && row >= S.call[j].row_begin) {
            y = S.call[j].y;
            rb = S.call[j].row_begin;
        }
    }
    return y + (row - rb);
}

// One ring slot: a lane's pair of blocks (DW dwords) as 16-byte groups plus a
// 4- or 8-byte tail, so the registers a slot lives in are the aligned tuples
// its loads write.
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2a __attribute__((ext_vector_type(2), aligned(4)));
template <int R> struct SlotTail;
template <> struct SlotTail<1> { typedef uint32_t type; };
template <> struct SlotTail<2> { typedef u32x2a type; };
template <int DW> struct Slot {
    static constexpr int Q = DW / 4;
    static constexpr int R = DW % 4;
    u32x4a v[Q];
    typename SlotTail<R>::type t;
    __device__ __forceinline__ void load(const uint32_t* src) {
        typedef __attribute__((address_space(1))) const u32x4a g4;
        typedef __attribute__((address_space(1))) const typename SlotTail<R>::type gt;
#pragma unroll
        for (int q = 0; q < Q; ++q) v[q] = *(g4*)(src + 4 * q);
        t = *(gt*)(src + 4 * Q);
    }
    __device__ __forceinline__ void to(uint32_t (&w)[DW]) const {
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            w[4 * q] = v[q].x;
            w[4 * q + 1] = v[q].y;
            w[4 * q + 2] = v[q].z;
            w[4 * q + 3] = v[q].w;
        }
        if constexpr (R == 1) {
            w[4 * Q] = t;
        } else {
            w[4 * Q] = t.x;
            w[4 * Q + 1] = t.y;
        }
    }
};

// Unit (item it, chunk c) of stage S into a ring slot; rows / pairs past the
// end re-read the last one (their results are dropped).
template <int QT, int LPR>
__device__ __forceinline__ void chain_load(CDesc& S, int it, int c, int slot, int pl, Slot<Fmt<QT>::DW>& w) {
    constexpr int DW = Fmt<QT>::DW;
    constexpr int SUB = 64 / LPR;
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
    const uint32_t* src = static_cast<const uint32_t*>(W) +
                          static_cast<size_t>(row - rb) * (static_cast<size_t>(S.np) * DW) + static_cast<size_t>(p) * DW;
    w.load(src);
}

// The eight elements of thread `sub`'s two x dwords of block g from the raw
// x in LDS (the element order of load8 in gemv_device.h).
template <int QT>
__device__ __forceinline__ void raw8(const float* __restrict__ raw, int g, int sub, float (&v)[8]) {
    const int blk = g & 1;
#pragma unroll
    for (int dd = 0; dd < 2; ++dd) {
        const int2 r = x_runs<QT>(blk, 2 * sub + dd);
        const float2 a = *reinterpret_cast<const float2*>(raw + g * kQK + r.x);
        const float2 b = *reinterpret_cast<const float2*>(raw + g * kQK + r.y);
        v[4 * dd] = a.x;
        v[4 * dd + 1] = a.y;
        v[4 * dd + 2] = b.x;
        v[4 * dd + 3] = b.y;
    }
}

template <int QT, int LPR>
__global__ __launch_bounds__(kChainThreads, 4) void gemv_chain_kernel(const SeqStageDesc* __restrict__ stages,
                                                                      int nstages, SeqSync* __restrict__ sync,
                                                                      unsigned spin_limit, int kmax,
                                                                      float* __restrict__ sink) {
    CDesc* st = (CDesc*)stages;
    constexpr int DW = Fmt<QT>::DW;
    constexpr int SUB = 64 / LPR;
    constexpr int D = ChainDepth<QT>::D;
    static_assert(D == 1 || D == 2, "the ring handles one or two slots");
    extern __shared__ float4 lds4[];
    constexpr int H = D + 1;  // handed-over units per wave and stage
    // Handed-over rows: per compute wave, H slots (+ one dump slot written by
    // the units before the window) of one (row, value) entry per lane; the
    // entry of lane slot * LPR holds the row of lane group `slot` (row -1:
    // nothing to store).  Every lane writes its own entry: no branch, no
    // shared address.
    __shared__ int2 hand[kChainCompute][H + 1][64];
    float* raw = reinterpret_cast<float*>(lds4);                       // [kmax] floats
    uint32_t* xl = reinterpret_cast<uint32_t*>(lds4 + kmax / 4);       // limbs, then block constants
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;

    if (wave == kChainCompute) {
        // ------------------------------------------------------------ control
        constexpr int kEntries = kChainCompute * H * SUB;
        for (int i = 0; i < kChainCompute * (H + 1); ++i) hand[i / (H + 1)][i % (H + 1)][lane] = make_int2(-1, 0);
        bool gave_up = false;
        unsigned barriers = 0;
        for (int s = 0; s < nstages; ++s) {
            CDesc& S = st[s];
            if (s > 0 && S.barrier && lane == 0 && !gave_up) {
                const unsigned target = barriers * (gridDim.x < kSeqGroups ? gridDim.x : kSeqGroups);
                unsigned polls = 0;
                while (chain_load_word(&sync->top[0]) < target) {
                    if (++polls > spin_limit) {
                        chain_store_word(&sync->error[0], 1u);
                        gave_up = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
            // x of stage s into LDS: rounds of 64 lanes x 16 bytes (K % 4 == 0;
            // lanes past K / 4 in the last round load nothing).
            const float4* xs = reinterpret_cast<const float4*>(S.x);
            const int n4 = S.K >> 2;
            for (int j = 0; 64 * j < n4; ++j) {
                if (64 * j + lane < n4) {
                    if (S.coherent) {
                        __builtin_amdgcn_global_load_lds(xs + 64 * j + lane, lds4 + 64 * j, 16, 0, 16);
                    } else {
                        __builtin_amdgcn_global_load_lds(xs + 64 * j + lane, lds4 + 64 * j, 16, 0, 0);
                    }
                }
            }
            if (s == 0) __builtin_amdgcn_s_barrier();  // B0: x requested before any weight
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            lds_barrier();  // B2: raw x in LDS
            lds_barrier();  // B3: limbs in LDS
            lds_barrier();  // B1: the stage's rows computed, the last ones handed over
            for (int e = lane; e < kEntries; e += 64) {
                const int w = e / (H * SUB), h = (e / SUB) % H, sl = e % SUB;
                int2& ent = hand[w][h][sl * LPR];
                const int2 v = ent;
                if (v.x >= 0) chain_store_y(chain_y(S, v.x), __builtin_bit_cast(float, v.y));
                ent = make_int2(-1, 0);
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the handed-over rows are stored
            if (s + 1 < nstages && st[s + 1].barrier) {
                ++barriers;
                if (lane == 0) {
                    const unsigned C = gridDim.x < kSeqGroups ? gridDim.x : kSeqGroups;
                    const unsigned g = blockIdx.x % C;
                    const unsigned members = (gridDim.x - g + C - 1) / C;
                    const unsigned old =
                        __hip_atomic_fetch_add(&sync->sub[g][0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (old == barriers * members - 1) {
                        __hip_atomic_fetch_add(&sync->top[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            }
        }
        // Count out; the last workgroup resets the counters for the next launch.
        if (lane == 0) {
            const unsigned done =
                __hip_atomic_fetch_add(&sync->exit[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (done == gridDim.x - 1) {
                for (int g = 0; g < kSeqGroups; ++g) chain_store_word(&sync->sub[g][0], 0u);
                chain_store_word(&sync->top[0], 0u);
                chain_store_word(&sync->exit[0], 0u);
            }
        }
        return;
    }

    // ---------------------------------------------------------------- compute
    const int slot = lane / LPR;
    const int pl = lane % LPR;
    const int gw = blockIdx.x * kChainCompute + wave;
    const int GW = gridDim.x * kChainCompute;
    float* wsink = sink + static_cast<size_t>(gw) * 64 + lane;  // this lane's sink word

    // A wave's units of a stage: nit row items x nch chunks, padded to a
    // multiple of D, and to at least D, with re-reads of its last unit (the
    // padding requests hit lines just requested; their sums are dropped).  So
    // every wave takes part in every stage and every stage starts at ring
    // slot 0: the ring loop has no guarded steps.
    auto stage_units = [&](int t) {
        const int items = st[t].items;
        return gw < items ? (items - gw + GW - 1) / GW * st[t].nch : 0;
    };
    auto padded = [&](int nu) { return nu > D ? (nu + D - 1) / D * D : D; };
    // (item, chunk) of unit j of stage t: the last real unit past the wave's
    // units (and the wave's first item when it has none: its rows clamp).
    auto coords = [&](int t, int j, int& it, int& c) {
        const int nch = st[t].nch;
        const int jj = min(j, max(stage_units(t) - 1, 0));
        it = gw + jj / nch * GW;
        c = jj % nch;
    };
    Slot<DW> wq[D];
    uint32_t xq[XLimbs<QT>::PAIR_DW];  // the lane's x limbs of the current chunk
    float4 c0, c1;
    for (int s = 0; s < nstages; ++s) {
        CDesc& S = st[s];
        if (s == 0) {
            __builtin_amdgcn_s_barrier();  // B0: the control wave's x requests go first
#pragma unroll
            for (int k = 0; k < D; ++k) {
                int it0, c0i;
                coords(0, k, it0, c0i);
                chain_load<QT, LPR>(S, it0, c0i, slot, pl, wq[k]);
            }
        }
        lds_barrier();  // B2: raw x of stage s in LDS
        // Limbs: four threads per block, as stage_x, from the raw x.
        const int np = S.np;
        float4* xc = reinterpret_cast<float4*>(xl + np * XLimbs<QT>::PAIR_DW);
        {
            const int sub = threadIdx.x & 3;
            for (int gb = static_cast<int>(threadIdx.x >> 2); gb < S.nb; gb += kChainCompute * 16) {
                float v[8];
                raw8<QT>(raw, gb, sub, v);
                emit_block<QT>(gb, sub, v, xl, xc);
            }
        }
        lds_barrier();  // B3: limbs of stage s ready

        const int nu = stage_units(s);
        const int npad = padded(nu);
        const int nch = S.nch;
        // A unit's row is stored after the request that refills its slot, so
        // the request proving that store complete is the one made one unit
        // later: the last D + 1 units of the stage hand their rows over.
        const int win = npad - H;
        int it = gw, c = 0;  // unit being computed
        // Prefetch cursor within the stage: unit pj (D ahead of the computed
        // one), item pit, chunk pc; held at the last real unit.
        int pj = D, pit, pc;
        coords(s, D, pit, pc);
        auto issue_here = [&](Slot<DW>& w) {
            chain_load<QT, LPR>(S, pit, pc, slot, pl, w);
            const bool adv = pj + 1 < nu;
            const bool wrap = pc + 1 == nch;
            pit = adv && wrap ? pit + GW : pit;
            pc = adv ? (wrap ? 0 : pc + 1) : pc;
            ++pj;
        };
        // The last D refills of the stage request the next stage's first D
        // units (after the last stage: re-reads of this stage's).
        const int tn = min(s + 1, nstages - 1);
        int kn = 0;
        auto issue_next = [&](Slot<DW>& w) {
            int itn, cn;
            coords(tn, s + 1 < nstages ? kn : npad, itn, cn);
            chain_load<QT, LPR>(st[tn], itn, cn, slot, pl, w);
            ++kn;
        };
        // A row's value: stored by this wave, or (last D + 1 units) handed
        // to the control wave through LDS while the wave's own store goes
        // to the sink; padding units store to the sink only.
        auto put = [&](int i, float v) {
            const int row = min(it * SUB + slot, S.rows - 1);
            const bool over = i >= win;  // handed over
            chain_store_y(over || i >= nu ? wsink : chain_y(S, row), v);
            // Keeps the store ahead of the next unit's request in issue order:
            // that request's completion is what proves it complete.
            asm volatile("" ::: "memory");
            const int hs = over ? i - win : H;
            hand[wave][hs][lane] =
                make_int2(over && i < nu && c == nch - 1 ? row : -1, __builtin_bit_cast(int, v));
        };
        // One loop for rows of one chunk and of several: the lane's x limbs
        // are (re)loaded from LDS when the unit's chunk differs from the one
        // they hold (at the stage's first unit for rows of one chunk, every
        // unit for longer rows).  Two loops would hold the ring in different
        // registers and copy it at each switch, waiting for it.
        float acc = 0.0f;
        int cx = -1;  // chunk whose limbs xq holds
        auto step = [&](Slot<DW>& ws, int i, auto&& issue) {
            const int p = c * LPR + pl;
            if (c != cx) {
                load_xq<QT>(xl, xc, min(p, np - 1), xq, c0, c1);
                cx = c;
            }
            uint32_t w[DW];
            ws.to(w);
            const float a = PairDot<QT>::run(w, xq, c0, c1, acc);
            acc = p < np ? a : acc;
            // The refill is issued after the slot's last read (hoisted above
            // it, the load would need other registers than the slot's).
            __builtin_amdgcn_sched_barrier(0);
            issue(ws);
            // The running row sum after every chunk (the last chunk's is the
            // result), so no store sits in a branch.
            put(i, __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(
                                              (lane | (LPR - 1)) << 2,
                                              __builtin_bit_cast(int, group_sum<LPR>(acc)))));
            acc = c == nch - 1 ? 0.0f : acc;
            if (++c == nch) {
                c = 0;
                it += GW;
            }
        };
        int i = 0;
        for (; i + D < npad; i += D) {
#pragma unroll
            for (int k = 0; k < D; ++k) step(wq[k], i + k, issue_here);
        }
#pragma unroll
        for (int k = 0; k < D; ++k) step(wq[k], i + k, issue_next);
        lds_barrier();  // B1: stage s done; the last rows are in LDS
    }
}

template <int QT, int LPR>
const void* chain_kernel_ptr() {
    return reinterpret_cast<const void*>(&gemv_chain_kernel<QT, LPR>);
}

const void* chain_kernel(int qtype, int lpr) {
    switch (qtype * 100 + lpr) {
        case 116: return chain_kernel_ptr<1, 16>();
        case 132: return chain_kernel_ptr<1, 32>();
        case 164: return chain_kernel_ptr<1, 64>();
        case 216: return chain_kernel_ptr<2, 16>();
        case 232: return chain_kernel_ptr<2, 32>();
        case 264: return chain_kernel_ptr<2, 64>();
        case 316: return chain_kernel_ptr<3, 16>();
        case 332: return chain_kernel_ptr<3, 32>();
        case 364: return chain_kernel_ptr<3, 64>();
        default: return nullptr;
    }
}

}  // namespace

size_t chain_sink_bytes() { return static_cast<size_t>(kChainMaxGrid) * kChainCompute * 64 * sizeof(float); }

int chain_lds_bytes(int qtype, int kmax) { return kmax * 4 + pair_lds_bytes(qtype, (kmax + kQK - 1) / kQK); }

hipError_t chain_grid(int qtype, int lpr, int lds_bytes, int device, int* grid) {
    const void* k = chain_kernel(qtype, lpr);
    if (k == nullptr) return hipErrorInvalidValue;
    int per_cu = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, kChainThreads, lds_bytes);
    if (e != hipSuccess) return e;
    int cus = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess) return e;
    if (per_cu < 1 || cus < 1) return hipErrorInvalidConfiguration;
    *grid = cus * (per_cu < 2 ? per_cu : 2);
    return hipSuccess;
}

hipError_t launch_chain(int qtype, int lpr, const SeqStageDesc* stages, int nstages, SeqSync* sync, int grid,
                        int lds_bytes, unsigned spin_limit, int kmax, float* sink, hipStream_t stream) {
    const void* k = chain_kernel(qtype, lpr);
    if (k == nullptr || nstages <= 0 || grid <= 0 || grid > kChainMaxGrid || kmax % kQK != 0) {
        return hipErrorInvalidValue;
    }
    void* args[] = {&stages, &nstages, &sync, &spin_limit, &kmax, &sink};
    return hipLaunchKernel(k, dim3(grid), dim3(kChainThreads), args, static_cast<size_t>(lds_bytes), stream);
}

const char* chain_kernel_name(int qtype, int lpr) {
    static thread_local char buf[64];
    const char* fmt = qtype == 1 ? "q8_0" : qtype == 2 ? "q4_0" : "q4_1";
    snprintf(buf, sizeof buf, "gemv_chain_%s_lpr%d", fmt, lpr);
    return buf;
}

}  // namespace mlq

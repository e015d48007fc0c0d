// Persistent decode GEMV chain fed through an LDS weight ring
// (MLQ_SEQ_LDS_RING): the weights of every stage of the chain stream from HBM
// without a pause at the stage boundaries, while the arithmetic waits for
// each stage's x.
//
// One 1024-thread workgroup per CU, two kinds of waves:
//  * Loader waves (kRingLoaders).  The CU takes rows b, b + G, b + 2G, ... of
//    every stage (G workgroups); loader l takes the CU's rows l, l + 4, ...,
//    and walks their work units -- one unit is a chunk of up to 64 pairs of a
//    row -- stage after stage, copying each unit's bytes into its own slice of
//    a ring in LDS (SL slots of 64 pairs; the whole ring is the 130-150 KB the
//    x limbs leave free).  It keeps R units in flight in registers (16-byte
//    buffer loads) and writes each to LDS once its slot has been released.
//    Weights never depend on x, so the loaders run ahead of the arithmetic
//    across stage boundaries for as long as their slices have room.  Their
//    cursor caches the stage's calls and the row's buffer resource, so a unit
//    costs a few scalar instructions: the scalar unit is shared by all waves
//    of the CU, and a cursor that looked the calls up per unit held the
//    loaders to a fraction of the HBM rate.
//  * Compute waves (kRingCompute) do everything that waits for x: per stage
//    they stage x into LDS as block-scaled integer limbs (gemv_device.h),
//    claim the stage's rows of the CU one at a time from an LDS counter (so
//    they finish together), read each unit's pair from its slot, release the
//    slot, and store each row's sum.  Between stages they store their rows,
//    wait for the stores, meet at an LDS counter, and one lane of the first
//    compute wave arrives at and polls the grid barrier before x is staged
//    again.  They hold no weight requests, so their memory waits cover only
//    their own x loads and y stores.
// Slot hand-over: per slot two LDS words, `ready` = k + 1 once the loader's
// unit k is in the slot and `done` = k + 1 once a compute wave has read it.
// Fences on LDS only ("local"), so no wait covers the loaders' weight
// requests.
// Per row the arithmetic is that of gemv.hip's lane-group width 64 (lane l
// takes pair 64 c + l of chunk c, the same pair dot, chunk order and DPP
// reduction): outputs are bit-identical to one launch per call.
// Grid barrier: the two-level counter tree of sequence.hip (agent-scope
// atomics, outputs stored with agent-scope stores, x of a stage that an
// earlier stage wrote loaded with agent-scope loads).  Every wait -- the grid
// barrier, the slot words and the compute waves' LDS counter -- is bounded by
// `spin_limit` polls: a wave that gives up sets `error` and carries on, so the
// kernel always ends (its outputs are then void).  All workgroups must be
// resident together: the host launches one per CU after checking occupancy.

#include "gemv_device.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

namespace mlq {
namespace {

constexpr int kRingLoaders = 4;
constexpr int kRingCompute = 12;
constexpr int kRingThreads = (kRingLoaders + kRingCompute) * 64;
constexpr int kRingMaxSlots = 64;
constexpr int kRingCtlBytes = 1024;  // LDS control words, ahead of the x limbs
constexpr int kRingLdsMax = 160 * 1024;

// Units in flight per loader wave (registers: R x KL x 4 VGPRs).
template <int QT> struct RingDepth { static constexpr int R = QT == 1 ? 4 : 8; };
// Bytes of one pair and of one unit (a slot) per format.
template <int QT> struct RingFmt {
    static constexpr int PB = Fmt<QT>::DW * 4;
    static constexpr int SB = 64 * PB;
    static constexpr int KL = (SB + 1023) / 1024;  // 16-byte loads per lane and unit
};

struct RingCtl {
    unsigned ready[kRingMaxSlots];
    unsigned done[kRingMaxSlots];
    unsigned cbar;    // compute waves' meeting counter
    unsigned claim;   // rows claimed by compute waves, over all stages
};
static_assert(sizeof(RingCtl) <= kRingCtlBytes, "control words fit their LDS");

#ifdef MLQ_RING_STAMPS
// Measurement build (`make stamps`): s_memrealtime stamps (100 MHz) of three
// workgroups at the points of each stage boundary, read back with
// mlq_hip_ring_stamps.  The stamps add stores and change no work.
__device__ unsigned long long g_ring_stamps[kRingStampWgs * kRingStampStages * kRingStampSlots];
#define RING_STAMP(stage, j)                                                                                    \
    do {                                                                                                        \
        if (stamp_wg >= 0 && (stage) < kRingStampStages && lane == 0)                                          \
            g_ring_stamps[(stamp_wg * kRingStampStages + (stage)) * kRingStampSlots + (j)] =                  \
                __builtin_amdgcn_s_memrealtime();                                                               \
    } while (0)
#else
#define RING_STAMP(stage, j) \
    do {                     \
    } while (0)
#endif

// Stage descriptors through the constant address space: scalar loads.
typedef __attribute__((address_space(4))) const SeqStageDesc RDesc;
typedef uint32_t ru4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ unsigned lds_load(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_store(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ unsigned dev_load(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void dev_store(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// LDS-only ordering: waits for the wave's LDS accesses, never for its
// global requests.
__device__ __forceinline__ void lds_release() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local"); }
__device__ __forceinline__ void lds_acquire() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local"); }

// Rows of stage S that CU b takes (rows b, b + G, ...).
__device__ __forceinline__ int ring_rows(RDesc& S, int b, int G) {
    return S.rows > b ? (S.rows - b - 1) / G + 1 : 0;
}

// Polls `*p` until it reaches `target` (wave-uniform); false after
// `spin_limit` polls.
__device__ __forceinline__ bool lds_wait_geq(const unsigned* p, unsigned target, unsigned spin_limit) {
    unsigned polls = 0;
    while (lds_load(p) < target) {
        if (++polls > spin_limit) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    return true;
}

// A loader wave's position in its share of the CU's work units: stage s,
// CU-local row i (loader lw takes rows lw, lw + kRingLoaders, ...), chunk c;
// the stage's shape and calls are cached when the stage is entered and the
// row's buffer resource and offset when the row is entered, so stepping to
// the next unit is a few scalar operations (the scalar unit is shared by all
// waves of the CU).
template <int QT>
struct RingCursor {
    int s, i, c, n, nch, np, ncalls;
    const void* W[kSeqMaxCalls];
    int rb[kSeqMaxCalls], M[kSeqMaxCalls];
    __amdgpu_buffer_rsrc_t rs;
    uint32_t row_off;
    __device__ __forceinline__ void set_row(int b, int G) {
        constexpr int PB = RingFmt<QT>::PB;
        const int row = b + i * G;
        const void* w = W[0];
        int r0 = 0, m = M[0];
#pragma unroll
        for (int j = 1; j < kSeqMaxCalls; ++j) {
            if (j < ncalls && row >= rb[j]) {
                w = W[j];
                r0 = rb[j];
                m = M[j];
            }
        }
        const uint32_t row_bytes = static_cast<uint32_t>(np) * PB;
        rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(w), static_cast<short>(0),
                                               static_cast<int>(static_cast<uint32_t>(m) * row_bytes), 0x00020000);
        row_off = static_cast<uint32_t>(row - r0) * row_bytes;
    }
    // First stage at or after s with a row for loader lw.
    __device__ __forceinline__ void enter(RDesc* st, int nstages, int b, int G, int lw) {
        for (; s < nstages; ++s) {
            RDesc& S = st[s];
            n = ring_rows(S, b, G);
            if (n > lw) {
                nch = S.nch;
                np = S.np;
                ncalls = S.ncalls;
#pragma unroll
                for (int j = 0; j < kSeqMaxCalls; ++j) {
                    W[j] = S.call[j].W;
                    rb[j] = S.call[j].row_begin;
                    M[j] = S.call[j].M;
                }
                i = lw;
                c = 0;
                set_row(b, G);
                return;
            }
        }
    }
    __device__ __forceinline__ void next(RDesc* st, int nstages, int b, int G, int lw) {
        if (++c < nch) return;
        c = 0;
        i += kRingLoaders;
        if (i < n) {
            set_row(b, G);
            return;
        }
        ++s;
        enter(st, nstages, b, G, lw);
    }
    // Issues the unit's 16-byte loads; returns its byte count (0 past the
    // end).  Buffer loads, range-checked against the call's weight bytes
    // (under 2 GiB): lanes past the unit's bytes, and every lane past the end,
    // load from an offset out of range, which returns zeros without a memory
    // access.
    __device__ __forceinline__ int issue(int nstages, int lane, ru4 (&r)[RingFmt<QT>::KL]) const {
        constexpr int PB = RingFmt<QT>::PB;
        constexpr uint32_t kOff = 0x7FFFFFF0u;
        const int bytes = s < nstages ? min(np - c * 64, 64) * PB : 0;
        const uint32_t base = row_off + static_cast<uint32_t>(c) * 64 * PB;
#pragma unroll
        for (int k = 0; k < RingFmt<QT>::KL; ++k) {
            const int o = 1024 * k + 16 * lane;
            r[k] = __builtin_bit_cast(ru4, __builtin_amdgcn_raw_buffer_load_b128(rs, o < bytes ? base + o : kOff, 0, 0));
        }
        return bytes;
    }
};

template <int QT, bool COHERENT>
__device__ __forceinline__ void ring_stage_x(RDesc& S, uint32_t* __restrict__ xl, float4* __restrict__ xc, int t) {
    constexpr int PER = kRingCompute * 16;  // blocks per round
    constexpr int ROUNDS = 3;               // nb <= 480 < 3 * PER
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(S.x), static_cast<short>(0),
                                                                        S.K * 4, 0x00020000);
    const int sub = t & 3, g0 = t >> 2, nb = S.nb;
    float v[ROUNDS][8];
#pragma unroll
    for (int r = 0; r < ROUNDS; ++r) load8<QT, COHERENT>(rs, min(g0 + r * PER, nb - 1), sub, v[r]);
#pragma unroll
    for (int r = 0; r < ROUNDS; ++r)
        if (g0 + r * PER < nb) emit_block<QT>(g0 + r * PER, sub, v[r], xl, xc);
}

template <int QT>
__global__ __launch_bounds__(kRingThreads, 1) void gemv_ring_kernel(const SeqStageDesc* __restrict__ stages,
                                                                    int nstages, SeqSync* __restrict__ sync,
                                                                    unsigned spin_limit, int x_bytes, int nslots) {
    using F = RingFmt<QT>;
    constexpr int DW = Fmt<QT>::DW;
    RDesc* st = (RDesc*)stages;
    extern __shared__ __attribute__((aligned(16))) char lds[];
    RingCtl& ctl = *reinterpret_cast<RingCtl*>(lds);
    uint32_t* xl = reinterpret_cast<uint32_t*>(lds + kRingCtlBytes);
    char* ring = lds + kRingCtlBytes + x_bytes;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int b = blockIdx.x, G = gridDim.x;
#ifdef MLQ_RING_STAMPS
    const int stamp_wg = b == 0 ? 0 : b == G / 2 + 1 ? 1 : b == G - 1 ? 2 : -1;
#endif

    for (int k = threadIdx.x; k < kRingMaxSlots; k += kRingThreads) {
        ctl.ready[k] = 0;
        ctl.done[k] = 0;
    }
    if (threadIdx.x == 0) {
        ctl.cbar = 0;
        ctl.claim = 0;
    }
    __syncthreads();

    // Loader lw owns ring slots [lw * SL, (lw + 1) * SL) and the units of rows
    // lw, lw + kRingLoaders, ... of every stage; its k-th unit goes to slot
    // lw * SL + k % SL.  ready[slot] = k + 1 once unit k is in the slot,
    // done[slot] = k + 1 once its compute wave has read it.
    const int SL = nslots / kRingLoaders;
    if (wave < kRingLoaders) {
        // ------------------------------------------------------------ loaders
        constexpr int R = RingDepth<QT>::R;
        const int lw = wave;
        RingCursor<QT> cur{};
        cur.rs = __builtin_amdgcn_make_buffer_rsrc(nullptr, static_cast<short>(0), 0, 0x00020000);
        cur.enter(st, nstages, b, G, lw);
        ru4 reg[R][F::KL];
        int nbytes[R];
#ifdef MLQ_RING_STAMPS
        int nstg[R];  // stage of each register set's unit
        int last_issued = -1, last_written = -1;
        auto stamp_issue = [&](int r) {
            nstg[r] = cur.s;
            if (lw == 0 && cur.s != last_issued) {
                RING_STAMP(cur.s, 22);  // first unit of the stage requested
                last_issued = cur.s;
            }
        };
#else
        auto stamp_issue = [](int) {};
#endif
#pragma unroll
        for (int r = 0; r < R; ++r) {
            stamp_issue(r);
            nbytes[r] = cur.issue(nstages, lane, reg[r]);
            cur.next(st, nstages, b, G, lw);
        }
        unsigned k = 0;  // this loader's unit count
        int q = 0;       // its slot: lw * SL + q, q = k % SL
        bool ok = true;
        bool live = nbytes[0] > 0;
        while (live) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (nbytes[r] == 0) {
                    live = false;
                    break;
                }
                const int slot = lw * SL + q;
                if (ok && k >= static_cast<unsigned>(SL) &&
                    !lds_wait_geq(&ctl.done[slot], k + 1 - static_cast<unsigned>(SL), spin_limit)) {
                    dev_store(&sync->error[0], 1u);
                    ok = false;
                }
                lds_acquire();
                char* dst = ring + slot * F::SB;
#pragma unroll
                for (int j = 0; j < F::KL; ++j)
                    if (1024 * j + 16 * lane < nbytes[r]) *reinterpret_cast<ru4*>(dst + 1024 * j + 16 * lane) = reg[r][j];
                lds_release();
                if (lane == 0) lds_store(&ctl.ready[slot], k + 1);
#ifdef MLQ_RING_STAMPS
                if (lw == 0) {
                    if (nstg[r] != last_written) RING_STAMP(nstg[r], 20);  // first unit of the stage in LDS
                    last_written = nstg[r];
                    RING_STAMP(nstg[r], 21);  // last unit so far
                }
#endif
                stamp_issue(r);
                nbytes[r] = cur.issue(nstages, lane, reg[r]);
                cur.next(st, nstages, b, G, lw);
                ++k;
                if (++q == SL) q = 0;
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return;
    }

    // ---------------------------------------------------------------- compute
    const int cw = wave - kRingLoaders;
    const int t = static_cast<int>(threadIdx.x) - kRingLoaders * 64;
    unsigned cbar_target = 0;
    bool ok = true;
    unsigned barriers = 0;
    auto meet = [&]() {  // every compute wave of the workgroup
        lds_release();
        if (lane == 0) __hip_atomic_fetch_add(&ctl.cbar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        cbar_target += kRingCompute;
        if (ok && !lds_wait_geq(&ctl.cbar, cbar_target, spin_limit)) {
            dev_store(&sync->error[0], 1u);
            ok = false;
        }
        lds_acquire();
    };
    // Compute waves claim the stage's rows one at a time from an LDS counter
    // (so they finish a stage together).  Row i is loader i % kRingLoaders's
    // row (i / kRingLoaders); kb[l] counts loader l's units before the stage.
    unsigned kb[kRingLoaders];
#pragma unroll
    for (int l = 0; l < kRingLoaders; ++l) kb[l] = 0;
    unsigned claim_base = 0;
    for (int s = 0; s < nstages; ++s) {
        RDesc& S = st[s];
        const int n = ring_rows(S, b, G), nch = S.nch, np = S.np;
        if (cw == 0) RING_STAMP(s, 0);  // stage entered
        if (s > 0) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's y stores have completed
            if (cw == 0) RING_STAMP(s, 1);
            meet();  // every compute wave is done with the old limbs and its stores
            if (cw == 0) RING_STAMP(s, 2);
            if (S.barrier) {
                ++barriers;
                if (cw == 0 && lane == 0) {
                    const unsigned C = G < kSeqGroups ? G : kSeqGroups;
                    const unsigned g = b % C;
                    const unsigned members = (G - g + C - 1) / C;
                    const unsigned old =
                        __hip_atomic_fetch_add(&sync->sub[g][0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (old == barriers * members - 1)
                        __hip_atomic_fetch_add(&sync->top[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    unsigned polls = 0;
                    while (ok && dev_load(&sync->top[0]) < barriers * C) {
                        if (++polls > spin_limit) {
                            dev_store(&sync->error[0], 1u);
                            ok = false;
                        }
                        __builtin_amdgcn_s_sleep(1);
                    }
                }
                meet();  // the grid has passed the barrier
                if (cw == 0) RING_STAMP(s, 3);
            }
        }
        float4* xc = reinterpret_cast<float4*>(xl + np * XLimbs<QT>::PAIR_DW);
        if (S.coherent) {
            ring_stage_x<QT, true>(S, xl, xc, t);
        } else {
            ring_stage_x<QT, false>(S, xl, xc, t);
        }
        if (cw == 0) RING_STAMP(s, 4);
        meet();  // limbs of stage s in LDS
        if (cw == 0) RING_STAMP(s, 5);
        bool first_unit = cw == 0;

        uint32_t xq[XLimbs<QT>::PAIR_DW];
        float4 c0, c1;
        if (nch == 1) load_xq<QT>(xl, xc, min(lane, np - 1), xq, c0, c1);
        for (;;) {
            unsigned ci = 0;
            if (lane == 0) ci = __hip_atomic_fetch_add(&ctl.claim, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            const int i = static_cast<int>(__builtin_amdgcn_readfirstlane(ci) - claim_base);
            if (i >= n) break;
            const int row = b + i * G;
            const int lw = i % kRingLoaders;
            unsigned k = kb[0];
#pragma unroll
            for (int l = 1; l < kRingLoaders; ++l) k = lw == l ? kb[l] : k;
            k += static_cast<unsigned>(i / kRingLoaders * nch);
            int q = static_cast<int>(k % static_cast<unsigned>(SL));
            float acc = 0.0f;
            for (int c = 0; c < nch; ++c) {
                const int slot = lw * SL + q;
                if (first_unit) RING_STAMP(s, 6);
                if (ok && !lds_wait_geq(&ctl.ready[slot], k + 1, spin_limit)) {
                    dev_store(&sync->error[0], 1u);
                    ok = false;
                }
                if (first_unit) RING_STAMP(s, 7);
                first_unit = false;
                lds_acquire();
                const int p = c * 64 + lane;
                if (nch > 1) load_xq<QT>(xl, xc, min(p, np - 1), xq, c0, c1);
                const uint32_t* src = reinterpret_cast<const uint32_t*>(ring + slot * F::SB) + lane * DW;
                uint32_t w[DW];
#pragma unroll
                for (int d = 0; d < DW; ++d) w[d] = src[d];
                const float a = PairDot<QT>::run(w, xq, c0, c1, acc);
                acc = p < np ? a : acc;
                lds_release();  // the slot's reads are complete
                if (lane == 0) lds_store(&ctl.done[slot], k + 1);
                ++k;
                if (++q == SL) q = 0;
            }
            const float v = group_sum<64>(acc);
            if (lane == 63) {
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
        }
        RING_STAMP(s, 8 + cw);  // this compute wave's rows of the stage done
#pragma unroll
        for (int l = 0; l < kRingLoaders; ++l)
            kb[l] += static_cast<unsigned>(n > l ? ((n - l - 1) / kRingLoaders + 1) * nch : 0);
        // Every compute wave has made its last (failed) claim of the stage, one
        // per wave past the stage's n rows.
        claim_base += static_cast<unsigned>(n + kRingCompute);
    }
    // Count out; the last workgroup resets the barrier words for the next launch.
    if (cw == 0 && lane == 0) {
        const unsigned done = __hip_atomic_fetch_add(&sync->exit[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == static_cast<unsigned>(G) - 1) {
            for (int g = 0; g < kSeqGroups; ++g) dev_store(&sync->sub[g][0], 0u);
            dev_store(&sync->top[0], 0u);
            dev_store(&sync->exit[0], 0u);
        }
    }
}

const void* ring_kernel(int qtype) {
    switch (qtype) {
        case 1: return reinterpret_cast<const void*>(&gemv_ring_kernel<1>);
        case 2: return reinterpret_cast<const void*>(&gemv_ring_kernel<2>);
        case 3: return reinterpret_cast<const void*>(&gemv_ring_kernel<3>);
        default: return nullptr;
    }
}

int ring_slot_bytes(int qtype) {
    return qtype == 1 ? RingFmt<1>::SB : qtype == 2 ? RingFmt<2>::SB : RingFmt<3>::SB;
}

}  // namespace

int ring_lds_bytes(int qtype, int kmax, int* nslots) {
    const int x_bytes = (pair_lds_bytes(qtype, (kmax + kQK - 1) / kQK) + 15) & ~15;
    const int sb = ring_slot_bytes(qtype);
    int s = (kRingLdsMax - kRingCtlBytes - x_bytes) / sb;
    s = s > kRingMaxSlots ? kRingMaxSlots : s;
    s -= s % kRingLoaders;  // each loader keeps its own slots
    *nslots = s;
    return kRingCtlBytes + x_bytes + s * sb;
}

hipError_t ring_grid(int qtype, int lds_bytes, int device, int* grid) {
    const void* k = ring_kernel(qtype);
    if (k == nullptr) return hipErrorInvalidValue;
    hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
    if (e != hipSuccess) return e;
    int per_cu = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, kRingThreads, lds_bytes);
    if (e != hipSuccess) return e;
    int cus = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess) return e;
    if (per_cu < 1 || cus < 1) return hipErrorInvalidConfiguration;
    *grid = cus;
    return hipSuccess;
}

hipError_t launch_ring(int qtype, const SeqStageDesc* stages, int nstages, SeqSync* sync, int grid, int lds_bytes,
                       unsigned spin_limit, int kmax, hipStream_t stream) {
    const void* k = ring_kernel(qtype);
    int nslots = 0;
    const int need = ring_lds_bytes(qtype, kmax, &nslots);
    if (k == nullptr || nstages <= 0 || grid <= 0 || lds_bytes != need || nslots < 2 * kRingLoaders) {
        return hipErrorInvalidValue;
    }
    int x_bytes = (pair_lds_bytes(qtype, (kmax + kQK - 1) / kQK) + 15) & ~15;
    void* args[] = {&stages, &nstages, &sync, &spin_limit, &x_bytes, &nslots};
    return hipLaunchKernel(k, dim3(grid), dim3(kRingThreads), args, static_cast<size_t>(lds_bytes), stream);
}

hipError_t ring_stamps_copy(void* host, size_t bytes) {
#ifdef MLQ_RING_STAMPS
    if (bytes != sizeof(g_ring_stamps)) return hipErrorInvalidValue;
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_ring_stamps), bytes);
#else
    (void)host;
    (void)bytes;
    return hipErrorNotSupported;
#endif
}

const char* ring_kernel_name(int qtype) {
    return qtype == 1 ? "gemv_ring_q8_0" : qtype == 2 ? "gemv_ring_q4_0" : "gemv_ring_q4_1";
}

}  // namespace mlq

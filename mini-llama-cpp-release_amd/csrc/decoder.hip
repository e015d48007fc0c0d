// Device-resident decode step (see decoder.h).
//
// Kernels for the ops between the quantized linears -- embedding lookup,
// residual add + RMSNorm, bias + RoPE + KV-cache write, decode attention,
// SwiGLU, an F32 GEMV for unquantized weights (tied embeddings) and the pick
// over F32 logits -- and the host side that loads a GGUF model the way
// load_gguf_model does and sequences one step.  Arithmetic follows the
// reference's f32 ops (src/ops.cpp:18-175, src/forward.cpp:462-726); sums are
// reduced in parallel, so results agree to rounding, not bit for bit.
#include "decoder.h"

#include "gguf_index.h"
#include "mlq_kernels.h"
#include "pick_key.h"
#include "xsplit_device.h"

#include "../../include/mlq_hip.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <string>

namespace mlq {

namespace {

constexpr int kNormThreads = 1024;
constexpr int kAttnThreads = 256;
// Decode attention: threads per head (>= head_dim) and cache rows in flight
// per lane group.  LLaMA-7B shape on MI355X, decode at positions 4..131:
// 256 threads 760.5-761.1 tokens/s, 512 threads 754.6-755.5 (4 rows ahead
// both); 256 x 8 rows 757, 1024 x 2 rows 716.
constexpr int kFlashThreads = 256;
constexpr int kFlashAhead = 4;
static_assert(kFlashThreads >= 256, "the RoPE step gives one thread per element of a head of up to 256");
constexpr int kMaxHeadDim = 256;
// Decode attention splits a head's positions over up to kAttnMaxSplits
// workgroups once there are more than kAttnSplitRows of them.
constexpr int kAttnSplitRows = 128;
constexpr int kAttnMaxSplits = 8;

// Sum (or max) over a workgroup of `nthreads`; every thread gets the result.
template <int NT, bool MAX>
__device__ __forceinline__ float wg_reduce(float v, float* part) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float w = __shfl_xor(v, o, 64);
        v = MAX ? fmaxf(v, w) : v + w;
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = part[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) r = MAX ? fmaxf(r, part[i]) : r + part[i];
    return r;
}

// x[dim] = embedding[token] (embed_token, src/forward.cpp:496-503).  A token
// out of range flags the step and reads row 0.
__global__ __launch_bounds__(256) void embed_kernel(const float* __restrict__ emb, int vocab, int dim,
                                                    DecodeState* st, float* __restrict__ x) {
    const int t = st->token;
    const bool ok = t >= 0 && t < vocab;
    if (!ok && blockIdx.x == 0 && threadIdx.x == 0) st->error |= kDecodeErrToken;
    const size_t row = static_cast<size_t>(ok ? t : 0) * dim;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < dim; i += gridDim.x * blockDim.x) x[i] = emb[row + i];
}

// x += delta (when given; forward_add) then out = rmsnorm(x) * w
// (rmsnorm, src/ops.cpp:18-41: mean of squares, 1 / sqrt(ms + eps)).
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(float* __restrict__ x,
                                                                   const float* __restrict__ delta,
                                                                   const float* __restrict__ w, int dim, float eps,
                                                                   float* __restrict__ out) {
    __shared__ float part[kNormThreads / 64];
    float ss = 0.0f;
    for (int i = threadIdx.x; i < dim; i += kNormThreads) {
        float v = x[i];
        if (delta != nullptr) {
            v = v + delta[i];
            x[i] = v;
        }
        ss += v * v;
    }
    ss = wg_reduce<kNormThreads, false>(ss, part);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(dim) + eps);
    for (int i = threadIdx.x; i < dim; i += kNormThreads) out[i] = x[i] * scale * w[i];
}

// The same for dim <= 4 * kNormThreads * VEC (x 16-byte aligned, dim % 4 == 0):
// every thread loads its float4s of x, delta and w once, keeps them in
// registers through the reduction and stores the results (one round trip to
// memory instead of three).
template <int VEC>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_vec_kernel(float* __restrict__ x,
                                                                       const float* __restrict__ delta,
                                                                       const float* __restrict__ w, int dim, float eps,
                                                                       float* __restrict__ out) {
    __shared__ float part[kNormThreads / 64];
    const int n4 = dim / 4;
    float4 xv[VEC], wv[VEC];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
        const int i = threadIdx.x + j * kNormThreads;
        const int ic = min(i, n4 - 1);
        float4 a = reinterpret_cast<const float4*>(x)[ic];
        wv[j] = reinterpret_cast<const float4*>(w)[ic];
        if (delta != nullptr) {
            const float4 d = reinterpret_cast<const float4*>(delta)[ic];
            a.x = a.x + d.x;
            a.y = a.y + d.y;
            a.z = a.z + d.z;
            a.w = a.w + d.w;
        }
        xv[j] = a;
        if (i < n4) ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
    }
    ss = wg_reduce<kNormThreads, false>(ss, part);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(dim) + eps);
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
        const int i = threadIdx.x + j * kNormThreads;
        if (i < n4) {
            const float4 a = xv[j];
            if (delta != nullptr) reinterpret_cast<float4*>(x)[i] = a;
            reinterpret_cast<float4*>(out)[i] = make_float4(a.x * scale * wv[j].x, a.y * scale * wv[j].y,
                                                            a.z * scale * wv[j].z, a.w * scale * wv[j].w);
        }
    }
}

// Optional q/k/v biases, RoPE on q and k (src/ops.cpp:109-175: normal pairs
// (2r, 2r+1) or NeoX pairs (r, r + hd/2), angle pos / theta^(2r/hd)), and
// the KV-cache write at [layer][pos][kv head][d] (KVCache::write).
__global__ __launch_bounds__(256) void rope_kv_kernel(float* __restrict__ q, float* __restrict__ k,
                                                      const float* __restrict__ v, const float* __restrict__ bq,
                                                      const float* __restrict__ bk, const float* __restrict__ bv,
                                                      int n_heads, int n_kv, int hd, float theta, int neox,
                                                      int max_seq, int layer, DecodeState* st,
                                                      float* __restrict__ kc, float* __restrict__ vc) {
    const int p0 = st->pos;
    const bool ok = p0 >= 0 && p0 < max_seq;
    if (!ok && blockIdx.x == 0 && threadIdx.x == 0) st->error |= kDecodeErrPos;
    const int pos = ok ? p0 : 0;
    const int half = hd / 2;
    const int nq = n_heads * half;
    const int nk = n_kv * half;
    const int nv = n_kv * hd;
    const size_t cache_row = (static_cast<size_t>(layer) * max_seq + pos) * n_kv * hd;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < nq + nk) {
        const bool is_q = i < nq;
        const int j = is_q ? i : i - nq;
        const int h = j / half;
        const int r = j % half;
        const int i0 = h * hd + (neox ? r : 2 * r);
        const int i1 = neox ? i0 + half : i0 + 1;
        const float freq = 1.0f / powf(theta, static_cast<float>(2 * r) / static_cast<float>(hd));
        const float ang = static_cast<float>(pos) * freq;
        const float c = cosf(ang);
        const float s = sinf(ang);
        float* t = is_q ? q : k;
        const float* b = is_q ? bq : bk;
        float a0 = t[i0];
        float a1 = t[i1];
        if (b != nullptr) {
            a0 = a0 + b[i0];
            a1 = a1 + b[i1];
        }
        const float r0 = a0 * c - a1 * s;
        const float r1 = a0 * s + a1 * c;
        t[i0] = r0;
        t[i1] = r1;
        if (!is_q) {
            kc[cache_row + i0] = r0;
            kc[cache_row + i1] = r1;
        }
    } else if (i < nq + nk + nv) {
        const int e = i - nq - nk;
        vc[cache_row + e] = bv != nullptr ? v[e] + bv[e] : v[e];
    }
}

// One workgroup per query head (attention_forward, src/forward.cpp:583-607):
// scores q.k_t / sqrt(hd) for t <= pos, softmax (max, exp, sum, divide),
// then sum_t p_t v_t.  Scores live in global scratch [head][max_seq].
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(const float* __restrict__ q,
                                                                 const float* __restrict__ kc,
                                                                 const float* __restrict__ vc,
                                                                 float* __restrict__ scores, float* __restrict__ out,
                                                                 int n_heads, int n_kv, int hd, int max_seq, int layer,
                                                                 const DecodeState* st) {
    __shared__ float qs[kMaxHeadDim];
    __shared__ float part[kAttnThreads / 64];
    __shared__ float acc_part[kAttnThreads];
    const int h = blockIdx.x;
    const int kvh = h / (n_heads / n_kv);
    const int p0 = st->pos;
    const int pos = (p0 >= 0 && p0 < max_seq) ? p0 : 0;
    float* sc = scores + static_cast<size_t>(h) * max_seq;
    const size_t layer_base = static_cast<size_t>(layer) * max_seq * n_kv * hd;
    const size_t t_stride = static_cast<size_t>(n_kv) * hd;
    for (int d = threadIdx.x; d < hd; d += kAttnThreads) qs[d] = q[h * hd + d];
    __syncthreads();
    const float scale = 1.0f / sqrtf(static_cast<float>(hd));
    float lmax = -INFINITY;
    for (int t = threadIdx.x; t <= pos; t += kAttnThreads) {
        const float* kp = kc + layer_base + t * t_stride + kvh * hd;
        float dot = 0.0f;
        for (int d = 0; d < hd; ++d) dot += qs[d] * kp[d];
        const float s = dot * scale;
        sc[t] = s;
        lmax = fmaxf(lmax, s);
    }
    const float m = wg_reduce<kAttnThreads, true>(lmax, part);
    float lsum = 0.0f;
    for (int t = threadIdx.x; t <= pos; t += kAttnThreads) {
        const float e = expf(sc[t] - m);
        sc[t] = e;
        lsum += e;
    }
    const float sum = wg_reduce<kAttnThreads, false>(lsum, part);
    for (int t = threadIdx.x; t <= pos; t += kAttnThreads) sc[t] = sc[t] / sum;
    __syncthreads();
    // Output: thread (g, d) sums t = g, g + G, ... for dimension d.
    const int groups = kAttnThreads / hd;
    const int g = threadIdx.x / hd;
    const int d = threadIdx.x % hd;
    float acc = 0.0f;
    if (g < groups) {
        for (int t = g; t <= pos; t += groups) acc += sc[t] * vc[layer_base + t * t_stride + kvh * hd + d];
    }
    acc_part[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x < hd) {
        float r = 0.0f;
        for (int gg = 0; gg < groups; ++gg) r += acc_part[gg * hd + threadIdx.x];
        out[h * hd + threadIdx.x] = r;
    }
}

// Sum over aligned groups of LPR lanes (a power of two up to 64), in every
// lane of the group: DPP within rows of 16, one swizzle across the two rows
// of a 32-lane half, a shuffle across halves.
template <int LPR>
__device__ __forceinline__ float lane_group_sum(float v) {
#define MLQ_ATTN_DPP(x, ctrl) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (x)), (ctrl), 0xF, 0xF, false))
    if (LPR >= 2) v += MLQ_ATTN_DPP(v, 0xB1);   // quad_perm [1,0,3,2]
    if (LPR >= 4) v += MLQ_ATTN_DPP(v, 0x4E);   // quad_perm [2,3,0,1]
    if (LPR >= 8) v += MLQ_ATTN_DPP(v, 0x141);  // row_half_mirror: 8-lane sums
    if (LPR >= 16) v += MLQ_ATTN_DPP(v, 0x140); // row_mirror: 16-lane sums
#undef MLQ_ATTN_DPP
    if (LPR >= 32) v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
    if (LPR >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// Decode attention for one query head per workgroup with the step's RoPE,
// biases and KV-cache write folded in (head_dim = 4 * LPR, a power of two up
// to 256).  Each workgroup rotates its q head and its kv head's k (as
// rope_kv_kernel does), uses this position's k and v from LDS and writes them
// to the cache; earlier positions come from the cache.  A cache row is read
// as LPR float4s by LPR lanes, ROWS = kFlashThreads / LPR rows at a time, so every load
// is a coalesced row segment.  The softmax is folded into the same pass
// (running maximum, sum and weighted v per row group, rescaled when the
// maximum grows), and the row groups are merged once at the end:
// sum_t e^(s_t - m) v_t / sum_t e^(s_t - m), the reference's
// softmax-then-sum to rounding.
// Latency structure (measured with in-kernel timestamps on MI355X): q, k, v
// are requested together with the position, the first pass's cache rows
// right after it (before the RoPE math), and the KV-cache row is stored
// before the first pass without being waited for -- every load and store
// here is unconditional (clamped indices; the query heads of one kv group
// store identical values), since a load or store inside a branch makes the
// compiler wait for all outstanding memory operations at the join.  The
// AHEAD rows of a pass are reduced together (DPP, no LDS round trips per
// step) and folded into the running softmax with selects.
// Long contexts: workgroup (h, s) of the grid's nsplit per head takes the s-th
// of S = min(nsplit, ceil((pos + 1) / kAttnSplitRows)) equal runs of
// positions (workgroups past S return at once; S = 1 is the single-workgroup
// path).  Each writes its (maximum, sum, weighted V) with agent-scope stores
// to part[h][s], waits for them, and counts in on cnt[h]; the last to arrive
// resets the count (graph replays need no memset) and merges the S states in
// split order — the protocol of the GEMM's split-K reduction.
template <int LPR>
__global__ __launch_bounds__(kFlashThreads) void attention_rope_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ bq, const float* __restrict__ bk, const float* __restrict__ bv, int n_heads, int n_kv,
    float theta, int neox, int max_seq, int layer, DecodeState* st, float* __restrict__ kc,
    float* __restrict__ vc, float* __restrict__ out, float* __restrict__ part, unsigned* __restrict__ cnt,
    int nsplit) {
    constexpr int HD = 4 * LPR;
    constexpr int ROWS = kFlashThreads / LPR;
    constexpr int AHEAD = kFlashAhead;
    __shared__ float4 qs4[LPR], ks4[LPR], vs4[LPR];
    __shared__ float gm[ROWS], gl[ROWS];
    __shared__ float4 gacc[ROWS][LPR];
    float* qs = reinterpret_cast<float*>(qs4);
    float* ks = reinterpret_cast<float*>(ks4);
    float* vs = reinterpret_cast<float*>(vs4);
    const int tid = threadIdx.x;
    const int h = blockIdx.x;
    const int group = n_heads / n_kv;
    const int kvh = h / group;
    const int half = HD / 2;
    // Threads 0..half-1 rotate pair tid of q, threads half..HD-1 pair
    // tid - half of k; every thread adds v's bias for element tid.  Threads
    // past HD load the last pair / element again; an absent bias reads the
    // value itself and adds zero.
    const bool is_q = tid < half;
    const int r = min(is_q ? tid : tid - half, half - 1);
    const int i0 = neox ? r : 2 * r;
    const int i1 = neox ? i0 + half : i0 + 1;
    const int te = min(tid, HD - 1);
    const float* src = is_q ? q + h * HD : k + kvh * HD;
    const bool has_b = is_q ? bq != nullptr : bk != nullptr;
    const float* bsrc = has_b ? (is_q ? bq + h * HD : bk + kvh * HD) : src;
    const float* bvsrc = bv != nullptr ? bv + kvh * HD : v + kvh * HD;
    float a0 = src[i0];
    float a1 = src[i1];
    float ve = v[kvh * HD + te];
    const float b0 = bsrc[i0], b1 = bsrc[i1], bve = bvsrc[te];
    a0 += has_b ? b0 : 0.0f;
    a1 += has_b ? b1 : 0.0f;
    ve += bv != nullptr ? bve : 0.0f;
    const size_t layer_base = static_cast<size_t>(layer) * max_seq * n_kv * HD;
    const size_t t_stride = static_cast<size_t>(n_kv) * HD;
    const float* kbase = kc + layer_base + kvh * HD;
    const float* vbase = vc + layer_base + kvh * HD;
    const int lr = tid / LPR;
    const int li = tid % LPR;
    // The first pass's cache rows of the run that starts at position 0 (split
    // 0), requested before the position word is back: they do not depend on
    // it.  Rows at or past the position (this step's row, or rows of an older,
    // longer generation) are selected away in the pass; a split that starts
    // later requests its own rows once the position is known.
    float4 kr[AHEAD], vr[AHEAD];
#pragma unroll
    for (int j = 0; j < AHEAD; ++j) {
        const int tj = min(lr + j * ROWS, max_seq - 1);
        kr[j] = *reinterpret_cast<const float4*>(kbase + tj * t_stride + 4 * li);
        vr[j] = *reinterpret_cast<const float4*>(vbase + tj * t_stride + 4 * li);
    }

    const int p0 = st->pos;
    const bool ok = p0 >= 0 && p0 < max_seq;
    const int split = blockIdx.y;
    if (!ok && h == 0 && split == 0 && tid == 0) st->error |= kDecodeErrPos;
    const int pos = ok ? p0 : 0;
    const int S = min(nsplit, (pos + kAttnSplitRows) / kAttnSplitRows);  // ceil((pos + 1) / kAttnSplitRows)
    if (split >= S) return;
    const int chunk = (pos + S) / S;  // ceil((pos + 1) / S)
    const int t_begin = split * chunk;
    const int t_end = min(pos + 1, t_begin + chunk);  // this workgroup's positions: [t_begin, t_end)
    // Rows read from the cache stay below pos and inside the run.
    const int last = max(min(t_end, pos) - 1, 0);
    if (t_begin != 0) {  // a later split: its first pass, ahead of the RoPE math
#pragma unroll
        for (int j = 0; j < AHEAD; ++j) {
            const int tj = min(t_begin + lr + j * ROWS, last);
            kr[j] = *reinterpret_cast<const float4*>(kbase + tj * t_stride + 4 * li);
            vr[j] = *reinterpret_cast<const float4*>(vbase + tj * t_stride + 4 * li);
        }
    }
    if (tid < HD) {
        const float freq = 1.0f / powf(theta, static_cast<float>(2 * r) / static_cast<float>(HD));
        const float ang = static_cast<float>(pos) * freq;
        const float c = cosf(ang);
        const float sn = sinf(ang);
        float* dst = is_q ? qs : ks;
        dst[i0] = a0 * c - a1 * sn;
        dst[i1] = a0 * sn + a1 * c;
        vs[tid] = ve;
    }
    __syncthreads();
    kc[layer_base + pos * t_stride + kvh * HD + te] = ks[te];
    vc[layer_base + pos * t_stride + kvh * HD + te] = vs[te];

    const float4 qv = qs4[li];
    const float4 kp = ks4[li];
    const float4 vp = vs4[li];
    const float scale = 1.0f / sqrtf(static_cast<float>(HD));
    float m = -INFINITY;
    float l = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    auto pass = [&](int t0, const float4 (&kc4)[AHEAD], const float4 (&vc4)[AHEAD]) {
        float dot[AHEAD];
#pragma unroll
        for (int j = 0; j < AHEAD; ++j) {
            const float4 kv = t0 + j * ROWS == pos ? kp : kc4[j];
            dot[j] = lane_group_sum<LPR>(qv.x * kv.x + qv.y * kv.y + qv.z * kv.z + qv.w * kv.w);
        }
        // Rows past the run (clamped re-reads, or at pos 0 a cache row not
        // yet written) are selected away before any arithmetic touches them.
#pragma unroll
        for (int j = 0; j < AHEAD; ++j) {
            const int t = t0 + j * ROWS;
            const bool in = t < t_end;
            const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const float4 vv = t == pos ? vp : in ? vc4[j] : z4;
            const float sc = in ? dot[j] * scale : 0.0f;
            const float mn = in ? fmaxf(m, sc) : m;
            const float c_old = in ? expf(m - mn) : 1.0f;
            const float p = in ? expf(sc - mn) : 0.0f;
            l = l * c_old + p;
            acc.x = acc.x * c_old + p * vv.x;
            acc.y = acc.y * c_old + p * vv.y;
            acc.z = acc.z * c_old + p * vv.z;
            acc.w = acc.w * c_old + p * vv.w;
            m = mn;
        }
    };
    pass(t_begin + lr, kr, vr);
    if (t_begin + lr + AHEAD * ROWS < t_end) {
        // Longer runs: the following passes, each requesting the next.
#pragma unroll
        for (int j = 0; j < AHEAD; ++j) {
            const int tj = min(t_begin + lr + (AHEAD + j) * ROWS, last);
            kr[j] = *reinterpret_cast<const float4*>(kbase + tj * t_stride + 4 * li);
            vr[j] = *reinterpret_cast<const float4*>(vbase + tj * t_stride + 4 * li);
        }
        for (int t0 = t_begin + lr + AHEAD * ROWS; t0 < t_end; t0 += AHEAD * ROWS) {
            float4 kc4[AHEAD], vc4[AHEAD];
#pragma unroll
            for (int j = 0; j < AHEAD; ++j) {
                kc4[j] = kr[j];
                vc4[j] = vr[j];
            }
            if (t0 + AHEAD * ROWS < t_end) {
#pragma unroll
                for (int j = 0; j < AHEAD; ++j) {
                    const int tj = min(t0 + (AHEAD + j) * ROWS, last);
                    kr[j] = *reinterpret_cast<const float4*>(kbase + tj * t_stride + 4 * li);
                    vr[j] = *reinterpret_cast<const float4*>(vbase + tj * t_stride + 4 * li);
                }
            }
            pass(t0, kc4, vc4);
        }
    }
    if (li == 0) {
        gm[lr] = m;
        gl[lr] = l;
    }
    gacc[lr][li] = acc;
    __syncthreads();
    if (tid < HD) {
        float mx = -INFINITY;
#pragma unroll
        for (int g = 0; g < ROWS; ++g) mx = fmaxf(mx, gm[g]);
        const int c4 = tid / 4;
        const int e = tid % 4;
        float num = 0.0f;
        float den = 0.0f;
#pragma unroll
        for (int g = 0; g < ROWS; ++g) {
            const bool rows = gm[g] != -INFINITY;  // false: a group without rows (pos + 1 < ROWS)
            const float w = rows ? expf(gm[g] - mx) : 0.0f;
            const float4 a = gacc[g][c4];
            num += rows ? w * (e == 0 ? a.x : e == 1 ? a.y : e == 2 ? a.z : a.w) : 0.0f;
            den += rows ? w * gl[g] : 0.0f;
        }
        if (S == 1) {
            out[h * HD + tid] = num / den;
        } else {
            float* ps = part + (static_cast<size_t>(h) * nsplit + split) * (HD + 2);
            if (tid == 0) {
                __hip_atomic_store(ps, mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(ps + 1, den, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __hip_atomic_store(ps + 2 + tid, num, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (S == 1) return;
    // Count in once this workgroup's state has reached the point of coherence.
    __shared__ unsigned last_in;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        const unsigned done = __hip_atomic_fetch_add(cnt + h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_in = done == static_cast<unsigned>(S) - 1 ? 1u : 0u;
        if (last_in) __hip_atomic_store(cnt + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (last_in == 0u || tid >= HD) return;
    const float* ph = part + static_cast<size_t>(h) * nsplit * (HD + 2);
    float mx = -INFINITY;
    for (int j = 0; j < S; ++j) mx = fmaxf(mx, __hip_atomic_load(ph + j * (HD + 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    float num = 0.0f;
    float den = 0.0f;
    for (int j = 0; j < S; ++j) {
        const float* pj = ph + j * (HD + 2);
        const float w = expf(__hip_atomic_load(pj, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - mx);
        den += w * __hip_atomic_load(pj + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        num += w * __hip_atomic_load(pj + 2 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    out[h * HD + tid] = num / den;
}

// ---- Batched prefill (rows r = 0..n-1 at positions start + r) ----

// X[r] = embedding[tokens[r]].
__global__ __launch_bounds__(256) void embed_rows_kernel(const float* __restrict__ emb, int vocab, int dim,
                                                         const int32_t* __restrict__ tokens, DecodeState* st,
                                                         float* __restrict__ X) {
    const int r = blockIdx.y;
    const int t = tokens[r];
    const bool ok = t >= 0 && t < vocab;
    if (!ok && blockIdx.x == 0 && threadIdx.x == 0) st->error |= kDecodeErrToken;
    const size_t row = static_cast<size_t>(ok ? t : 0) * dim;
    float* x = X + static_cast<size_t>(r) * dim;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < dim; i += gridDim.x * blockDim.x) x[i] = emb[row + i];
}

// One workgroup per row: X[r] += D[r] (when given), H[r] = rmsnorm(X[r]) * w.
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_rows_kernel(float* __restrict__ X,
                                                                        const float* __restrict__ D,
                                                                        const float* __restrict__ w, int dim,
                                                                        float eps, float* __restrict__ H) {
    __shared__ float part[kNormThreads / 64];
    const size_t off = static_cast<size_t>(blockIdx.x) * dim;
    float* x = X + off;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < dim; i += kNormThreads) {
        float v = x[i];
        if (D != nullptr) {
            v = v + D[off + i];
            x[i] = v;
        }
        ss += v * v;
    }
    ss = wg_reduce<kNormThreads, false>(ss, part);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(dim) + eps);
    for (int i = threadIdx.x; i < dim; i += kNormThreads) H[off + i] = x[i] * scale * w[i];
}

// Row kernels whose output goes straight to a prefill GEMM as its split x
// (xsplit_device.h; the GEMM then makes no split launch of its own).
// Workgroup `row` of 256 threads holds the row's half blocks in registers
// (thread t: half blocks t + 256 c); rows n .. npad - 1 write a zero split
// (the GEMM's padded token tile).  C = ceil(2 nb / 256) half blocks per
// thread (dim = 32 nb <= 256 * 16 * kXsCache).
//
// add_rmsnorm_rows_kernel's step for a GEMM input: X[r] += D[r] (when given),
// then the split of rmsnorm(X[r]) * w.
template <int QT, int C>
__global__ __launch_bounds__(256) void add_rmsnorm_split_rows_kernel(float* __restrict__ X,
                                                                     const float* __restrict__ D,
                                                                     const float* __restrict__ w, int dim, float eps,
                                                                     int n, int nb, _Float16* __restrict__ xs,
                                                                     float* __restrict__ bsum,
                                                                     float* __restrict__ scale) {
    __shared__ float part[4];
    const int row = blockIdx.x;
    const bool valid = row < n;
    const size_t off = static_cast<size_t>(valid ? row : 0) * dim;
    float v[C][16], wv[C][16];
    float ss = 0.0f;
    // Every load is unconditional (half blocks past the row re-read the last
    // one, D absent reads X again; both are selected away): a load under a
    // branch makes the compiler wait for it at the join, one round trip per
    // half block.  The norm weights are requested with the row.
    const float* const Dp = D != nullptr ? D + off : X + off;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int k0 = min(16 * (static_cast<int>(threadIdx.x) + 256 * c), dim - 16);
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const float4 a = *reinterpret_cast<const float4*>(w + k0 + i);
            wv[c][i] = a.x;
            wv[c][i + 1] = a.y;
            wv[c][i + 2] = a.z;
            wv[c][i + 3] = a.w;
        }
    }
    float dv[C][16];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int k0 = min(16 * (static_cast<int>(threadIdx.x) + 256 * c), dim - 16);
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const float4 a = *reinterpret_cast<const float4*>(X + off + k0 + i);
            const float4 d = *reinterpret_cast<const float4*>(Dp + k0 + i);
            v[c][i] = a.x;
            v[c][i + 1] = a.y;
            v[c][i + 2] = a.z;
            v[c][i + 3] = a.w;
            dv[c][i] = d.x;
            dv[c][i + 1] = d.y;
            dv[c][i + 2] = d.z;
            dv[c][i + 3] = d.w;
        }
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int k0 = 16 * (static_cast<int>(threadIdx.x) + 256 * c);
        const bool in = valid && k0 < dim;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float a = D != nullptr ? v[c][i] + dv[c][i] : v[c][i];
            v[c][i] = in ? a : 0.0f;
            ss += v[c][i] * v[c][i];
        }
        if (in && D != nullptr) {
#pragma unroll
            for (int i = 0; i < 16; i += 4)
                *reinterpret_cast<float4*>(X + off + k0 + i) =
                    make_float4(v[c][i], v[c][i + 1], v[c][i + 2], v[c][i + 3]);
        }
    }
    ss = wg_reduce<256, false>(ss, part);
    const float sc = 1.0f / sqrtf(ss / static_cast<float>(dim) + eps);
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int k0 = 16 * (static_cast<int>(threadIdx.x) + 256 * c);
        if (valid && k0 < dim) {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[c][i] = v[c][i] * sc * wv[c][i];
        }
    }
    __syncthreads();  // part is reused by the split's maximum
    xsplit_emit_row<QT, C>(row, nb, v, xs, bsum, scale, part);
}

// swiglu_kernel's step for a GEMM input: the split of silu(g) * u per row.
template <int QT, int C>
__global__ __launch_bounds__(256) void swiglu_split_rows_kernel(const float* __restrict__ G,
                                                                const float* __restrict__ U, int hidden, int n,
                                                                int nb, _Float16* __restrict__ xs,
                                                                float* __restrict__ bsum, float* __restrict__ scale) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    const bool valid = row < n;
    const size_t off = static_cast<size_t>(valid ? row : 0) * hidden;
    float v[C][16], uv[C][16];
    // Unconditional loads (half blocks past the row re-read the last one and
    // are selected away), all issued before any is used.
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int k0 = min(16 * (static_cast<int>(threadIdx.x) + 256 * c), hidden - 16);
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const float4 g = *reinterpret_cast<const float4*>(G + off + k0 + i);
            const float4 u = *reinterpret_cast<const float4*>(U + off + k0 + i);
            v[c][i] = g.x;
            v[c][i + 1] = g.y;
            v[c][i + 2] = g.z;
            v[c][i + 3] = g.w;
            uv[c][i] = u.x;
            uv[c][i + 1] = u.y;
            uv[c][i + 2] = u.z;
            uv[c][i + 3] = u.w;
        }
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int k0 = 16 * (static_cast<int>(threadIdx.x) + 256 * c);
        const bool in = valid && k0 < hidden;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float gv = v[c][i];
            const float sig = 1.0f / (1.0f + expf(-gv));
            v[c][i] = in ? gv * sig * uv[c][i] : 0.0f;
        }
    }
    xsplit_emit_row<QT, C>(row, nb, v, xs, bsum, scale, red);
}

// rope_kv_kernel for every row (position start + r): workgroups (0 .. R-1,
// row) rotate the row's q heads in place and write the rotated k heads to the
// cache (k itself is left as it was: only the cache is read after this);
// workgroups (R.., row), when launched, copy v (+ bias) to the cache (without
// a v bias the q/k/v GEMM writes v into the cache itself).  Thread (hg, r) of rotating
// workgroup b computes the angle of pair r once (the same expressions as
// rope_kv_kernel, so the same values) and applies it to heads
// b HG + hg, (b + R) HG + hg, ... of q and then k (HG = 256 / (hd / 2)): one
// cosf / sinf / powf per pair index and workgroup instead of one per rotated
// pair.
__global__ __launch_bounds__(256) void rope_kv_rows_kernel(float* __restrict__ Q, float* __restrict__ K,
                                                           const float* __restrict__ V, const float* __restrict__ bq,
                                                           const float* __restrict__ bk, const float* __restrict__ bv,
                                                           int n_heads, int n_kv, int hd, float theta, int neox,
                                                           int max_seq, int layer, int start, float* __restrict__ kc,
                                                           float* __restrict__ vc, int rot_wgs) {
    const int row = blockIdx.y;
    const int pos = start + row;
    const int half = hd / 2;
    const int nv = n_kv * hd;
    const size_t cache_row = (static_cast<size_t>(layer) * max_seq + pos) * nv;
    if (static_cast<int>(blockIdx.x) >= rot_wgs) {
        const int e = (blockIdx.x - rot_wgs) * blockDim.x + threadIdx.x;
        const float* v = V + static_cast<size_t>(row) * nv;
        if (e < nv) vc[cache_row + e] = bv != nullptr ? v[e] + bv[e] : v[e];
        return;
    }
    const int HG = static_cast<int>(blockDim.x) / half;  // head groups (hd <= 512)
    const int hg = threadIdx.x / half;
    const int r = threadIdx.x % half;
    if (hg >= HG) return;
    float* q = Q + static_cast<size_t>(row) * n_heads * hd;
    float* k = K + static_cast<size_t>(row) * nv;
    const float freq = 1.0f / powf(theta, static_cast<float>(2 * r) / static_cast<float>(hd));
    const float ang = static_cast<float>(pos) * freq;
    const float c = cosf(ang);
    const float sn = sinf(ang);
    const int o0 = neox ? r : 2 * r;
    const int o1 = neox ? r + half : 2 * r + 1;
    for (int h = blockIdx.x * HG + hg; h < n_heads + n_kv; h += rot_wgs * HG) {
        const bool is_q = h < n_heads;
        const int hh = is_q ? h : h - n_heads;
        float* t = (is_q ? q : k) + hh * hd;
        const float* b = is_q ? bq : bk;
        float a0 = t[o0];
        float a1 = t[o1];
        if (b != nullptr) {
            a0 = a0 + b[hh * hd + o0];
            a1 = a1 + b[hh * hd + o1];
        }
        const float r0 = a0 * c - a1 * sn;
        const float r1 = a0 * sn + a1 * c;
        // rotated q in place (attention reads it); rotated k only into the cache
        float* dst = is_q ? t : kc + cache_row + hh * hd;
        dst[o0] = r0;
        dst[o1] = r1;
    }
}

// Causal attention of prefill rows: workgroup (head h, query rows r0 ..
// r0 + QR - 1) attends from positions start + r over cache rows 0 .. start + r
// (all written before).  A cache row is read by a group of LPR lanes, V4
// float4s per lane (float4 li + LPR v: each load is a coalesced row segment),
// ROWS = 256 / LPR rows per pass plus A - 1 passes in flight.  Each cache row
// is read once for the QR query rows.  Per pass a lane group takes the scores
// of its A rows, then updates its running maximum, sum and weighted V once
// (one rescale per pass, not per row); rows past a query's position enter
// through selects.  At the end the groups of a wave are merged with a
// butterfly of shuffles and the waves through LDS, in a fixed order.  The
// result equals the reference's max - exp - sum - divide - weighted sum to
// rounding (src/forward.cpp:584-611 and src/ops.cpp:43-71 for one row).  Several float4s per lane
// put more rows in each wave instruction: the score reductions and the
// softmax arithmetic, which every lane of a group repeats, are shared by
// more rows.
constexpr int kPrefillAttnThreads = 256;
template <int LPR, int V4, int QR, int A>
__global__ __launch_bounds__(kPrefillAttnThreads) void attention_rows_kernel(const float* __restrict__ Q,
                                                                             const float* __restrict__ kc,
                                                                             const float* __restrict__ vc, int n_heads,
                                                                             int n_kv, int max_seq, int layer,
                                                                             int start, int n, float* __restrict__ out) {
    constexpr int HD = 4 * LPR * V4;
    constexpr int NT = kPrefillAttnThreads;
    constexpr int ROWS = NT / LPR;
    constexpr int NW = NT / 64;
    static_assert(LPR <= 64 && 64 % LPR == 0, "lane groups within a wave");
    __shared__ float gm[QR][NW], gl[QR][NW];
    __shared__ float4 gacc[QR][NW][LPR * V4];
    const int tid = threadIdx.x;
    const int h = blockIdx.x;
    const int r0 = blockIdx.y * QR;
    const int kvh = h / (n_heads / n_kv);
    const size_t layer_base = static_cast<size_t>(layer) * max_seq * n_kv * HD;
    const size_t t_stride = static_cast<size_t>(n_kv) * HD;
    const float* kbase = kc + layer_base + kvh * HD;
    const float* vbase = vc + layer_base + kvh * HD;
    const int lr = tid / LPR;
    const int li = tid % LPR;
    // Query rows past n repeat row n - 1 (their results are not stored).
    float4 qv[QR][V4];
    int posq[QR];
#pragma unroll
    for (int q = 0; q < QR; ++q) {
        const int row = min(r0 + q, n - 1);
        posq[q] = start + row;
        const float* qrow = Q + static_cast<size_t>(row) * n_heads * HD + h * HD;
#pragma unroll
        for (int v = 0; v < V4; ++v) qv[q][v] = *reinterpret_cast<const float4*>(qrow + 4 * (li + LPR * v));
    }
    const int pos = posq[QR - 1];  // the last query row sees the most cache rows
    const float scale = 1.0f / sqrtf(static_cast<float>(HD));
    float m[QR], l[QR];
    float4 acc[QR][V4];
#pragma unroll
    for (int q = 0; q < QR; ++q) {
        m[q] = -INFINITY;
        l[q] = 0.0f;
#pragma unroll
        for (int v = 0; v < V4; ++v) acc[q][v] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    // Cache rows past pos re-read row pos (they are masked for every query).
    auto load_rows = [&](int t0, float4 (&kr)[A][V4], float4 (&vr)[A][V4]) {
#pragma unroll
        for (int j = 0; j < A; ++j) {
            const int tj = min(t0 + j * ROWS, pos);
#pragma unroll
            for (int v = 0; v < V4; ++v) {
                kr[j][v] = *reinterpret_cast<const float4*>(kbase + tj * t_stride + 4 * (li + LPR * v));
                vr[j][v] = *reinterpret_cast<const float4*>(vbase + tj * t_stride + 4 * (li + LPR * v));
            }
        }
    };
    auto pass = [&](int t0, const float4 (&kc4)[A][V4], const float4 (&vc4)[A][V4]) {
#pragma unroll
        for (int q = 0; q < QR; ++q) {
            float sc[A];
            float bm = -INFINITY;
#pragma unroll
            for (int j = 0; j < A; ++j) {
                float d = 0.0f;
#pragma unroll
                for (int v = 0; v < V4; ++v)
                    d += qv[q][v].x * kc4[j][v].x + qv[q][v].y * kc4[j][v].y + qv[q][v].z * kc4[j][v].z +
                         qv[q][v].w * kc4[j][v].w;
                d = lane_group_sum<LPR>(d);
                const bool in = t0 + j * ROWS <= posq[q];
                sc[j] = in ? d * scale : -INFINITY;
                bm = fmaxf(bm, sc[j]);
            }
            const float mn = fmaxf(m[q], bm);
            const float base = mn == -INFINITY ? 0.0f : mn;  // no row of this query yet
            const float c_old = expf(m[q] - base);            // 0 while the running state is empty
            float p[A];
            float ps = 0.0f;
#pragma unroll
            for (int j = 0; j < A; ++j) {
                p[j] = expf(sc[j] - base);  // 0 for masked rows
                ps += p[j];
            }
            l[q] = l[q] * c_old + ps;
#pragma unroll
            for (int v = 0; v < V4; ++v) {
                float4 a = acc[q][v];
                a.x *= c_old;
                a.y *= c_old;
                a.z *= c_old;
                a.w *= c_old;
#pragma unroll
                for (int j = 0; j < A; ++j) {
                    a.x = __builtin_fmaf(p[j], vc4[j][v].x, a.x);
                    a.y = __builtin_fmaf(p[j], vc4[j][v].y, a.y);
                    a.z = __builtin_fmaf(p[j], vc4[j][v].z, a.z);
                    a.w = __builtin_fmaf(p[j], vc4[j][v].w, a.w);
                }
                acc[q][v] = a;
            }
            m[q] = mn;
        }
    };
    float4 kr[A][V4], vr[A][V4];
    load_rows(lr, kr, vr);
    for (int t0 = lr; t0 <= pos; t0 += A * ROWS) {
        float4 kc4[A][V4], vc4[A][V4];
#pragma unroll
        for (int j = 0; j < A; ++j)
#pragma unroll
            for (int v = 0; v < V4; ++v) {
                kc4[j][v] = kr[j][v];
                vc4[j][v] = vr[j][v];
            }
        if (t0 + A * ROWS <= pos) load_rows(t0 + A * ROWS, kr, vr);
        pass(t0, kc4, vc4);
    }
    // Merge the lane groups of each wave (butterfly over the group index),
    // then the waves through LDS.  An empty state (m = -inf) has l = 0 and
    // acc = 0 and gets weight 0.
#pragma unroll
    for (int o = LPR; o < 64; o <<= 1) {
#pragma unroll
        for (int q = 0; q < QR; ++q) {
            const float mp = __shfl_xor(m[q], o, 64);
            const float lp = __shfl_xor(l[q], o, 64);
            const float mn = fmaxf(m[q], mp);
            const float base = mn == -INFINITY ? 0.0f : mn;
            const float a = expf(m[q] - base), b = expf(mp - base);
            l[q] = l[q] * a + lp * b;
#pragma unroll
            for (int v = 0; v < V4; ++v) {
                float4 t = acc[q][v];
                t.x = t.x * a + __shfl_xor(t.x, o, 64) * b;
                t.y = t.y * a + __shfl_xor(t.y, o, 64) * b;
                t.z = t.z * a + __shfl_xor(t.z, o, 64) * b;
                t.w = t.w * a + __shfl_xor(t.w, o, 64) * b;
                acc[q][v] = t;
            }
            m[q] = mn;
        }
    }
    const int w = tid >> 6;
    if ((tid & 63) < LPR) {
#pragma unroll
        for (int q = 0; q < QR; ++q) {
            if (li == 0) {
                gm[q][w] = m[q];
                gl[q][w] = l[q];
            }
#pragma unroll
            for (int v = 0; v < V4; ++v) gacc[q][w][li + LPR * v] = acc[q][v];
        }
    }
    __syncthreads();
    for (int e0 = tid; e0 < QR * HD; e0 += NT) {
        const int q = e0 / HD;
        const int d = e0 % HD;
        float mx = -INFINITY;
#pragma unroll
        for (int g = 0; g < NW; ++g) mx = fmaxf(mx, gm[q][g]);
        const int c4 = d / 4;
        const int e = d % 4;
        float num = 0.0f;
        float den = 0.0f;
#pragma unroll
        for (int g = 0; g < NW; ++g) {
            const bool rows = gm[q][g] != -INFINITY;  // false: a wave without rows
            const float wgt = rows ? expf(gm[q][g] - mx) : 0.0f;
            const float4 a = gacc[q][g][c4];
            num += rows ? wgt * (e == 0 ? a.x : e == 1 ? a.y : e == 2 ? a.z : a.w) : 0.0f;
            den += rows ? wgt * gl[q][g] : 0.0f;
        }
        if (r0 + q < n) out[static_cast<size_t>(r0 + q) * n_heads * HD + h * HD + d] = num / den;
    }
}

// Causal attention of prefill rows on MFMA (head_dim HD = 64 or 128).
// Workgroup (head h, 16 W / KS query rows; the blocks with the most cache
// rows are launched first), wave w: query rows 16 (w % (W / KS)) .. + 15 and
// key blocks ks, ks + KS, ... of them with ks = w / (W / KS).  With KS = 2
// the two waves of a query tile each walk half of its key blocks (half the
// serial chain of the longest tiles) and merge their softmax states through
// LDS at the end: M = max(m0, m1), o = o0 e^(m0 - M) + o1 e^(m1 - M), the
// same for the sums.
// Key blocks of 32 cache rows are staged in LDS, KS at a time, as fp16 hi +
// lo (K as rows, V transposed), so every f32 product becomes hi*hi + hi*lo + lo*hi in
// v_mfma_f32_16x16x32_f16 (the dropped lo*lo term is 2^-22 of the product):
//  * scores, transposed: S^T[key][query] = K . Q^T (A = K rows of the block,
//    B = the wave's query rows, held in registers), then times 1/sqrt(HD);
//  * online softmax per query (lane column): the block's maximum and sum over
//    the lane's 8 keys and the three other lanes of its column (shuffles);
//  * O^T[d][query] += V^T . P^T: the lane's own 8 probabilities are the B
//    operand (its keys are the slots 8g .. 8g + 7 of the transposed V tile:
//    keys 4g .. 4g + 3 and 16 + 4g .. 16 + 4g + 3), so P never leaves
//    registers.
// Keys past a query's position get probability 0; cache rows past the
// block's last position re-read that row (finite, weight 0).  The result
// equals the reference's max - exp - sum - divide - weighted sum to rounding
// (src/forward.cpp:584-611 and src/ops.cpp:43-71 for one row).
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
constexpr int kMfmaAttnKeys = 32;  // cache rows per block

// v = hi + lo to 2^-22 of v: hi = fp16(v), lo = fp16(v - hi).
__device__ __forceinline__ _Float16 f16_hi(float v) { return static_cast<_Float16>(v); }
__device__ __forceinline__ _Float16 f16_lo(float v, _Float16 hi) {
    return static_cast<_Float16>(v - static_cast<float>(hi));
}

// Slot of key k (0..31) in a transposed V tile (the P^T operand's order).
__device__ __forceinline__ int attn_slot(int k) { return k < 16 ? 8 * (k >> 2) + (k & 3) : 8 * ((k - 16) >> 2) + 4 + (k & 3); }

template <int HD, int W, int PF, int KS>
__global__ __launch_bounds__(64 * W) void attention_rows_mfma_kernel(const float* __restrict__ Q,
                                                                  const float* __restrict__ kc,
                                                                  const float* __restrict__ vc, int n_heads, int n_kv,
                                                                  int max_seq, int layer, int start, int n,
                                                                  float* __restrict__ out) {
    constexpr int KB = kMfmaAttnKeys;
    constexpr int DC = HD / 32;  // d chunks of the score products
    constexpr int DT = HD / 16;  // d tiles of the output
    constexpr int KROW = HD + 8;  // halves per K row in LDS (16-byte aligned, banks spread)
    constexpr int VROW = KB + 8;  // halves per V^T row
    constexpr int NT = 64 * W;
    constexpr int QW = W / KS;          // query tiles of 16 rows per workgroup
    constexpr int KBS = KS * KB;        // keys staged per step
    constexpr int TPK = NT / KBS;       // threads per K row
    constexpr int KPT = HD / TPK;       // K elements per thread
    constexpr int VPT = KBS * HD / NT;  // V elements per thread (one d, VPT consecutive keys of one block)
    static_assert(W % KS == 0 && KPT % 8 == 0 && VPT % 4 == 0 && KB % VPT == 0, "staging map");
    static_assert(HD == 64 || HD == 128, "head_dim");
    constexpr int KSZ = KB * KROW;  // halves of one K buffer
    constexpr int VSZ = HD * VROW;  // halves of one V^T buffer
    // [K hi: KS][K lo: KS][V^T hi: KS][V^T lo: KS]; after the last step the
    // merge of the KS states reuses it.
    __shared__ __attribute__((aligned(16))) _Float16 smem[KS * (2 * KSZ + 2 * VSZ)];
    static_assert(KS == 1 || (KS - 1) * QW * 64 * (4 * (HD / 16) + 2) * 4 <= KS * (2 * KSZ + 2 * VSZ) * 2,
                  "merge area");
    _Float16* const khi = smem;
    _Float16* const klo = smem + KS * KSZ;
    _Float16* const vhi = smem + 2 * KS * KSZ;
    _Float16* const vlo = smem + 2 * KS * KSZ + KS * VSZ;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int i16 = lane & 15;
    const int g = lane >> 4;
    const int wave = tid >> 6;
    const int qw = wave % QW;
    const int ks = wave / QW;
    const int h = blockIdx.x;
    const int kvh = h / (n_heads / n_kv);
    const size_t layer_base = static_cast<size_t>(layer) * max_seq * n_kv * HD;
    const size_t t_stride = static_cast<size_t>(n_kv) * HD;
    const float* kbase = kc + layer_base + kvh * HD;
    const float* vbase = vc + layer_base + kvh * HD;
    const int qb0 = (gridDim.y - 1 - blockIdx.y) * 16 * QW;
    const int last_pos = start + min(qb0 + 16 * QW, n) - 1;  // the workgroup's last query position
    // This lane's query (rows past n repeat row n - 1; not stored).
    const int qrow = min(qb0 + 16 * qw + i16, n - 1);
    const int qpos = start + qrow;
    h8_t qh[DC], ql[DC];
    {
        const float* qp = Q + static_cast<size_t>(qrow) * n_heads * HD + h * HD + 8 * g;
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            const float4 a = *reinterpret_cast<const float4*>(qp + 32 * c);
            const float4 b = *reinterpret_cast<const float4*>(qp + 32 * c + 4);
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const _Float16 hh = f16_hi(v[j]);
                qh[c][j] = hh;
                ql[c][j] = f16_lo(v[j], hh);
            }
        }
    }
    // Staging maps (keys of a step: KS blocks of KB): K thread -> key
    // tid / TPK, elements (tid % TPK) * KPT ..; V thread -> d = tid % HD,
    // keys (tid / HD) * VPT ...
    const int k_key = tid / TPK;
    const int k_d0 = (tid % TPK) * KPT;
    const int v_d = tid % HD;
    const int v_k0 = (tid / HD) * VPT;
    _Float16* const kst_hi = khi + (k_key / KB) * KSZ + (k_key % KB) * KROW + k_d0;
    _Float16* const kst_lo = klo + (k_key / KB) * KSZ + (k_key % KB) * KROW + k_d0;
    _Float16* const vst_hi = vhi + (v_k0 / KB) * VSZ + v_d * VROW;
    _Float16* const vst_lo = vlo + (v_k0 / KB) * VSZ + v_d * VROW;
    // PF steps in flight: step sb is staged from register set sb % PF.
    float kreg[PF][KPT], vreg[PF][VPT];
    auto load_block = [&](int sb, int u) {
        const int t = min(sb * KBS + k_key, last_pos);
        const float* kp = kbase + static_cast<size_t>(t) * t_stride + k_d0;
#pragma unroll
        for (int i = 0; i < KPT; i += 4) {
            const float4 a = *reinterpret_cast<const float4*>(kp + i);
            kreg[u][i] = a.x;
            kreg[u][i + 1] = a.y;
            kreg[u][i + 2] = a.z;
            kreg[u][i + 3] = a.w;
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int tv = min(sb * KBS + v_k0 + i, last_pos);
            vreg[u][i] = vbase[static_cast<size_t>(tv) * t_stride + v_d];
        }
    };
    auto store_block = [&](int u) {
        h8_t hk, lk;
#pragma unroll
        for (int i = 0; i < KPT; i += 8) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const _Float16 hh = f16_hi(kreg[u][i + j]);
                hk[j] = hh;
                lk[j] = f16_lo(kreg[u][i + j], hh);
            }
            *reinterpret_cast<h8_t*>(kst_hi + i) = hk;
            *reinterpret_cast<h8_t*>(kst_lo + i) = lk;
        }
        typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int i = 0; i < VPT; i += 4) {  // four consecutive keys share four consecutive slots
            h4_t hv, lv;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const _Float16 hh = f16_hi(vreg[u][i + j]);
                hv[j] = hh;
                lv[j] = f16_lo(vreg[u][i + j], hh);
            }
            const int slot = attn_slot(v_k0 % KB + i);
            *reinterpret_cast<h4_t*>(vst_hi + slot) = hv;
            *reinterpret_cast<h4_t*>(vst_lo + slot) = lv;
        }
    };
    const float scale = 1.0f / sqrtf(static_cast<float>(HD));
    const f4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
    f4_t o[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] = zero;
    float m = -INFINITY, l = 0.0f;
    const int nkb = last_pos / KB + 1;   // key blocks
    const int nsb = (nkb + KS - 1) / KS;  // steps (a step's blocks past nkb - 1 are all masked)
    const _Float16* const kh_w = khi + ks * KSZ;
    const _Float16* const kl_w = klo + ks * KSZ;
    const _Float16* const vh_w = vhi + ks * VSZ;
    const _Float16* const vl_w = vlo + ks * VSZ;
#pragma unroll
    for (int u = 0; u < PF; ++u)
        if (u < nsb) load_block(u, u);
    auto step = [&](int sb, int u) {
        __syncthreads();  // the previous step's readers are done
        store_block(u);
        __syncthreads();
        if (sb + PF < nsb) load_block(sb + PF, u);
        const int kb = sb * KS + ks;  // this wave's key block
        // S^T for the two 16-key tiles: three product terms in separate
        // accumulators (independent MFMA chains), summed after.
        f4_t s[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            f4_t a0 = zero, a1 = zero, a2 = zero;
            const _Float16* kh = kh_w + (16 * kt + i16) * KROW + 8 * g;
            const _Float16* kl = kl_w + (16 * kt + i16) * KROW + 8 * g;
#pragma unroll
            for (int c = 0; c < DC; ++c) {
                const h8_t ah = *reinterpret_cast<const h8_t*>(kh + 32 * c);
                const h8_t al = *reinterpret_cast<const h8_t*>(kl + 32 * c);
                a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, qh[c], a0, 0, 0, 0);
                a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, ql[c], a1, 0, 0, 0);
                a2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, qh[c], a2, 0, 0, 0);
            }
            s[kt] = a0 + (a1 + a2);
        }
        // Scores of this lane: keys kb*32 + 16 kt + 4 g + q for query qpos.
        float sc[8];
        float bm = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int key = kb * KB + 16 * kt + 4 * g + q;
                const float v = key <= qpos ? s[kt][q] * scale : -INFINITY;
                sc[4 * kt + q] = v;
                bm = fmaxf(bm, v);
            }
        bm = fmaxf(bm, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, bm), 0x401F)));
        bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
        const float mn = fmaxf(m, bm);
        const float base = mn == -INFINITY ? 0.0f : mn;
        const float c_old = expf(m - base);
        float ps = 0.0f;
        h8_t ph, pl;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float p = expf(sc[j] - base);
            ps += p;
            const _Float16 hh = f16_hi(p);
            ph[j] = hh;
            pl[j] = f16_lo(p, hh);
        }
        ps += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, ps), 0x401F));
        ps += __shfl_xor(ps, 32, 64);
        l = l * c_old + ps;
        m = mn;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            f4_t a0 = o[t] * c_old, a1 = zero, a2 = zero;
            const h8_t vh = *reinterpret_cast<const h8_t*>(vh_w + (16 * t + i16) * VROW + 8 * g);
            const h8_t vl = *reinterpret_cast<const h8_t*>(vl_w + (16 * t + i16) * VROW + 8 * g);
            a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, ph, a0, 0, 0, 0);
            a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, pl, a1, 0, 0, 0);
            a2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, ph, a2, 0, 0, 0);
            o[t] = a0 + (a1 + a2);
        }
    };
    for (int sb0 = 0; sb0 < nsb; sb0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u)
            if (sb0 + u < nsb) step(sb0 + u, u);
    }
    if (KS > 1) {
        // Waves ks >= 1 leave (m, l, O^T) in LDS; wave 0 of the tile folds
        // them in, in ks order.  Wave 0 saw key 0, so its maximum is finite.
        float* const mrg = reinterpret_cast<float*>(smem);
        constexpr int PER = 4 * DT + 2;  // floats per lane
        __syncthreads();  // every wave is done with the staged keys
        if (ks > 0) {
            float* dst = mrg + (((ks - 1) * QW + qw) * PER) * 64;
#pragma unroll
            for (int t = 0; t < DT; ++t)
#pragma unroll
                for (int q = 0; q < 4; ++q) dst[(4 * t + q) * 64 + lane] = o[t][q];
            dst[(4 * DT) * 64 + lane] = m;
            dst[(4 * DT + 1) * 64 + lane] = l;
        }
        __syncthreads();
        if (ks > 0) return;
#pragma unroll
        for (int j = 1; j < KS; ++j) {
            const float* src = mrg + (((j - 1) * QW + qw) * PER) * 64;
            const float m1 = src[(4 * DT) * 64 + lane];
            const float l1 = src[(4 * DT + 1) * 64 + lane];
            const float mx = fmaxf(m, m1);
            const float c0 = expf(m - mx);
            const float c1 = expf(m1 - mx);  // 0 when that wave saw no key of this query
#pragma unroll
            for (int t = 0; t < DT; ++t)
#pragma unroll
                for (int q = 0; q < 4; ++q) o[t][q] = o[t][q] * c0 + src[(4 * t + q) * 64 + lane] * c1;
            l = l * c0 + l1 * c1;
            m = mx;
        }
    }
    // O^T[d = 16 t + 4 g + q][this lane's query] / l.
    if (qb0 + 16 * qw + i16 < n) {
        const float inv = 1.0f / l;
        float* op = out + static_cast<size_t>(qrow) * n_heads * HD + h * HD + 4 * g;
#pragma unroll
        for (int t = 0; t < DT; ++t)
            *reinterpret_cast<float4*>(op + 16 * t) =
                make_float4(o[t][0] * inv, o[t][1] * inv, o[t][2] * inv, o[t][3] * inv);
    }
}

// Y[r][M] = W[M][K] . X[r] for F32 weights: one wave per (row of W, row of X).
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ W, const float* __restrict__ X,
                                                       float* __restrict__ Y, int M, int K) {
    const int row = blockIdx.x * 4 + static_cast<int>(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const float* w = W + static_cast<size_t>(row) * K;
    const float* x = X + static_cast<size_t>(blockIdx.y) * K;
    float acc = 0.0f;
    for (int k = lane; k < K; k += 64) acc += w[k] * x[k];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (lane == 0) Y[static_cast<size_t>(blockIdx.y) * M + row] = acc;
}

// out = silu(gate) * up (swiglu, src/ops.cpp:95-107).
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                     float* __restrict__ out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float v = g[i];
        const float sig = 1.0f / (1.0f + expf(-v));
        out[i] = v * sig * u[i];
    }
}

// y[M] = W[M][K] . x for F32 weights: one wave per row.
__global__ __launch_bounds__(256) void gemv_f32_kernel(const float* __restrict__ W, const float* __restrict__ x,
                                                       float* __restrict__ y, int M, int K) {
    const int row = blockIdx.x * 4 + static_cast<int>(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const float* w = W + static_cast<size_t>(row) * K;
    float acc = 0.0f;
    for (int k = lane; k < K; k += 64) acc += w[k] * x[k];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (lane == 0) y[row] = acc;
}

// Greedy pick over F32 logits in one workgroup: st->next = first index of the
// maximum, or -1 with the error bit when a logit is not finite.
__global__ __launch_bounds__(1024) void pick_f32_kernel(const float* __restrict__ logits, int n, DecodeState* st) {
    __shared__ unsigned long long part[16];
    unsigned long long best = 0;
    for (int i = threadIdx.x; i < n; i += 1024) {
        const unsigned long long k = pick_key(logits[i], i);
        best = k > best ? k : best;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long other = __shfl_xor(best, o, 64);
        best = other > best ? other : best;
    }
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < 16; ++i) best = part[i] > best ? part[i] : best;
        best = part[0] > best ? part[0] : best;
        st->next = pick_token(best);
    }
}

// End of a step: the next input token (the prompt's, or this step's pick,
// which is also stored as a generated token) and the next position.
__global__ void advance_kernel(DecodeState* st, int32_t* io) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    const int p = st->pos;
    const int np = st->n_prompt;
    if (p + 1 < np) {
        st->token = io[p + 1];
    } else {
        const int picked = st->next;
        const int g = p + 1 - np;
        if (g >= 0 && g < st->n_out) io[np + g] = picked;
        if (picked < 0) st->error |= kDecodeErrLogits;
        st->token = picked < 0 ? 0 : picked;
    }
    st->pos = p + 1;
}

int qtype_of_ggml(uint32_t t) {
    switch (t) {
        case kGgmlQ8_0: return MLQ_Q8_0;
        case kGgmlQ4_0: return MLQ_Q4_0;
        case kGgmlQ4_1: return MLQ_Q4_1;
        default: return -1;
    }
}

float fp16_value(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h >> 15) << 31;
    const int e = (h >> 10) & 31;
    const uint32_t m = h & 1023;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {  // subnormal: m * 2^-24, exact in f32
            const float v = static_cast<float>(m) * 5.9604644775390625e-08f;
            std::memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | (static_cast<uint32_t>(e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// Block bytes to f32 rows of `row` values, as dequantize_from_q8_0 / _q4_0 /
// _q4_1 (src/quant.cpp:172-360): d * q, d * (n - 8), d * n + m (one multiply,
// then one add).
void dequantize_rows(int qtype, const uint8_t* blk, size_t rows, size_t row, float* out) {
    const size_t nb = (row + 31) / 32;
    const size_t bb = static_cast<size_t>(block_bytes(qtype));
    for (size_t r = 0; r < rows; ++r) {
        for (size_t b = 0; b < nb; ++b) {
            const uint8_t* p = blk + (r * nb + b) * bb;
            uint16_t dh;
            std::memcpy(&dh, p, 2);
            const float d = fp16_value(dh);
            float m = 0.0f;
            if (qtype == MLQ_Q4_1) {
                uint16_t mh;
                std::memcpy(&mh, p + 2, 2);
                m = fp16_value(mh);
            }
            for (size_t j = 0; j < 32; ++j) {
                const size_t col = b * 32 + j;
                if (col >= row) break;
                float v;
                if (qtype == MLQ_Q8_0) {
                    v = d * static_cast<float>(static_cast<int8_t>(p[2 + j]));
                } else {
                    const int off = qtype == MLQ_Q4_0 ? 2 : 4;
                    const uint8_t byte = p[off + (j & 15)];
                    const int n = j < 16 ? (byte & 15) : (byte >> 4);
                    if (qtype == MLQ_Q4_0) {
                        v = d * static_cast<float>(n - 8);
                    } else {
                        v = d * static_cast<float>(n);
                        v = v + m;
                    }
                }
                out[r * row + col] = v;
            }
        }
    }
}

std::string shape_text(const std::vector<int>& s) {
    std::string t = "[";
    for (size_t i = 0; i < s.size(); ++i) t += (i ? ", " : "") + std::to_string(s[i]);
    return t + "]";
}

}  // namespace

// ------------------------------------------------------------------ loading

void Decoder::check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string("HIP error in ") + what + ": " + hipGetErrorString(e));
}

std::unique_ptr<Decoder> Decoder::from_gguf(const std::string& path, int device, int max_seq_len) {
    GgufIndex g;
    if (!g.open(path)) throw std::runtime_error("GGUF parse error: " + g.error);

    // Config (build_config, src/gguf_loader.cpp:241-310).
    DecoderConfig c;
    {
        auto get_int = [&](const std::string& key, int fallback) {
            int64_t v = 0;
            return g.get_int(key, v) ? static_cast<int>(v) : fallback;
        };
        auto get_float = [&](const std::string& key, float fallback) {
            double v = 0.0;
            return g.get_float(key, v) ? static_cast<float>(v) : fallback;
        };
        std::string arch;
        if (g.get_string("general.architecture", arch) && arch == "qwen2") c.rope_neox = 1;
        c.n_layers = get_int("qwen2.block_count", get_int("llama.block_count", 0));
        c.dim = get_int("qwen2.embedding_length", get_int("llama.embedding_length", 0));
        c.hidden_dim = get_int("qwen2.feed_forward_length", get_int("llama.feed_forward_length", 0));
        c.n_heads = get_int("qwen2.attention.head_count", get_int("llama.attention.head_count", 0));
        c.n_kv_heads = get_int("qwen2.attention.head_count_kv", get_int("llama.attention.head_count_kv", 0));
        c.max_seq_len = get_int("qwen2.context_length", get_int("llama.context_length", 0));
        c.rope_theta = get_float("qwen2.rope.freq_base", get_float("llama.rope.freq_base", 10000.0f));
        c.rms_norm_eps = get_float("qwen2.attention.layer_norm_rms_epsilon",
                                   get_float("llama.attention.layer_norm_rms_epsilon", 1e-5f));
        // Without the token list the vocabulary keeps ModelConfig's default
        // (include/mini_llama/model.h:18), as in the reference.
        c.vocab_size = 128;
        uint64_t vocab = 0;
        if (g.get_string_array_size("tokenizer.ggml.tokens", vocab)) c.vocab_size = static_cast<int>(vocab);
        if (c.n_layers <= 0 || c.dim <= 0 || c.hidden_dim <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 ||
            c.max_seq_len <= 0 || c.vocab_size <= 0) {
            throw std::runtime_error("Failed to build config: Invalid model config from GGUF: dim=" +
                                     std::to_string(c.dim) + " layers=" + std::to_string(c.n_layers) +
                                     " heads=" + std::to_string(c.n_heads) + " vocab=" + std::to_string(c.vocab_size));
        }
        if (c.dim % c.n_heads != 0) throw std::runtime_error("Failed to build config: dim not divisible by n_heads");
        if (c.n_heads % c.n_kv_heads != 0) {
            throw std::runtime_error("Failed to build config: n_heads not divisible by n_kv_heads");
        }
        c.head_dim = c.dim / c.n_heads;
    }
    if (c.head_dim % 2 != 0 || c.head_dim > kMaxHeadDim) {
        throw std::runtime_error("HIP decoder: head_dim " + std::to_string(c.head_dim) +
                                 " is not supported (even, at most " + std::to_string(kMaxHeadDim) + ")");
    }
    if (max_seq_len > 0 && max_seq_len < c.max_seq_len) c.max_seq_len = max_seq_len;

    std::unique_ptr<Decoder> d(new Decoder);
    d->cfg_ = c;
    d->device_ = device;
    d->check(hipSetDevice(device), "hipSetDevice");
    d->check(hipStreamCreateWithFlags(&d->stream_, hipStreamNonBlocking), "hipStreamCreateWithFlags");

    auto alloc = [&](size_t bytes) {
        void* p = nullptr;
        d->check(hipMalloc(&p, bytes == 0 ? 4 : bytes), "hipMalloc");
        d->allocs_.push_back(p);
        return p;
    };
    auto upload = [&](const void* src, size_t bytes) {
        void* p = alloc(bytes);
        d->check(hipMemcpy(p, src, bytes, hipMemcpyHostToDevice), "hipMemcpy");
        return p;
    };

    // Tensors by the loader's names (map_tensor_name, src/gguf_loader.cpp:15-84),
    // reported under the model's names as load_weight does.
    const std::string fail = "Failed to load GGUF weights: ";
    auto tensor = [&](const std::string& gguf_name, const std::string& model_name, bool required) -> const GgufTensor* {
        const int64_t i = g.find(gguf_name);
        if (i < 0) {
            if (required) throw std::runtime_error(fail + "Missing tensor: " + model_name);
            return nullptr;
        }
        const GgufTensor& t = g.tensors[static_cast<size_t>(i)];
        if (t.type != kGgmlF32 && qtype_of_ggml(t.type) < 0) {
            if (t.nbytes == 0) throw std::runtime_error(fail + "Failed to read tensor: " + model_name);
            throw std::runtime_error(fail + "Unsupported GGUF tensor type: " + std::to_string(t.type));
        }
        return &t;
    };
    auto shape_of = [](const GgufTensor& t) {
        std::vector<int> s;
        if (t.dims.size() == 2) return std::vector<int>{static_cast<int>(t.dims[1]), static_cast<int>(t.dims[0])};
        for (uint64_t v : t.dims) s.push_back(static_cast<int>(v));
        return s;
    };
    // F32 roles (load_f32): F32 as stored, quantized ones dequantized.
    auto load_f32 = [&](const GgufTensor& t, const std::vector<int>& want, const std::string& what) -> float* {
        const std::vector<int> s = shape_of(t);
        if (s != want) {
            throw std::runtime_error(fail + "GGUF " + what + ": shape mismatch. expected " + shape_text(want) +
                                     ", got " + shape_text(s));
        }
        size_t numel = 1;
        for (int v : s) numel *= static_cast<size_t>(v);
        const uint8_t* src = g.tensor_data(t);
        if (t.type == kGgmlF32) return static_cast<float*>(upload(src, numel * 4));
        const size_t row = s.size() >= 2 ? static_cast<size_t>(s.back()) : numel;
        std::vector<float> tmp(numel);
        dequantize_rows(qtype_of_ggml(t.type), src, numel / row, row, tmp.data());
        return static_cast<float*>(upload(tmp.data(), numel * 4));
    };
    auto load_linear = [&](const GgufTensor& t, int rows, int cols, const std::string& what) -> Linear {
        const std::vector<int> s = shape_of(t);
        const std::vector<int> want{rows, cols};
        if (s != want) {
            throw std::runtime_error(fail + "GGUF " + what + ": shape mismatch, expected " + shape_text(want) +
                                     ", got " + shape_text(s));
        }
        Linear l;
        l.qtype = t.type == kGgmlF32 ? 0 : qtype_of_ggml(t.type);
        l.M = rows;
        l.K = cols;
        if (l.qtype != 0) {
            const size_t need = static_cast<size_t>(rows) * ((cols + 31) / 32) * block_bytes(l.qtype);
            if (need != t.nbytes) {
                throw std::runtime_error(fail + "GGUF " + what + ": block count mismatch for " + shape_text(want));
            }
        }
        l.data = upload(g.tensor_data(t), t.nbytes);
        return l;
    };

    const int q_dim = c.n_heads * c.head_dim;
    const int kv_dim = c.n_kv_heads * c.head_dim;
    const GgufTensor* emb = tensor("token_embd.weight", "token_embedding", true);
    d->layers_.resize(c.n_layers);
    struct Pending {
        const GgufTensor* t[12];
    };
    std::vector<Pending> lt(c.n_layers);
    for (int l = 0; l < c.n_layers; ++l) {
        const std::string gp = "blk." + std::to_string(l) + ".";
        const std::string mp = "layers." + std::to_string(l) + ".";
        Pending& p = lt[l];
        p.t[0] = tensor(gp + "attn_norm.weight", mp + "attention_norm", true);
        p.t[1] = tensor(gp + "attn_q.weight", mp + "wq", true);
        p.t[2] = tensor(gp + "attn_k.weight", mp + "wk", true);
        p.t[3] = tensor(gp + "attn_v.weight", mp + "wv", true);
        p.t[4] = tensor(gp + "attn_q.bias", mp + "bq", false);
        p.t[5] = tensor(gp + "attn_k.bias", mp + "bk", false);
        p.t[6] = tensor(gp + "attn_v.bias", mp + "bv", false);
        p.t[7] = tensor(gp + "attn_output.weight", mp + "wo", true);
        p.t[8] = tensor(gp + "ffn_norm.weight", mp + "ffn_norm", true);
        p.t[9] = tensor(gp + "ffn_gate.weight", mp + "w_gate", true);
        p.t[10] = tensor(gp + "ffn_up.weight", mp + "w_up", true);
        p.t[11] = tensor(gp + "ffn_down.weight", mp + "w_down", true);
    }
    const GgufTensor* fnorm = tensor("output_norm.weight", "final_norm", true);
    const GgufTensor* out = tensor("output.weight", "lm_head", false);

    // Shapes as validate_loaded_shapes (src/gguf_loader.cpp:204-238).
    d->embedding_ = load_f32(*emb, {c.vocab_size, c.dim}, "token_embedding");
    d->final_norm_ = load_f32(*fnorm, {c.dim}, "final_norm");
    if (out != nullptr) {
        d->lm_head_ = load_linear(*out, c.vocab_size, c.dim, "lm_head");
    } else {  // tied: the F32 embedding serves as the output projection
        d->lm_head_ = Linear{0, c.vocab_size, c.dim, d->embedding_};
    }
    for (int l = 0; l < c.n_layers; ++l) {
        const std::string pre = "layers." + std::to_string(l) + ".";
        Layer& L = d->layers_[l];
        const Pending& p = lt[l];
        L.attn_norm = load_f32(*p.t[0], {c.dim}, pre + "attention_norm");
        L.wq = load_linear(*p.t[1], q_dim, c.dim, pre + "wq");
        L.wk = load_linear(*p.t[2], kv_dim, c.dim, pre + "wk");
        L.wv = load_linear(*p.t[3], kv_dim, c.dim, pre + "wv");
        if (p.t[4]) L.bq = load_f32(*p.t[4], {q_dim}, pre + "bq");
        if (p.t[5]) L.bk = load_f32(*p.t[5], {kv_dim}, pre + "bk");
        if (p.t[6]) L.bv = load_f32(*p.t[6], {kv_dim}, pre + "bv");
        L.wo = load_linear(*p.t[7], c.dim, q_dim, pre + "wo");
        L.ffn_norm = load_f32(*p.t[8], {c.dim}, pre + "ffn_norm");
        L.w_gate = load_linear(*p.t[9], c.hidden_dim, c.dim, pre + "w_gate");
        L.w_up = load_linear(*p.t[10], c.hidden_dim, c.dim, pre + "w_up");
        L.w_down = load_linear(*p.t[11], c.dim, c.hidden_dim, pre + "w_down");
    }

    // Activations, scratch, cache and state.
    auto f32buf = [&](size_t n) { return static_cast<float*>(alloc(n * 4)); };
    d->x_ = f32buf(c.dim);
    d->h_ = f32buf(c.dim);
    d->q_ = f32buf(q_dim);
    d->k_ = f32buf(kv_dim);
    d->v_ = f32buf(kv_dim);
    d->att_ = f32buf(q_dim);
    d->proj_ = f32buf(c.dim);
    d->gate_ = f32buf(c.hidden_dim);
    d->up_ = f32buf(c.hidden_dim);
    d->act_ = f32buf(c.hidden_dim);
    d->ff_ = f32buf(c.dim);
    d->logits_ = f32buf(c.vocab_size);
    d->scores_ = f32buf(static_cast<size_t>(c.n_heads) * c.max_seq_len);
    const size_t cache = static_cast<size_t>(c.n_layers) * c.max_seq_len * kv_dim;
    d->kcache_ = f32buf(cache);
    d->vcache_ = f32buf(cache);
    d->check(hipMemset(d->kcache_, 0, cache * 4), "hipMemset");
    d->check(hipMemset(d->vcache_, 0, cache * 4), "hipMemset");
    d->state_ = static_cast<DecodeState*>(alloc(sizeof(DecodeState)));
    d->check(hipMemset(d->state_, 0, sizeof(DecodeState)), "hipMemset");
    d->pick_ = alloc(sizeof(PickState));
    d->check(hipMemset(d->pick_, 0, sizeof(PickState)), "hipMemset");
    // Split decode attention: partial states and arrival counts (zero; the
    // last workgroup of each head resets its count).
    d->attn_splits_ = std::max(1, std::min(kAttnMaxSplits, (c.max_seq_len + kAttnSplitRows - 1) / kAttnSplitRows));
    d->attn_part_ = f32buf(static_cast<size_t>(c.n_heads) * d->attn_splits_ * (c.head_dim + 2));
    d->attn_cnt_ = static_cast<unsigned*>(alloc(static_cast<size_t>(c.n_heads) * sizeof(unsigned)));
    d->check(hipMemset(d->attn_cnt_, 0, static_cast<size_t>(c.n_heads) * sizeof(unsigned)), "hipMemset");
    d->check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    return d;
}

Decoder::~Decoder() {
    if (device_ >= 0) (void)hipSetDevice(device_);
    if (stream_) (void)hipStreamSynchronize(stream_);
    if (graph_) (void)hipGraphExecDestroy(graph_);
    for (hipEvent_t ev : inflight_)
        if (ev) (void)hipEventDestroy(ev);
    for (void* p : allocs_) (void)hipFree(p);
    if (stream_) (void)hipStreamDestroy(stream_);
}

// ---------------------------------------------------------------- one step

void Decoder::linear_group(hipStream_t s, const Linear* const* ws, float* const* ys, int n, const float* x) {
    // Consecutive quantized weights of one format and width share a launch.
    int i = 0;
    while (i < n) {
        const Linear& w = *ws[i];
        if (w.qtype == 0) {
            hipLaunchKernelGGL(gemv_f32_kernel, dim3((w.M + 3) / 4), dim3(256), 0, s,
                               static_cast<const float*>(w.data), x, ys[i], w.M, w.K);
            check(hipGetLastError(), "gemv_f32_kernel");
            ++i;
            continue;
        }
        GemvGroup g{};
        int rows = 0;
        int j = i;
        while (j < n && j - i < kGroupMaxCalls && ws[j]->qtype == w.qtype && ws[j]->K == w.K) {
            g.W[j - i] = ws[j]->data;
            g.y[j - i] = ys[j];
            g.row_begin[j - i] = rows;
            rows += ws[j]->M;
            ++j;
        }
        g.ncalls = j - i;
        const LinearShape shape{w.qtype, rows, w.K, (w.K + 31) / 32, 1};
        check(launch_gemv_group(shape, g, x, s), "launch_gemv_group");
        i = j;
    }
}

void Decoder::launch_norm(hipStream_t s, const float* delta, const float* w) {
    const int dim = cfg_.dim;
    if (dim % 4 == 0 && dim <= 4 * kNormThreads * 2) {
        if (dim <= 4 * kNormThreads) {
            hipLaunchKernelGGL(add_rmsnorm_vec_kernel<1>, dim3(1), dim3(kNormThreads), 0, s, x_, delta, w, dim,
                               cfg_.rms_norm_eps, h_);
        } else {
            hipLaunchKernelGGL(add_rmsnorm_vec_kernel<2>, dim3(1), dim3(kNormThreads), 0, s, x_, delta, w, dim,
                               cfg_.rms_norm_eps, h_);
        }
    } else {
        hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(1), dim3(kNormThreads), 0, s, x_, delta, w, dim, cfg_.rms_norm_eps,
                           h_);
    }
    check(hipGetLastError(), "add_rmsnorm_kernel");
}

bool Decoder::launch_attention_rope(hipStream_t s, int l) {
    const DecoderConfig& c = cfg_;
    const Layer& L = layers_[l];
#define MLQ_ATTN(LPR)                                                                                            \
    hipLaunchKernelGGL((attention_rope_kernel<LPR>), dim3(c.n_heads, attn_splits_), dim3(kFlashThreads), 0, s, q_, \
                       k_, v_, L.bq, L.bk, L.bv, c.n_heads, c.n_kv_heads, c.rope_theta, c.rope_neox, c.max_seq_len, l, \
                       state_, kcache_, vcache_, att_, attn_part_, attn_cnt_, attn_splits_)
    switch (c.head_dim) {
        case 16: MLQ_ATTN(4); break;
        case 32: MLQ_ATTN(8); break;
        case 64: MLQ_ATTN(16); break;
        case 128: MLQ_ATTN(32); break;
        case 256: MLQ_ATTN(64); break;
        default: return false;
    }
#undef MLQ_ATTN
    check(hipGetLastError(), "attention_rope_kernel");
    return true;
}

// Quantized weights of one (grouped) launch: consecutive ones of one format
// and width share it.  `norm`: stage rmsnorm(x) * norm_w instead of x;
// `acc`: add the rows into y.  F32 weights are not allowed here.
void Decoder::linear_fused(hipStream_t s, const Linear* const* ws, float* const* ys, int n, const float* x,
                           const float* norm_w, bool acc) {
    int i = 0;
    while (i < n) {
        const Linear& w = *ws[i];
        GemvGroup g{};
        int rows = 0;
        int j = i;
        while (j < n && j - i < kGroupMaxCalls && ws[j]->qtype == w.qtype && ws[j]->K == w.K) {
            g.W[j - i] = ws[j]->data;
            g.y[j - i] = ys[j];
            g.row_begin[j - i] = rows;
            rows += ws[j]->M;
            ++j;
        }
        g.ncalls = j - i;
        g.norm_w = norm_w;
        g.norm_eps = cfg_.rms_norm_eps;
        const LinearShape shape{w.qtype, rows, w.K, (w.K + 31) / 32, 1};
        check(launch_gemv_decode(shape, g, x, norm_w != nullptr, acc, s), "launch_gemv_decode");
        i = j;
    }
}

// One decode step.  Where a layer's linears are quantized, the RMSNorm is
// done by the consuming GEMVs (norm mode, reading the residual stream x_),
// the residual add by the producing ones (o and down accumulate into x_) and
// SwiGLU by the gate/up launch (GLU mode, when gate and up share a format and
// rows of at most 64 pairs): per layer q/k/v -> attention -> o -> gate/up +
// SwiGLU -> down, five launches.  Otherwise
// (F32 weights) the separate add + RMSNorm kernel runs, with `pending` the
// residual delta it still has to add.
void Decoder::enqueue_step(hipStream_t s, bool pick, bool advance) {
    const DecoderConfig& c = cfg_;
    auto quant = [](const Linear& w) { return w.qtype != 0; };
    hipLaunchKernelGGL(embed_kernel, dim3((c.dim + 255) / 256), dim3(256), 0, s, embedding_, c.vocab_size, c.dim,
                       state_, x_);
    check(hipGetLastError(), "embed_kernel");
    const float* pending = nullptr;
    for (int l = 0; l < c.n_layers; ++l) {
        const Layer& L = layers_[l];
        const Linear* qkv[3] = {&L.wq, &L.wk, &L.wv};
        float* qkv_y[3] = {q_, k_, v_};
        if (pending == nullptr && quant(L.wq) && quant(L.wk) && quant(L.wv)) {
            linear_fused(s, qkv, qkv_y, 3, x_, L.attn_norm, false);
        } else {
            launch_norm(s, pending, L.attn_norm);
            pending = nullptr;
            linear_group(s, qkv, qkv_y, 3, h_);
        }
        if (!launch_attention_rope(s, l)) {
            const int q_dim = c.n_heads * c.head_dim;
            const int kv_dim = c.n_kv_heads * c.head_dim;
            const int rope_threads = q_dim / 2 + kv_dim / 2 + kv_dim;
            hipLaunchKernelGGL(rope_kv_kernel, dim3((rope_threads + 255) / 256), dim3(256), 0, s, q_, k_, v_, L.bq,
                               L.bk, L.bv, c.n_heads, c.n_kv_heads, c.head_dim, c.rope_theta, c.rope_neox,
                               c.max_seq_len, l, state_, kcache_, vcache_);
            check(hipGetLastError(), "rope_kv_kernel");
            hipLaunchKernelGGL(attention_kernel, dim3(c.n_heads), dim3(kAttnThreads), 0, s, q_, kcache_, vcache_,
                               scores_, att_, c.n_heads, c.n_kv_heads, c.head_dim, c.max_seq_len, l, state_);
            check(hipGetLastError(), "attention_kernel");
        }
        const Linear* wo[1] = {&L.wo};
        if (quant(L.wo)) {
            float* wo_y[1] = {x_};
            linear_fused(s, wo, wo_y, 1, att_, nullptr, true);
        } else {
            float* wo_y[1] = {proj_};
            linear_group(s, wo, wo_y, 1, att_);
            pending = proj_;
        }
        const Linear* gu[2] = {&L.w_gate, &L.w_up};
        float* gu_y[2] = {gate_, up_};
        const LinearShape gu_shape{L.w_gate.qtype, L.w_gate.M, L.w_gate.K, (L.w_gate.K + 31) / 32, 1};
        if (pending == nullptr && quant(L.w_gate) && L.w_up.qtype == L.w_gate.qtype && L.w_up.M == L.w_gate.M &&
            L.w_up.K == L.w_gate.K && gemv_glu_supported(gu_shape)) {
            // gate, up and SwiGLU in one launch (FFN RMSNorm staged)
            GemvGroup g{};
            g.W[0] = L.w_gate.data;
            g.W[1] = L.w_up.data;
            g.y[0] = act_;
            g.row_begin[1] = L.w_gate.M;
            g.ncalls = 2;
            g.norm_w = L.ffn_norm;
            g.norm_eps = c.rms_norm_eps;
            check(launch_gemv_glu(gu_shape, g, x_, s), "launch_gemv_glu");
        } else {
            if (pending == nullptr && quant(L.w_gate) && quant(L.w_up)) {
                linear_fused(s, gu, gu_y, 2, x_, L.ffn_norm, false);
            } else {
                launch_norm(s, pending, L.ffn_norm);
                pending = nullptr;
                linear_group(s, gu, gu_y, 2, h_);
            }
            hipLaunchKernelGGL(swiglu_kernel, dim3((c.hidden_dim + 255) / 256), dim3(256), 0, s, gate_, up_, act_,
                               c.hidden_dim);
            check(hipGetLastError(), "swiglu_kernel");
        }
        const Linear* wd[1] = {&L.w_down};
        if (quant(L.w_down)) {
            float* wd_y[1] = {x_};
            linear_fused(s, wd, wd_y, 1, act_, nullptr, true);
        } else {
            float* wd_y[1] = {ff_};
            linear_group(s, wd, wd_y, 1, act_);
            pending = ff_;
        }
    }
    if (!pick && advance) {  // a prompt step before the last: no logits needed
        hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(64), 0, s, state_, io_);
        check(hipGetLastError(), "advance_kernel");
        return;
    }
    const bool fused_head = pending == nullptr && quant(lm_head_);
    const LinearShape head{lm_head_.qtype, lm_head_.M, lm_head_.K, (lm_head_.K + 31) / 32, 1};
    if (pick && fused_head) {
        check(launch_gemv_pick_norm(head, lm_head_.data, x_, final_norm_, c.rms_norm_eps, nullptr,
                                    static_cast<PickState*>(pick_), &state_->next, s),
              "launch_gemv_pick_norm");
    } else if (fused_head) {
        const Linear* lm[1] = {&lm_head_};
        float* lm_y[1] = {logits_};
        linear_fused(s, lm, lm_y, 1, x_, final_norm_, false);
    } else {
        launch_norm(s, pending, final_norm_);
        if (pick && quant(lm_head_)) {
            check(launch_gemv_pick(head, lm_head_.data, h_, nullptr, static_cast<PickState*>(pick_), &state_->next, s),
                  "launch_gemv_pick");
        } else {
            const Linear* lm[1] = {&lm_head_};
            float* lm_y[1] = {logits_};
            linear_group(s, lm, lm_y, 1, h_);
            if (pick) {
                hipLaunchKernelGGL(pick_f32_kernel, dim3(1), dim3(1024), 0, s, logits_, c.vocab_size, state_);
                check(hipGetLastError(), "pick_f32_kernel");
            }
        }
    }
    if (advance) {
        hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(64), 0, s, state_, io_);
        check(hipGetLastError(), "advance_kernel");
    }
}

void Decoder::ensure_prefill() {
    if (X_ != nullptr) return;
    const DecoderConfig& c = cfg_;
    const size_t R = kPrefillRows;
    auto buf = [&](size_t n) {
        void* p = nullptr;
        check(hipMalloc(&p, n * 4), "hipMalloc");
        allocs_.push_back(p);
        return static_cast<float*>(p);
    };
    const int q_dim = c.n_heads * c.head_dim;
    const int kv_dim = c.n_kv_heads * c.head_dim;
    X_ = buf(R * c.dim);
    H_ = buf(R * c.dim);
    Q_ = buf(R * q_dim);
    K_ = buf(R * kv_dim);
    V_ = buf(R * kv_dim);
    ATT_ = buf(R * q_dim);
    PROJ_ = buf(R * c.dim);
    GATE_ = buf(R * c.hidden_dim);
    UP_ = buf(R * c.hidden_dim);
    ACT_ = buf(R * c.hidden_dim);
    FF_ = buf(R * c.dim);
}

// One linear over `rows` rows of X (row-major [rows][K] in, [rows][M] out):
// the MFMA GEMM where it applies, else the GEMV kernels over a batch of rows.
void Decoder::linear_rows(hipStream_t s, const Linear& w, const float* X, float* Y, int rows) {
    if (w.qtype == 0) {
        hipLaunchKernelGGL(gemm_f32_kernel, dim3((w.M + 3) / 4, rows), dim3(256), 0, s,
                           static_cast<const float*>(w.data), X, Y, w.M, w.K);
        check(hipGetLastError(), "gemm_f32_kernel");
        return;
    }
    const LinearShape shape{w.qtype, w.M, w.K, (w.K + 31) / 32, rows};
    if (rows > 1 && gemm_supported(shape)) {
        ensure_workspace(s, gemm_workspace_bytes(shape));
        check(launch_gemm(shape, w.data, X, Y, ws_, ws_bytes_, s), "launch_gemm");
        return;
    }
    GemvGroup g{};
    g.W[0] = w.data;
    g.y[0] = Y;
    g.ncalls = 1;
    check(launch_gemv_group(shape, g, X, s), "launch_gemv_group");
}

// The GEMM workspace grows to `need` bytes (a retired one is kept until the
// decoder closes: launches queued before the growth may still use it).
void Decoder::ensure_workspace(hipStream_t s, size_t need) {
    if (need <= ws_bytes_) return;
    check(hipStreamSynchronize(s), "hipStreamSynchronize");
    void* p = nullptr;
    check(hipMalloc(&p, need), "hipMalloc");
    // Split-K counters start at zero: cleared on this stream, ahead of the
    // GEMM (a plain hipMemset runs on the null stream, which this non-blocking
    // stream does not wait for).
    check(hipMemsetAsync(p, 0, need, s), "hipMemsetAsync");
    allocs_.push_back(p);
    ws_ = p;
    ws_bytes_ = need;
}

void Decoder::linear_rows_group(hipStream_t s, int n, const Linear* const* w, const float* X, float* const* Y,
                                int rows) {
    bool grouped = rows > 1 && n > 1;
    for (int g = 0; grouped && g < n; ++g)
        grouped = w[g]->qtype != 0 && w[g]->qtype == w[0]->qtype && w[g]->K == w[0]->K;
    if (grouped) {
        LinearShape total{w[0]->qtype, 0, w[0]->K, (w[0]->K + 31) / 32, rows};
        const void* wd[3];
        int M[3];
        for (int g = 0; g < n; ++g) {
            wd[g] = w[g]->data;
            M[g] = w[g]->M;
            total.M += M[g];
        }
        if (gemm_supported(total)) {
            ensure_workspace(s, gemm_workspace_bytes(total));
            const hipError_t e = launch_gemm_group(total, n, wd, Y, M, X, ws_, ws_bytes_, s);
            if (e != hipErrorNotSupported) {
                check(e, "launch_gemm_group");
                return;
            }
        }
    }
    for (int g = 0; g < n; ++g) linear_rows(s, *w[g], X, Y[g], rows);
}

bool Decoder::prefill_batched() const {
    const int hd = cfg_.head_dim;
    return hd == 16 || hd == 32 || hd == 64 || hd == 128 || hd == 256;
}

// forward_batch over tokens[0..n) (device pointer) at positions start..:
// every layer for all rows at once; X_ row n-1 ends as the last token's
// residual stream (its final norm and lm_head are the caller's).
// Where the GEMM of `ng` weights over `rows` rows reads a split x that the
// kernel producing its input can write itself (same qtype and K for all, a
// chunk GEMM that splits x, K <= 16 384); false: the usual plain-x path.
bool Decoder::split_target(int ng, const Linear* const* w, int rows, SplitTarget& t) const {
    for (int g = 0; g < ng; ++g) {
        if (w[g]->qtype == 0 || w[g]->qtype != w[0]->qtype || w[g]->K != w[0]->K) return false;
        t.M[g] = w[g]->M;
        t.w[g] = w[g]->data;
    }
    const int K = w[0]->K;
    if (K % 32 != 0 || K > 256 * kXsCache * 16) return false;
    t.ng = ng;
    t.shape = LinearShape{w[0]->qtype, 0, K, K / 32, rows};
    for (int g = 0; g < ng; ++g) t.shape.M += t.M[g];
    t.sx = gemm_split_x(t.shape, ng, t.M);
    return t.sx.ok;
}

namespace {
// C = half blocks per thread, from the row width (at most kXsCache).
template <int QT>
void launch_norm_split(hipStream_t s, int npad, float* X, const float* D, const float* w, int dim, float eps, int n,
                       char* ws, const GemmSplitX& sx) {
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(npad), dim3(256), 0, s, X, D, w, dim, eps, n, dim / 32,
                           reinterpret_cast<_Float16*>(ws + sx.xs), reinterpret_cast<float*>(ws + sx.bsum),
                           reinterpret_cast<float*>(ws + sx.scale));
    };
    switch ((dim / 16 + 255) / 256) {
        case 1: go(add_rmsnorm_split_rows_kernel<QT, 1>); break;
        case 2: go(add_rmsnorm_split_rows_kernel<QT, 2>); break;
        case 3: go(add_rmsnorm_split_rows_kernel<QT, 3>); break;
        default: go(add_rmsnorm_split_rows_kernel<QT, 4>); break;
    }
}
template <int QT>
void launch_swiglu_split(hipStream_t s, int npad, const float* G, const float* U, int hidden, int n, char* ws,
                         const GemmSplitX& sx) {
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(npad), dim3(256), 0, s, G, U, hidden, n, hidden / 32,
                           reinterpret_cast<_Float16*>(ws + sx.xs), reinterpret_cast<float*>(ws + sx.bsum),
                           reinterpret_cast<float*>(ws + sx.scale));
    };
    switch ((hidden / 16 + 255) / 256) {
        case 1: go(swiglu_split_rows_kernel<QT, 1>); break;
        case 2: go(swiglu_split_rows_kernel<QT, 2>); break;
        case 3: go(swiglu_split_rows_kernel<QT, 3>); break;
        default: go(swiglu_split_rows_kernel<QT, 4>); break;
    }
}
}  // namespace

// The GEMM of a split target whose split x is in the workspace.
void Decoder::gemm_split(hipStream_t s, const SplitTarget& t, float* const* Y) {
    check(launch_gemm_group(t.shape, t.ng, t.w, Y, t.M, nullptr, ws_, ws_bytes_, s, true), "launch_gemm_group");
}

// X += D (when given), then the rmsnorm of X times w into the GEMM of `t`:
// written split into the workspace when t is a split target, else as H.
void Decoder::norm_into(hipStream_t s, const SplitTarget* t, float* X, const float* D, const float* w, int n) {
    const DecoderConfig& c = cfg_;
    if (t == nullptr) {
        hipLaunchKernelGGL(add_rmsnorm_rows_kernel, dim3(n), dim3(kNormThreads), 0, s, X, D, w, c.dim,
                           c.rms_norm_eps, H_);
        check(hipGetLastError(), "add_rmsnorm_rows_kernel");
        return;
    }
    ensure_workspace(s, t->sx.ws_bytes);
    char* ws = static_cast<char*>(ws_);
    switch (t->shape.qtype) {
        case 1: launch_norm_split<1>(s, t->sx.npad, X, D, w, c.dim, c.rms_norm_eps, n, ws, t->sx); break;
        case 2: launch_norm_split<2>(s, t->sx.npad, X, D, w, c.dim, c.rms_norm_eps, n, ws, t->sx); break;
        default: launch_norm_split<3>(s, t->sx.npad, X, D, w, c.dim, c.rms_norm_eps, n, ws, t->sx); break;
    }
    check(hipGetLastError(), "add_rmsnorm_split_rows_kernel");
}

void Decoder::enqueue_prefill(hipStream_t s, const int32_t* tokens, int n, int start) {
    const DecoderConfig& c = cfg_;
    const int kv_dim = c.n_kv_heads * c.head_dim;
    hipLaunchKernelGGL(embed_rows_kernel, dim3((c.dim + 255) / 256, n), dim3(256), 0, s, embedding_, c.vocab_size,
                       c.dim, tokens, state_, X_);
    check(hipGetLastError(), "embed_rows_kernel");
    for (int l = 0; l < c.n_layers; ++l) {
        const Layer& L = layers_[l];
        // q/k/v: the attention RMSNorm writes the grouped GEMM's split x
        // itself where the GEMM splits x (saves the split launch per GEMM).
        {
            const Linear* w[3] = {&L.wq, &L.wk, &L.wv};
            // Without a v bias, v goes straight into this pass's cache rows
            // (rows start .. start + n - 1 are contiguous, kv_dim apart).
            float* const vdst = L.bv == nullptr
                                    ? vcache_ + (static_cast<size_t>(l) * c.max_seq_len + start) * kv_dim
                                    : V_;
            float* y[3] = {Q_, K_, vdst};
            SplitTarget t;
            if (split_target(3, w, n, t)) {
                norm_into(s, &t, X_, l == 0 ? nullptr : FF_, L.attn_norm, n);
                gemm_split(s, t, y);
            } else {
                norm_into(s, nullptr, X_, l == 0 ? nullptr : FF_, L.attn_norm, n);
                linear_rows_group(s, 3, w, H_, y, n);
            }
        }
        // Rotating workgroups: about four head steps each.
        const int rope_hg = 256 / (c.head_dim / 2);
        const int rot_wgs = std::max(1, (c.n_heads + c.n_kv_heads + 4 * rope_hg - 1) / (4 * rope_hg));
        const int copy_wgs = L.bv == nullptr ? 0 : (kv_dim + 255) / 256;  // v (+ bias) into the cache
        hipLaunchKernelGGL(rope_kv_rows_kernel, dim3(rot_wgs + copy_wgs, n), dim3(256), 0, s, Q_, K_,
                           V_, L.bq, L.bk, L.bv, c.n_heads, c.n_kv_heads, c.head_dim, c.rope_theta, c.rope_neox,
                           c.max_seq_len, l, start, kcache_, vcache_, rot_wgs);
        check(hipGetLastError(), "rope_kv_rows_kernel");
#define MLQ_ATTN_MFMA(HD, W, PF, KS)                                                                             \
    hipLaunchKernelGGL((attention_rows_mfma_kernel<HD, W, PF, KS>),                                              \
                       dim3(c.n_heads, (n + 16 * (W / KS) - 1) / (16 * (W / KS))), dim3(64 * W), 0, s, Q_, kcache_,  \
                       vcache_, c.n_heads, c.n_kv_heads, c.max_seq_len, l, start, n, ATT_)
#define MLQ_ATTN_ROWS(LPR, V4, QR, A)                                                                           \
    hipLaunchKernelGGL((attention_rows_kernel<LPR, V4, QR, A>), dim3(c.n_heads, (n + QR - 1) / QR),            \
                       dim3(kPrefillAttnThreads), 0, s, Q_, kcache_, vcache_, c.n_heads, c.n_kv_heads, c.max_seq_len, l, \
                       start, n, ATT_)
        // VALU kernel (other head sizes): (lanes per cache row, float4s per lane, query rows per workgroup,
        // passes in flight).  LLaMA-7B shape (32 heads x 128, 512 rows, MI355X):
        // prefill 27.7 ms with one float4 per lane (32 lanes per row, per-row
        // softmax update) -> 25.4-25.6 ms at (16, 2, 4, 2); (8, 4, 4, 1) 25.7,
        // (8, 4, 2, 1) 25.5-25.9, 8 query rows 26.2-28.7, (32, 1, 4, 2-4) 26.5-26.9.
        switch (c.head_dim) {
            case 16: MLQ_ATTN_ROWS(4, 1, 4, 2); break;
            case 32: MLQ_ATTN_ROWS(8, 1, 4, 2); break;
            // MFMA: (waves, key steps in flight, key splits).  LLaMA-7B shape,
            // 512 rows, kernel µs per layer: (4, 2, 1) 43.0, (4, 2, 2) 41.0,
            // (4, 1, 2) 37.8, (8, 2, 2) 32.4, (8, 1, 2) 31.3, (8, 1, 4) 37.1,
            // (16, 1, 2) 43.5 (spills).
            case 64: MLQ_ATTN_MFMA(64, 8, 1, 2); break;
            case 128: MLQ_ATTN_MFMA(128, 8, 1, 2); break;
            default: MLQ_ATTN_ROWS(32, 2, 4, 2); break;
        }
#undef MLQ_ATTN_ROWS
#undef MLQ_ATTN_MFMA
        check(hipGetLastError(), "attention_rows_kernel");
        linear_rows(s, L.wo, ATT_, PROJ_, n);
        {
            const Linear* w[2] = {&L.w_gate, &L.w_up};
            float* y[2] = {GATE_, UP_};
            SplitTarget t;
            if (split_target(2, w, n, t)) {
                norm_into(s, &t, X_, PROJ_, L.ffn_norm, n);
                gemm_split(s, t, y);
            } else {
                norm_into(s, nullptr, X_, PROJ_, L.ffn_norm, n);
                linear_rows_group(s, 2, w, H_, y, n);
            }
        }
        {
            const Linear* w[1] = {&L.w_down};
            float* y[1] = {FF_};
            SplitTarget t;
            if (split_target(1, w, n, t)) {
                ensure_workspace(s, t.sx.ws_bytes);
                char* ws = static_cast<char*>(ws_);
                switch (t.shape.qtype) {
                    case 1: launch_swiglu_split<1>(s, t.sx.npad, GATE_, UP_, c.hidden_dim, n, ws, t.sx); break;
                    case 2: launch_swiglu_split<2>(s, t.sx.npad, GATE_, UP_, c.hidden_dim, n, ws, t.sx); break;
                    default: launch_swiglu_split<3>(s, t.sx.npad, GATE_, UP_, c.hidden_dim, n, ws, t.sx); break;
                }
                check(hipGetLastError(), "swiglu_split_rows_kernel");
                gemm_split(s, t, y);
            } else {
                const int nh = n * c.hidden_dim;
                hipLaunchKernelGGL(swiglu_kernel, dim3((nh + 255) / 256), dim3(256), 0, s, GATE_, UP_, ACT_, nh);
                check(hipGetLastError(), "swiglu_kernel");
                linear_rows(s, L.w_down, ACT_, FF_, n);
            }
        }
    }
    // Residual of the last layer into the rows' streams.
    hipLaunchKernelGGL(add_rmsnorm_rows_kernel, dim3(n), dim3(kNormThreads), 0, s, X_, FF_, final_norm_, c.dim,
                       c.rms_norm_eps, H_);
    check(hipGetLastError(), "add_rmsnorm_rows_kernel");
}

void Decoder::prefill(const int* tokens, int n, int start, float* logits_host) {
    const DecoderConfig& c = cfg_;
    if (n <= 0) throw std::runtime_error("forward_batch: empty batch");
    for (int i = 0; i < n; ++i) {
        if (tokens[i] < 0 || tokens[i] >= c.vocab_size) throw std::out_of_range("forward_token token id out of range");
    }
    if (start < 0 || static_cast<long long>(start) + n > c.max_seq_len) {
        throw std::out_of_range("forward_token position out of range");
    }
    check(hipSetDevice(device_), "hipSetDevice");
    if (!prefill_batched() || n == 1) {
        for (int i = 0; i < n; ++i) forward(tokens[i], start + i, logits_host);
        return;
    }
    ensure_io(static_cast<size_t>(n));
    ensure_prefill();
    DecodeState st{};
    check(hipMemcpyAsync(state_, &st, sizeof st, hipMemcpyHostToDevice, stream_), "hipMemcpyAsync");
    check(hipMemcpyAsync(io_, tokens, static_cast<size_t>(n) * 4, hipMemcpyHostToDevice, stream_), "hipMemcpyAsync");
    for (int c0 = 0; c0 < n; c0 += kPrefillRows) {
        const int rows = std::min(kPrefillRows, n - c0);
        enqueue_prefill(stream_, io_ + c0, rows, start + c0);
        if (c0 + rows == n) {
            // Logits of the last token: its normed row through the lm_head.
            const Linear* lm[1] = {&lm_head_};
            float* lm_y[1] = {logits_};
            linear_group(stream_, lm, lm_y, 1, H_ + static_cast<size_t>(rows - 1) * c.dim);
        }
    }
    if (logits_host != nullptr) {
        check(hipMemcpyAsync(logits_host, logits_, static_cast<size_t>(c.vocab_size) * 4, hipMemcpyDeviceToHost,
                             stream_),
              "hipMemcpyAsync");
    }
    check(hipMemcpyAsync(&st, state_, sizeof st, hipMemcpyDeviceToHost, stream_), "hipMemcpyAsync");
    check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
    if (st.error != 0) throw std::runtime_error("HIP decoder: device step reported error " + std::to_string(st.error));
}

void Decoder::ensure_io(size_t need) {
    if (need <= io_cap_) return;
    check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
    if (graph_) {
        (void)hipGraphExecDestroy(graph_);
        graph_ = nullptr;
    }
    void* p = nullptr;
    check(hipMalloc(&p, need * 4), "hipMalloc");
    allocs_.push_back(p);
    io_ = static_cast<int32_t*>(p);
    io_cap_ = need;
}

void Decoder::forward(int token, int pos, float* logits_host) {
    const DecoderConfig& c = cfg_;
    if (token < 0 || token >= c.vocab_size) throw std::out_of_range("forward_token token id out of range");
    if (pos < 0 || pos >= c.max_seq_len) throw std::out_of_range("forward_token position out of range");
    check(hipSetDevice(device_), "hipSetDevice");
    DecodeState st{};
    st.pos = pos;
    st.token = token;
    check(hipMemcpyAsync(state_, &st, sizeof st, hipMemcpyHostToDevice, stream_), "hipMemcpyAsync");
    enqueue_step(stream_, false, false);
    check(hipMemcpyAsync(logits_host, logits_, static_cast<size_t>(c.vocab_size) * 4, hipMemcpyDeviceToHost, stream_),
          "hipMemcpyAsync");
    check(hipMemcpyAsync(&st, state_, sizeof st, hipMemcpyDeviceToHost, stream_), "hipMemcpyAsync");
    check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
    if (st.error != 0) throw std::runtime_error("HIP decoder: device step reported error " + std::to_string(st.error));
}

void Decoder::generate(const int* prompt, int n_prompt, int n_new, int* out) {
    const DecoderConfig& c = cfg_;
    if (n_prompt <= 0) throw std::runtime_error("forward_batch: empty batch");
    if (n_new <= 0) return;
    for (int i = 0; i < n_prompt; ++i) {
        if (prompt[i] < 0 || prompt[i] >= c.vocab_size) throw std::out_of_range("forward_token token id out of range");
    }
    if (static_cast<long long>(n_prompt) + n_new - 1 > c.max_seq_len) {
        throw std::out_of_range("forward_token position out of range");
    }
    check(hipSetDevice(device_), "hipSetDevice");
    // One upload: the state, then the prompt; the generated tokens follow it.
    ensure_io(static_cast<size_t>(n_prompt) + n_new);
    const bool batched = prefill_batched() && n_prompt > 2;
    if (batched) ensure_prefill();
    // The decode step (pick, feed back, advance) is recorded once, on an idle
    // stream, before anything of this call is queued.
    if (graph_ == nullptr) {
        check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
        hipGraph_t gr = nullptr;
        check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        try {
            enqueue_step(stream_, true, true);
        } catch (...) {
            (void)hipStreamEndCapture(stream_, &gr);
            if (gr) (void)hipGraphDestroy(gr);
            throw;
        }
        check(hipStreamEndCapture(stream_, &gr), "hipStreamEndCapture");
        const hipError_t e = hipGraphInstantiate(&graph_, gr, nullptr, nullptr, 0);
        (void)hipGraphDestroy(gr);
        check(e, "hipGraphInstantiate");
    }
    // With a batched prefill of prompt tokens 0..n_prompt-2 the first
    // recorded step starts at the last prompt token.
    DecodeState st{};
    st.pos = batched ? n_prompt - 1 : 0;
    st.token = batched ? prompt[n_prompt - 1] : prompt[0];
    st.n_prompt = n_prompt;
    st.n_out = n_new;
    check(hipMemcpyAsync(state_, &st, sizeof st, hipMemcpyHostToDevice, stream_), "hipMemcpyAsync");
    check(hipMemcpyAsync(io_, prompt, static_cast<size_t>(n_prompt) * 4, hipMemcpyHostToDevice, stream_),
          "hipMemcpyAsync");
    // Prompt tokens before the last: one batched pass (the MFMA GEMMs), or
    // steps without the lm_head; every later step picks and feeds back.
    if (batched) {
        for (int c0 = 0; c0 < n_prompt - 1; c0 += kPrefillRows) {
            enqueue_prefill(stream_, io_ + c0, std::min(kPrefillRows, n_prompt - 1 - c0), c0);
        }
    } else {
        for (int i = 0; i + 1 < n_prompt; ++i) enqueue_step(stream_, false, true);
    }
    // The host runs at most kGenerateInflight steps ahead of the device, so a
    // long generation never has thousands of dispatches queued at once.
    for (hipEvent_t& ev : inflight_)
        if (ev == nullptr) check(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "hipEventCreateWithFlags");
    for (int i = 0; i < n_new; ++i) {
        hipEvent_t& ev = inflight_[i % kGenerateInflight];
        if (i >= kGenerateInflight) check(hipEventSynchronize(ev), "hipEventSynchronize");
        check(hipGraphLaunch(graph_, stream_), "hipGraphLaunch");
        check(hipEventRecord(ev, stream_), "hipEventRecord");
    }
    check(hipMemcpyAsync(out, io_ + n_prompt, static_cast<size_t>(n_new) * 4, hipMemcpyDeviceToHost, stream_),
          "hipMemcpyAsync");
    check(hipMemcpyAsync(&st, state_, sizeof st, hipMemcpyDeviceToHost, stream_), "hipMemcpyAsync");
    check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
    if (st.error & kDecodeErrLogits) throw std::runtime_error("sampler: logits must be finite");
    if (st.error != 0) throw std::runtime_error("HIP decoder: device step reported error " + std::to_string(st.error));
}

}  // namespace mlq

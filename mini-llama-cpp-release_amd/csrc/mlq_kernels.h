// Internal interface between the C-ABI layer (mlq_abi.hip) and the kernel
// translation units.  Not installed; the public surface is include/mlq_hip.h.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace mlq {

constexpr int kQK = 32;  // elements per block (quantized_tensor.h:24, 37, 51)

inline int block_bytes(int qtype) {
    switch (qtype) {
        case 1: return 34;  // BlockQ8_0 {u16 d; i8 qs[32]}
        case 2: return 18;  // BlockQ4_0 {u16 d; u8 qs[16]}
        case 3: return 20;  // BlockQ4_1 {u16 d; u16 m; u8 qs[16]}
        default: return 0;
    }
}

// Shape of one quantized linear launch.  W is row-major [M][nb] blocks.
struct LinearShape {
    int qtype;
    int M;      // out_features
    int K;      // in_features
    int nb;     // ceil(K / 32)
    int rows;   // batch rows of x / y
};

// Decode GEMV, rows == 1 (or a small batch launched as rows x GEMV).
// Returns hipSuccess or the launch error.
hipError_t launch_gemv(const LinearShape& s, const void* w, const float* x, float* y,
                       hipStream_t stream);
const char* gemv_kernel_name(const LinearShape& s);

// Up to kGroupMaxCalls GEMVs that read the same x (a fused q/k/v or gate/up
// launch): their rows are concatenated in call order, call j owning rows
// [row_begin[j], row_begin[j] + M_j) of the launch's s.M rows.  Each row is
// computed exactly as by a launch of its own call.
constexpr int kGroupMaxCalls = 4;

struct PickState;

struct GemvGroup {
    const void* W[kGroupMaxCalls];
    float* y[kGroupMaxCalls];
    int row_begin[kGroupMaxCalls];
    int ncalls;
    PickState* pick;  // greedy-pick launches only (launch_gemv_pick)
    int32_t* token;
    const float* norm_w;  // norm launches only: RMSNorm weights [K]
    float norm_eps;
};

hipError_t launch_gemv_group(const LinearShape& s, const GemvGroup& g, const float* x, hipStream_t stream);
// The same group with the reference's f32 arithmetic (each weight dequantized
// to f32, f32 multiply-adds with x); one token row, an even block count.
hipError_t launch_gemv_f32(const LinearShape& s, const GemvGroup& g, const float* x, hipStream_t stream);

// Greedy pick fused into the GEMV (one call, rows == 1): besides y (skipped
// when y is null) the launch writes *token = the first index of the largest
// y, or -1 when any y is not finite.  Workgroup b folds its best key into
// key[b % kPickGroups] and arrives on sub[b % kPickGroups]; the last arrival
// of a group bumps `top`, and the last of those decodes the token.  Every
// word is zero before a launch and left at zero by it; launches that share a
// PickState must not overlap in time.
constexpr int kPickGroups = 8;

struct PickState {
    unsigned long long key[kPickGroups][16];  // one 128-byte line each
    unsigned sub[kPickGroups][32];
    unsigned top[32];
};

hipError_t launch_gemv_pick(const LinearShape& s, const void* w, const float* x, float* y, PickState* ps,
                            int32_t* token, hipStream_t stream);

// Decode-step forms of a (grouped) GEMV, rows == 1 or a batch:
//  norm:       stage rmsnorm(x) * g.norm_w (eps g.norm_eps) instead of x
//              (src/ops.cpp:18-41) -- each workgroup normalises its own copy;
//  accumulate: y += W x (the residual add; y must not overlap x).
hipError_t launch_gemv_decode(const LinearShape& s, const GemvGroup& g, const float* x, bool norm, bool accumulate,
                              hipStream_t stream);
// The decode step's SwiGLU: g.W[0] = gate, g.W[1] = up (s.M rows each,
// g.row_begin[1] = s.M), rows == 1 or a batch; y[0][i] = silu(gate_i . h) *
// (up_i . h) with h = rmsnorm(x) * g.norm_w (src/ops.cpp:72-107).  Rows of at
// most 64 pairs only (gemv_glu_supported); hipErrorNotSupported otherwise.
bool gemv_glu_supported(const LinearShape& s);
hipError_t launch_gemv_glu(const LinearShape& s, const GemvGroup& g, const float* x, hipStream_t stream);
// The greedy pick over W . (rmsnorm(x) * norm_w): the final norm and lm_head
// of a decode step in one launch.
hipError_t launch_gemv_pick_norm(const LinearShape& s, const void* w, const float* x, const float* norm_w,
                                 float norm_eps, float* y, PickState* ps, int32_t* token, hipStream_t stream);

// Measurement: the weight stream of a grouped GEMV launch (same grid, units
// and ring) without the arithmetic -- the per-launch floor.  `sink` holds
// kFloorSinkWords words the kernel overwrites.
constexpr int kFloorSinkWords = 1 << 16;
hipError_t launch_stream_floor(const LinearShape& s, const GemvGroup& g, uint32_t* sink, hipStream_t stream);
// The floor's two parts: kProbeEmpty launches the floor's grid with no work;
// kProbeLoad streams the same weight bytes with plain coalesced 16-byte loads.
constexpr int kProbeEmpty = 1;
constexpr int kProbeLoad = 2;
hipError_t launch_stream_probe(const LinearShape& s, const GemvGroup& g, int mode, uint32_t* sink,
                               hipStream_t stream);

// Batched prefill GEMM for rows > 1 (MFMA).  Needs a device workspace of
// gemm_workspace_bytes(s) bytes (split x, scales, split-K partials) that no
// other launch uses concurrently.  Returns hipErrorNotSupported when the shape
// has no MFMA path (the caller runs the GEMV kernels per row instead).
bool gemm_supported(const LinearShape& s);
size_t gemm_workspace_bytes(const LinearShape& s);
hipError_t launch_gemm(const LinearShape& s, const void* w, const float* x, float* y, void* ws,
                       size_t ws_bytes, hipStream_t stream);
const char* gemm_kernel_name(const LinearShape& s);
// Up to three linears that read the same x (same qtype, K and rows; e.g. q, k
// and v of one layer) as one GEMM launch: linear g has M[g] rows and writes
// y[g] ([rows][M[g]]); s.M is ignored (the total is the sum).  A row gets the
// arithmetic of a single call of its linear, with the tile shape and K split
// that the group's total M selects.
// hipErrorNotSupported when the shape has no grouped path (no chunk kernel, or
// a weight other than the last whose M is not a multiple of the tile height):
// then launch the linears one by one.  The workspace is sized for a LinearShape
// whose M is the total.
// x_split: the workspace already holds x split as the GEMM reads it (written
// by the kernel that produced x, at the offsets gemm_split_x gives); `x` is
// not read and no split launch is made.
hipError_t launch_gemm_group(const LinearShape& s, int n, const void* const* w, float* const* y, const int* M,
                             const float* x, void* ws, size_t ws_bytes, hipStream_t stream, bool x_split = false);
// Whether launch_gemm_group would launch that group (rather than return
// hipErrorNotSupported), so a caller sizes a workspace only when it will.
bool gemm_group_supported(const LinearShape& s, int n, const int* M, const float* x);

// Where a grouped (or, n = 1, single) GEMM of `rows` > 128 token rows reads
// its split x inside the workspace (xsplit_device.h's layout: xs [npad][nb][64]
// halves, bsum [npad][nb], scale [npad]; byte offsets), and the workspace size
// the launch needs.  ok = false: the call would not read a split x (the
// producer then writes plain x and the launch splits it).
struct GemmSplitX {
    bool ok;
    int npad;
    size_t xs, bsum, scale, ws_bytes;
};
GemmSplitX gemm_split_x(const LinearShape& s, int n, const int* M);

// Persistent GEMV over a chain of linears (sequence.hip).  A stage is up to
// kSeqMaxCalls GEMVs reading the same x; their rows are concatenated in call
// order (call j owns rows [row_begin, row_begin + M)).  Descriptors live in
// device memory for as long as any launch that uses them.
constexpr int kSeqMaxCalls = kGroupMaxCalls;

struct SeqCallDesc {
    const void* W;   // [M][nb] blocks
    float* y;        // [M]
    int M;
    int row_begin;
};

struct SeqStageDesc {
    const float* x;  // [K]
    int K;
    int nb;          // blocks per row (even)
    int np;          // pairs per row
    int nch;         // chunks per row: ceil(np / lane-group width)
    int rows;        // sum of M over the stage's calls
    int items;       // row items: ceil(rows / (64 / lane-group width))
    int ncalls;
    int barrier;     // 1: wait for every earlier stage of the launch first
    int coherent;    // 1: x was written by an earlier stage of the same launch
    SeqCallDesc call[kSeqMaxCalls];
};

// Barrier words of one launch (each on its own 128-byte line); zero before
// the first launch and left at zero by every launch that completes.
// Workgroup b arrives on sub[b % kSeqGroups]; the last arrival of a group
// bumps `top`, which every workgroup polls.
constexpr int kSeqGroups = 8;

struct SeqSync {
    unsigned sub[kSeqGroups][32];
    unsigned top[32];
    unsigned exit[32];
    unsigned error[32];  // error[0] set when a barrier wait gave up (the launch's outputs are void)
};

bool sequence_supported(int qtype, int K);
int sequence_lpr(int K);                 // lane-group width for rows of K elements: 16 or 64
int sequence_stage_lds_bytes(int qtype, int K);  // x area of a stage
hipError_t sequence_grid(int qtype, int lpr, int lds_bytes, int device, int* grid);
hipError_t launch_sequence(int qtype, int lpr, const SeqStageDesc* stages, int nstages, SeqSync* sync,
                           int grid, int lds_bytes, unsigned spin_limit, hipStream_t stream);
const char* sequence_kernel_name(int qtype, int lpr);

// Pipelined chain kernel (chain.hip): the same stage descriptors, stages of
// K % 32 == 0; kmax = largest K of the launch.
int chain_lds_bytes(int qtype, int kmax);
hipError_t chain_grid(int qtype, int lpr, int lds_bytes, int device, int* grid);
hipError_t launch_chain(int qtype, int lpr, const SeqStageDesc* stages, int nstages, SeqSync* sync, int grid,
                        int lds_bytes, unsigned spin_limit, int kmax, float* sink, hipStream_t stream);
size_t chain_sink_bytes();  // device words a launch's compute lanes store dropped values to
const char* chain_kernel_name(int qtype, int lpr);

// LDS-ring chain kernel (ring.hip): the same stage descriptors, stages whose
// lane-group width is 64; kmax = largest K of the launch.  ring_lds_bytes
// gives the launch's LDS and its ring slots.
int ring_lds_bytes(int qtype, int kmax, int* nslots);
hipError_t ring_grid(int qtype, int lds_bytes, int device, int* grid);
hipError_t launch_ring(int qtype, const SeqStageDesc* stages, int nstages, SeqSync* sync, int grid, int lds_bytes,
                       unsigned spin_limit, int kmax, hipStream_t stream);
const char* ring_kernel_name(int qtype);
// Boundary timestamps of the measurement build (MLQ_RING_STAMPS): per
// workgroup 0, G/2 + 1 and G - 1, per stage, kRingStampSlots s_memrealtime
// values (slot meanings in include/mlq_hip.h).  hipErrorNotSupported in a
// normal build.
constexpr int kRingStampWgs = 3;
constexpr int kRingStampStages = 256;
constexpr int kRingStampSlots = 24;
hipError_t ring_stamps_copy(void* host, size_t bytes);

// Device forward ops (ops.hip) behind the op-by-op device interfaces of the
// reference (include/mini_llama/cuda_ops.h, cuda_attention.h, cuda_matmul.h).
constexpr int kOpSilu = 0;
constexpr int kOpMul = 1;
constexpr int kOpAdd = 2;
constexpr int kOpAttnMaxHeadDim = 512;
hipError_t launch_op_rmsnorm(const float* x, const float* w, int n, float eps, float* y, hipStream_t s);
hipError_t launch_op_elementwise(int op, const float* a, const float* b, size_t n, float* y, hipStream_t s);
hipError_t launch_op_softmax(const float* x, int n, float* y, hipStream_t s);
hipError_t launch_op_embedding(const float* table, int dim, int token, float* y, hipStream_t s);
hipError_t launch_op_rope(float* x, int n_heads, int head_dim, int pos, float theta, bool neox, hipStream_t s);
hipError_t launch_op_attention_decode(const float* q, const float* keys, const float* values, int layer,
                                      int max_seq, int n_heads, int n_kv_heads, int head_dim, int pos,
                                      float* out, hipStream_t s);
hipError_t launch_op_matmul_f32(const float* a, const float* b, int m, int k, int n, bool b_transposed, float* c,
                                hipStream_t s);

// Device quantizer and synthetic-data generator.
hipError_t launch_quantize(int qtype, const float* src, int rows, int row_len, void* dst,
                           hipStream_t stream);
hipError_t launch_fill_normal(float* dst, size_t n, uint64_t seed, float mean, float stddev,
                              hipStream_t stream);

}  // namespace mlq

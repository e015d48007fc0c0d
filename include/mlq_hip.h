/*
 * mlq_hip.h -- C ABI of the MI355X (gfx950) quantized-linear path for
 * mini-llama.cpp (yus3nable/mini-llama-cpp-release).
 *
 * Plain C: no HIP, torch or C++ types in any signature.  Pointers are either
 * host pointers or device pointers obtained from this library (or any HIP
 * allocation on the same device); which one is stated per argument.  Streams
 * are passed as `void*` holding a hipStream_t (NULL = the library's stream for
 * that device).
 *
 * Every entry point returns MLQ_OK (0) or a nonzero MLQ_ERR_* code; the message
 * of the last failure on the calling thread is returned by mlq_hip_last_error().
 * Messages follow the reference's own wording so callers that match on them
 * keep working (src/cuda_quant.cu:150-243, 253-255, 299-301).
 *
 * Citations name the reference interface each entry replaces (paths relative
 * to the reference repository).
 */
#ifndef MLQ_HIP_H
#define MLQ_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Quant types, numbered as mini_llama::QuantType
 * (include/mini_llama/quantized_tensor.h:13-18). */
#define MLQ_F32 0
#define MLQ_Q8_0 1
#define MLQ_Q4_0 2
#define MLQ_Q4_1 3

/* Bytes per 32-element block: BlockQ8_0 / BlockQ4_0 / BlockQ4_1
 * (include/mini_llama/quantized_tensor.h:26-59; src/gguf.cpp:178-197). */
#define MLQ_BLOCK_ELEMS 32
#define MLQ_Q8_0_BLOCK_BYTES 34
#define MLQ_Q4_0_BLOCK_BYTES 18
#define MLQ_Q4_1_BLOCK_BYTES 20

/* Error codes. */
#define MLQ_OK 0
#define MLQ_ERR_INVALID 1    /* bad argument: null pointer, unknown type, bad flags  */
#define MLQ_ERR_SHAPE 2      /* shape or block-count mismatch, empty tensor          */
#define MLQ_ERR_DEVICE 3     /* no such device / tensor on another device            */
#define MLQ_ERR_HIP 4        /* a HIP runtime call failed                            */
#define MLQ_ERR_NOT_BUILT 5  /* library built without kernels for this device        */
#define MLQ_ERR_LIMIT 6      /* a size exceeds a documented limit                    */

/* Flags for mlq_hip_quant_linear. */
#define MLQ_X_ON_DEVICE 0x1  /* x is a device pointer (else host, copied in)          */
#define MLQ_Y_ON_DEVICE 0x2  /* y is a device pointer (else host, copied out)         */
#define MLQ_ASYNC 0x4        /* device x and y: return without synchronizing          */

typedef struct mlq_weight_s* mlq_weight_t;

/* Thread-local message of the last failure ("" if none). */
const char* mlq_hip_last_error(void);

/* 1 when the HIP kernels are compiled in (cuda_quant_built,
 * include/mini_llama/cuda_quant.h:11; cuda_backend_built, backend.h:21). */
int mlq_hip_built(void);

/* Number of visible HIP devices (cuda_device_count,
 * include/mini_llama/cuda_runtime.h; used by cuda_backend_available,
 * src/backend.cpp:34-41). */
int mlq_hip_device_count(int* count);

/* One-line device summary into buf (cuda_format_device_info /
 * cuda_device_summary, src/backend.cpp:43-49). */
int mlq_hip_device_info(int device, char* buf, size_t len);

/* Properties of `device` (cuda_get_device_info, include/mini_llama/cuda_runtime.h:8-16,
 * src/cuda_runtime.cpp:63-93): name, gfx architecture, major.minor of the
 * architecture (9.5 for gfx950), memory, CU count, driver and runtime versions. */
typedef struct mlq_device_props {
    char name[256];
    char arch[64];
    int major;
    int minor;
    size_t total_memory_bytes;
    int compute_units;
    int driver_version;
    int runtime_version;
} mlq_device_props;
int mlq_hip_device_props(int device, mlq_device_props* out);

/* Select `device` for the calling thread and create its stream (the
 * cudaSetDevice every CudaDeviceBuffer op does, src/cuda_runtime.cpp:187-218). */
int mlq_hip_init(int device);

/* Copy `n_blocks` raw blocks of an [out_features, in_features] weight from host
 * memory to `device` and return a handle
 * (upload_q8_0/q4_0/q4_1_linear_weight, src/model.cpp:145-272; validation
 * mirrors their messages).  The bytes are stored exactly as given. */
int mlq_hip_upload_weight(int device, int qtype, const void* host_blocks, size_t n_blocks,
                          int out_features, int in_features, mlq_weight_t* out);

/* Wrap blocks already resident on `device` (not owned; the caller keeps them
 * alive).  Mirrors the `const void* q*_device, size_t block_count` pair of
 * cuda_q*_linear_device_weight / _device_input (include/mini_llama/cuda_quant.h:21-86). */
int mlq_hip_wrap_weight(int device, int qtype, const void* device_blocks, size_t n_blocks,
                        int out_features, int in_features, mlq_weight_t* out);

/* Release a handle (and its device memory if uploaded).  NULL is a no-op. */
int mlq_hip_free_weight(mlq_weight_t w);

/* Properties of a handle; any out pointer may be NULL. */
int mlq_hip_weight_info(mlq_weight_t w, int* qtype, int* out_features, int* in_features,
                        size_t* n_blocks, const void** device_blocks, int* device);

/* y[rows, out_features] = x[rows, in_features] * W^T in f32.
 * rows == 1 is decode (the GEMV kernels); rows > 1 is the batched prefill
 * GEMM.  With flags 0, x and y are host pointers: x is copied in, y copied back
 * and the call returns when y is ready (cuda_q*_linear_device_weight,
 * include/mini_llama/cuda_quant.h:21-28).  With MLQ_X_ON_DEVICE |
 * MLQ_Y_ON_DEVICE both live on the weight's device
 * (cuda_q*_linear_device_input, include/mini_llama/cuda_quant.h:30-36); add
 * MLQ_ASYNC to return right after the launch on `stream`. */
int mlq_hip_quant_linear(mlq_weight_t w, const float* x, int rows, float* y, int flags,
                         void* stream);

/* The device-pointer form of mlq_hip_quant_linear (MLQ_X_ON_DEVICE |
 * MLQ_Y_ON_DEVICE | MLQ_ASYNC) that allocates nothing: batched calls
 * (rows > 1) use a fixed 48 MiB scratch array the library holds on each GPU
 * (from library set-up until the process ends) instead of the stream's
 * workspace, so the call works under graph capture, in serving loops and in
 * harnesses that forbid hipMalloc, from the first call on.  A shape whose GEMM
 * needs more scratch is refused with MLQ_ERR_LIMIT (2048 token rows of a
 * 4096x4096 weight fit, 4096 do not).  All calls on one GPU share the scratch: calls that
 * overlap in time on one GPU (different streams, or a graph replayed while
 * another runs) race and give wrong results, and such a race can leave a
 * split-K arrival counter of the scratch off zero, after which every later
 * batched call of this entry on that GPU is wrong too, until the process
 * ends.  Serialise the calls of one GPU (one stream, or events).  Results equal
 * mlq_hip_quant_linear bit for bit.  No counterpart in the reference; for
 * callers that cannot allocate. */
int mlq_hip_quant_linear_noalloc(mlq_weight_t w, const float* x, int rows, float* y, void* stream);

/* Device-pointer form without a handle: cuda_q8_0/q4_0/q4_1_linear_device_input
 * (include/mini_llama/cuda_quant.h:30-86, src/cuda_quant.cu:289-496).  x and y
 * are device pointers on `device`; the call is asynchronous on `stream`. */
int mlq_hip_quant_linear_device(int device, int qtype, const void* device_blocks, size_t n_blocks,
                                int out_features, int in_features, const float* x, int rows,
                                float* y, void* stream);

/* Several independent linears in one call (one launch each, issued from C):
 * the decode step's per-layer projections without a host round trip per call.
 * All handles must be on one device; x/y are device pointers. */
typedef struct mlq_linear_call {
    mlq_weight_t w;
    const float* x;
    float* y;
    int rows;
} mlq_linear_call;
int mlq_hip_quant_linear_many(const mlq_linear_call* calls, int n, void* stream);

/* Up to 4 linears that read the same x, in one launch: the fused q/k/v or
 * gate/up projection of a decode step (rows == 1: GEMVs, per call equal to
 * mlq_hip_quant_linear bit for bit) or of a batched prefill (rows > 1: one
 * grouped MFMA GEMM over up to 3 weights when each weight but the last is a
 * whole number of the GEMM's row tiles -- 64 or 128 rows --, else one launch
 * per call; per call within the linear's tolerance of mlq_hip_quant_linear,
 * whose K split may differ because the group's total rows pick it).  Same x,
 * rows, in_features and quant type for every call; outputs disjoint from each
 * other and from x.  No counterpart in the reference (its forward issues one
 * linear per projection, src/forward.cpp:172-227).  Asynchronous on `stream`. */
int mlq_hip_quant_linear_fused(const mlq_linear_call* calls, int n, void* stream);

/* The same fused launch (one token row, an even block count) with the
 * reference's f32 arithmetic instead of the integer block sums: each weight
 * dequantized to f32 as quantized_linear's dequant functions do
 * (src/quant.cpp:413-429, 435-460: d * (q - 8), d * q, d * q + m) and
 * multiplied into an f32 sum of x; each lane sums its elements in k order
 * with fused multiply-adds and the lanes' sums meet in a butterfly.  Slower
 * than mlq_hip_quant_linear_fused (about three VALU operations and an LDS
 * read of x per weight against about one), closer to the CPU's f32 sums;
 * there for callers that want that and to price the integer path.
 * Asynchronous on `stream`. */
int mlq_hip_quant_linear_fused_f32(const mlq_linear_call* calls, int n, void* stream);

/* Measurement, not a linear: streams exactly the weights a fused launch of
 * `calls` (as mlq_hip_quant_linear_fused; x and y are ignored) would read,
 * with the GEMV kernels' grid, work units and request ring, and no
 * arithmetic; `sink` is a device buffer of 65536 words it overwrites.  Its
 * time is the floor of a GEMV launch of that shape (launch plus weight
 * stream).  Asynchronous on `stream`. */
int mlq_hip_stream_floor(const mlq_linear_call* calls, int n, void* sink, void* stream);

/* Measurement, not a linear: the floor's two parts, for the same `calls` and
 * `sink`.  MLQ_PROBE_EMPTY launches the floor's grid and does nothing (the
 * cost of a launch); MLQ_PROBE_LOAD streams the same weight bytes with plain
 * coalesced 16-byte loads, each thread reading every T-th unit of the calls'
 * weights taken back to back (the cost of the bytes without the GEMV's work
 * units; a tail under 16 bytes per weight is not read).  Asynchronous on
 * `stream`. */
#define MLQ_PROBE_EMPTY 1
#define MLQ_PROBE_LOAD 2
int mlq_hip_stream_probe(const mlq_linear_call* calls, int n, int mode, void* sink, void* stream);

/* Greedy pick fused into the decode GEMV of an output projection (lm_head):
 * y = W x as mlq_hip_quant_linear (bit for bit; y may be NULL when the logits
 * are not needed) and *token = the first index of the largest y, or -1 when
 * any y is infinite or NaN.  Replaces downloading the logits
 * (compute_logits_device, src/forward.cpp:849-853) and picking on the host
 * (MiniSampler::sample_greedy, src/sampler.cpp:91-95: validate_logits,
 * src/sampler.cpp:15-24, then argmax, src/ops.cpp:179-192), so greedy decode
 * moves 4 bytes per token instead of the logits.  x, y and token are device
 * pointers on the weight's device; asynchronous on `stream`.  Uses a small
 * per-stream state the library creates on the stream's first call (which
 * must not be under graph capture); calls on one stream are ordered by it. */
int mlq_hip_quant_linear_argmax(mlq_weight_t w, const float* x, float* y, int32_t* token, void* stream);

/* Synchronous form: the token is returned to the host.  Fails with
 * MLQ_ERR_INVALID and the reference's message "sampler: logits must be
 * finite" when any logit is not finite (src/sampler.cpp:19-22). */
int mlq_hip_sample_greedy(mlq_weight_t w, const float* x, float* y, int* token, void* stream);

/* Quantize an f32 [rows, row_len] matrix that is already on `device` into
 * blocks on the same device, bit-identical to the reference quantizers:
 * quantize_to_q8_0 / quantize_to_q4_0 (src/quant.cpp:112-170, 207-270) and
 * the Q4_1 routine of tests/test_cuda_quant.cpp:129-180 (including its
 * round-half-up fp16 scale encoding, src/quant.cpp:19-55). */
int mlq_hip_quantize(int device, int qtype, const float* src, int rows, int row_len,
                     void* device_blocks, void* stream);

/* ---- device memory, streams, events and graphs (plumbing for callers that
 * have no HIP runtime of their own, e.g. ctypes/cgo bindings) ---- */
int mlq_hip_malloc(int device, size_t bytes, void** out);
int mlq_hip_free(void* ptr);
int mlq_hip_memcpy_htod(void* dst, const void* src, size_t bytes);
int mlq_hip_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int mlq_hip_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream);
int mlq_hip_memset(void* ptr, int value, size_t bytes);
int mlq_hip_stream(int device, void** stream);       /* the library's stream for device */
/* A new non-blocking stream on `device` (default priority) and its release.
 * The library keeps per-stream state (batched-call workspace, pick state)
 * until the process ends; destroy a stream only when no graph recorded on it
 * is replayed any more. */
int mlq_hip_stream_create(int device, void** stream);
int mlq_hip_stream_destroy(void* stream);
int mlq_hip_synchronize(void* stream);
int mlq_hip_event_create(void** ev);
int mlq_hip_event_destroy(void* ev);
int mlq_hip_event_record(void* ev, void* stream);
int mlq_hip_event_elapsed_ms(void* start, void* stop, float* ms);

/* Capture mlq_hip_quant_linear_many(calls, n) into a graph and instantiate it;
 * replay with mlq_hip_graph_launch.  Buffers are baked in at capture time,
 * including the stream's batched-call workspace: when a later, larger batched
 * call grows that workspace, the old buffer is kept (never freed) for the
 * graphs that recorded it.  Replays of such a graph share its workspace with
 * nothing else as long as they run on the stream it was recorded on. */
typedef struct mlq_graph_s* mlq_graph_t;
int mlq_hip_graph_capture_many(const mlq_linear_call* calls, int n, void* stream, mlq_graph_t* out);
int mlq_hip_graph_launch(mlq_graph_t g, void* stream);
int mlq_hip_graph_destroy(mlq_graph_t g);

/* Record any asynchronous launches this thread issues on `stream` between
 * begin and end (mlq_hip_quant_linear with device x/y and MLQ_ASYNC, _many,
 * _fused, _argmax, sequence launches) as one graph, e.g. a whole decode step.
 * Calls that synchronize or copy host memory fail under capture, and so does
 * the first batched or picking call on a stream (it creates the stream's
 * state): make one of each before capturing.  No counterpart in the
 * reference, which launches eagerly (src/cuda_quant.cu:289-496). */
int mlq_hip_graph_begin(int device, void* stream);
int mlq_hip_graph_end(int device, void* stream, mlq_graph_t* out);

/* A decode step's chain of GEMVs run as one persistent launch (per run of
 * same-format stages).  No counterpart in the reference, whose forward pass
 * launches one kernel per linear (src/forward.cpp:172-227, through
 * src/cuda_quant.cu:289-496); per call the results equal those of
 * mlq_hip_quant_linear on the same inputs, bit for bit.
 *
 * calls[i] are GEMV calls (rows == 1) on one device, with an even number of
 * blocks per row and at most 15 360 input features.  Consecutive calls with
 * equal stage[i] form one stage (at most 4 calls): they read the same x, run
 * concurrently, and no call of the stage writes where the stage reads or
 * another of its calls writes.  stage == NULL puts every call in a stage of
 * its own.  No y may overlap any weight of the sequence.
 * Modes:
 *   MLQ_SEQ_PERSISTENT   one launch; each stage starts after every earlier
 *                        stage has written its outputs (device-wide barrier),
 *                        so a call may read any earlier call's y;
 *   MLQ_SEQ_PER_STAGE    one launch per stage, ordered by the stream (same
 *                        semantics, no device-wide barrier);
 *   MLQ_SEQ_INDEPENDENT  one launch without barriers: no call may read any
 *                        call's output (checked when the sequence is created);
 *   MLQ_SEQ_PIPELINED    the semantics of MLQ_SEQ_PERSISTENT (device-wide
 *                        barrier before every stage) in one launch whose
 *                        weight requests run ahead across the barriers: per
 *                        workgroup a control wave stores a stage's last rows,
 *                        synchronizes the grid and loads the next x while the
 *                        compute waves' next-stage weights are in flight.
 *                        Every call needs in_features % 32 == 0.
 *   MLQ_SEQ_LDS_RING     the semantics of MLQ_SEQ_PERSISTENT in one launch
 *                        whose weight stream does not wait for x: per CU,
 *                        loader waves copy the weights of every stage, in
 *                        order, into a ring in LDS as far ahead as the ring
 *                        holds, and compute waves take them from there once
 *                        the stage's x is staged.  Every call needs rows
 *                        that a single launch sums in 64-lane groups (e.g.
 *                        in_features 4096 and 11008; not 896 or 1024) and a
 *                        weight under 2 GiB.
 * The sequence keeps the pointers (buffers must outlive it and any graph
 * captured from it); launches of one sequence must not overlap in time. */
typedef struct mlq_sequence_s* mlq_sequence_t;
#define MLQ_SEQ_PERSISTENT 0
#define MLQ_SEQ_PER_STAGE 1
#define MLQ_SEQ_INDEPENDENT 2
#define MLQ_SEQ_PIPELINED 3
#define MLQ_SEQ_LDS_RING 4
int mlq_hip_sequence_create(const mlq_linear_call* calls, int n, const int* stage, int mode,
                            mlq_sequence_t* out);
/* Measurement, not part of the linear: the last MLQ_SEQ_LDS_RING launch's
 * boundary timestamps, from a library built with `make stamps`
 * (libmlq_hip_stamps.so; MLQ_ERR_NOT_BUILT from the normal build).  `host`
 * receives 3 x 256 x 24 uint64 s_memrealtime values (100 MHz): for
 * workgroups 0, G/2 + 1 and G - 1 (G = the launch's grid), per stage (the
 * first 256), slots 0 stage entered by the first compute wave, 1 its y stores
 * complete, 2 every compute wave done, 3 grid barrier passed (barrier stages),
 * 4 x staged, 5 every compute wave's x staged, 6/7 before / after the wait for
 * its first unit, 8 + w compute wave w done with the stage's rows (w < 12),
 * 20 / 21 / 22 loader 0's first unit of the stage in LDS / its last unit in
 * LDS / its first unit of the stage requested.  No counterpart in the
 * reference. */
#define MLQ_RING_STAMP_WORDS (3 * 256 * 24)
int mlq_hip_ring_stamps(uint64_t* host, size_t words);
int mlq_hip_sequence_launch(mlq_sequence_t seq, void* stream);
/* After the launch's stream has been synchronized: the number of launches
 * whose device-wide barrier wait gave up (outputs void), then cleared. */
int mlq_hip_sequence_status(mlq_sequence_t seq, int* barrier_timeouts);
/* Bound of each barrier wait in polls (default 1 << 20, about a second). */
int mlq_hip_sequence_set_spin_limit(mlq_sequence_t seq, unsigned polls);
int mlq_hip_sequence_info(mlq_sequence_t seq, int* stages, int* launches, int* grid);
int mlq_hip_sequence_destroy(mlq_sequence_t seq);
int mlq_hip_graph_capture_sequence(mlq_sequence_t seq, void* stream, mlq_graph_t* out);

/* Fill an f32 device array with N(mean, std) from a counter-based generator
 * (splitmix64 + Box-Muller) -- synthetic weights and inputs for benchmarks. */
int mlq_hip_fill_normal(float* device_dst, size_t n, uint64_t seed, float mean, float stddev,
                        void* stream);

/* ---- Device forward ops around the linears ----
 * The op-by-op device interfaces of the reference's forward
 * (include/mini_llama/cuda_ops.h:9-75, cuda_attention.h:11-31,
 * cuda_matmul.h:8-38; kernels src/cuda_ops.cu:30-170, src/cuda_attention.cu,
 * cuBLAS in src/cuda_matmul.cpp) on device pointers of `device`,
 * asynchronous on `stream` (NULL: the library's stream for the device).  The
 * arithmetic is the reference's CPU ops' in f32 (src/ops.cpp:19-79, 109-176,
 * src/forward.cpp:580-600).  Every pointer must lie inside a device allocation
 * of at least the size the shape implies (else MLQ_ERR_LIMIT /
 * MLQ_ERR_DEVICE, and nothing is launched). */
/* y = x / sqrt(mean(x^2) + eps) * weight over n elements (cuda_rmsnorm*). */
int mlq_hip_rmsnorm(int device, const float* x, const float* weight, int n, float eps, float* y, void* stream);
/* y = x / (1 + exp(-x)) (cuda_silu*); y = a * b (cuda_elementwise_mul*);
 * y = a + b (cuda_elementwise_add*). */
int mlq_hip_silu(int device, const float* x, size_t n, float* y, void* stream);
int mlq_hip_mul(int device, const float* a, const float* b, size_t n, float* y, void* stream);
int mlq_hip_add(int device, const float* a, const float* b, size_t n, float* y, void* stream);
/* Softmax of one vector of n elements (cuda_softmax). */
int mlq_hip_softmax(int device, const float* x, int n, float* y, void* stream);
/* y[dim] = row `token` of the [vocab][dim] table (cuda_embedding_lookup_device_weight). */
int mlq_hip_embedding(int device, const float* table, int vocab, int dim, int token, float* y, void* stream);
/* RoPE in place on x [n_heads][head_dim] at position pos (cuda_rope*): pairs
 * (2i, 2i+1) or, with neox != 0, (i, i + head_dim/2) (RopeType::NeoX). */
int mlq_hip_rope(int device, float* x, int n_heads, int head_dim, int pos, float theta, int neox, void* stream);
/* Single-token attention (cuda_attention_decode*): out [n_heads][head_dim] from
 * q [n_heads][head_dim] over positions 0..pos of `layer` of a KV cache laid out
 * [n_layers][max_seq_len][n_kv_heads][head_dim] (CudaKVCache); scores scaled
 * by 1/sqrt(head_dim); query head h reads kv head h / (n_heads / n_kv_heads).
 * head_dim up to 512. */
int mlq_hip_attention_decode(int device, const float* q, const float* keys, const float* values, int n_layers,
                             int layer, int max_seq_len, int n_heads, int n_kv_heads, int head_dim, int pos,
                             float* out, void* stream);
/* C[m][n] = A[m][k] * B in f32 with B [k][n], or, with b_transposed != 0, B
 * stored as [n][k] (a linear's W: C = x W^T) (cuda_matmul, cuda_linear*). */
int mlq_hip_matmul_f32(int device, const float* a, const float* b, int m, int k, int n, int b_transposed, float* c,
                       void* stream);

/* Kernel selection introspection: name of the kernel the next call with this
 * shape would launch (for profiles and tests). */
int mlq_hip_kernel_name(int qtype, int rows, int out_features, int in_features, char* buf,
                        size_t len);

/* ---- GGUF ingest: quantized linear weights straight from a model file ----
 * The file is memory-mapped read-only and indexed once; a weight's raw block
 * bytes go from the mapping to device memory without an intermediate host
 * copy of the tensor (the reference reads each tensor into a std::vector,
 * read_gguf_tensor_raw, src/gguf.cpp:586-622, copies it into a
 * QuantizedTensor, load_quantized_tensor, src/gguf_loader.cpp:110-184, and
 * then uploads, src/model.cpp:145-272).  Block layouts are ggml's, so real
 * llama.cpp files load unchanged. */
typedef struct mlq_gguf_s* mlq_gguf_t;

/* Map and parse `path` (GGUFReader::load, src/gguf.cpp:371-530): version 3
 * only, the reader's limits, data section aligned to general.alignment
 * (default 32).  On failure the message is the reader's load_error. */
int mlq_hip_gguf_open(const char* path, mlq_gguf_t* out);
int mlq_hip_gguf_close(mlq_gguf_t g);
/* GGUFReader's version, n_tensors, n_metadata and data_offset (any may be NULL). */
int mlq_hip_gguf_header(mlq_gguf_t g, uint32_t* version, uint64_t* n_tensors, uint64_t* n_metadata,
                        uint64_t* data_offset);
/* Metadata entry i: key, GGUF value type and value rendered as
 * GGUFMetadataKV::value_str (include/mini_llama/gguf.h:55-59).  Buffers too
 * small give MLQ_ERR_LIMIT; NULL buffers are skipped. */
int mlq_hip_gguf_metadata(mlq_gguf_t g, uint64_t i, char* key, size_t key_cap, uint32_t* type, char* value,
                          size_t value_cap);
/* Tensor i (GGUFTensorInfo, include/mini_llama/gguf.h:46-51): name, dims
 * (ne0 first, 8 slots, unused ones 0), GGML type, offset in the data section
 * and data bytes (gguf_tensor_data_size; 0 for types without a known size). */
int mlq_hip_gguf_tensor(mlq_gguf_t g, uint64_t i, char* name, size_t name_cap, uint32_t* n_dims, uint64_t* dims,
                        uint32_t* ggml_type, uint64_t* offset, uint64_t* nbytes);
/* Index of the tensor named `name` ("Missing tensor: NAME" otherwise). */
int mlq_hip_gguf_find(mlq_gguf_t g, const char* name, uint64_t* index);
/* Host pointer to tensor i's bytes inside the mapping (valid until close). */
int mlq_hip_gguf_tensor_data(mlq_gguf_t g, uint64_t i, const void** data, uint64_t* nbytes);
/* Upload the 2-D Q8_0 / Q4_0 / Q4_1 tensor `name` ([ne0 = in, ne1 = out])
 * to `device` as a weight handle owning its memory, byte for byte.
 * Validation messages follow the upload's (src/model.cpp:145-272). */
int mlq_hip_gguf_upload_weight(mlq_gguf_t g, const char* name, int device, mlq_weight_t* out);

/* ---- Device-resident decode (forward_token with every op on the device) ----
 * A llama / qwen2 model loaded from a GGUF file as load_gguf_model loads it
 * (src/gguf_loader.cpp:320-456: config from metadata, tensor names, F32 norms,
 * embedding and biases, dequantized where stored quantized, tied lm_head),
 * its quantized linears on the GEMV kernels and the ops between them
 * (RMSNorm, RoPE, KV cache, attention, SwiGLU, residuals) as HIP kernels.
 * The position and input token of a step live in device memory, so greedy
 * generation replays one recorded step per token with the pick of one step
 * feeding the next: one upload and one download per call, none per token. */
typedef struct mlq_decoder_s* mlq_decoder_t;

/* ModelConfig (include/mini_llama/model.h:17-29); rope_neox = 1 for qwen2. */
typedef struct mlq_decoder_config {
    int n_layers, dim, hidden_dim, n_heads, n_kv_heads, head_dim, vocab_size, max_seq_len;
    float rope_theta, rms_norm_eps;
    int rope_neox;
} mlq_decoder_config;

/* Load `gguf_path` onto `device`.  max_seq_len > 0 caps the KV cache below
 * the model's context length.  Messages as the loader's ("GGUF parse error:
 * ...", "Failed to build config: ...", "Failed to load GGUF weights: Missing
 * tensor: layers.0.wq", ...). */
int mlq_hip_decoder_open(const char* gguf_path, int device, int max_seq_len, mlq_decoder_t* out);
int mlq_hip_decoder_config(mlq_decoder_t d, mlq_decoder_config* out);
/* forward_token (src/forward.cpp:865-903) with ctx.pos = pos: logits
 * [vocab_size] to host memory.  Positions below pos hold what earlier calls
 * wrote (zeros otherwise), as the reference's KV cache. */
int mlq_hip_decoder_forward(mlq_decoder_t d, int token, int pos, float* logits);
/* forward_batch (src/batch.cpp:33-52) over n tokens at positions
 * start_pos..start_pos+n-1, batched: every layer runs on all rows at once,
 * the linears as MFMA GEMMs (the reference runs the tokens one by one).
 * Logits of the last token to host memory when `logits` is not NULL. */
int mlq_hip_decoder_prefill(mlq_decoder_t d, const int* tokens, int n, int start_pos, float* logits);
/* Greedy generation: the prompt at positions 0..n_prompt-1 (forward_batch,
 * src/batch.cpp:33-52; batched as mlq_hip_decoder_prefill), then n_new
 * tokens, each the first maximum of the previous step's logits
 * (MiniSampler::sample_greedy), into out_tokens.
 * Fails with "sampler: logits must be finite" as the sampler does. */
int mlq_hip_decoder_generate(mlq_decoder_t d, const int* prompt, int n_prompt, int n_new, int* out_tokens);
int mlq_hip_decoder_close(mlq_decoder_t d);

#ifdef __cplusplus
}
#endif

#endif /* MLQ_HIP_H */

// C-ABI of the MI355X quantized-linear path (declared in include/mlq_hip.h).
//
// Validation order and messages mirror the reference's CUDA wrappers
// (src/cuda_quant.cu:150-243 shape checks, :253-255 null weight, :299-301
// device mismatch) and weight upload (src/model.cpp:145-272), with "cuda"
// replaced by "hip".  Every check runs on the host before any launch, so a
// malformed call never reaches a kernel.

#include "decoder.h"
#include "gguf_index.h"
#include "mlq_kernels.h"

#include "../../include/mlq_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <condition_variable>
#include <cstdio>
#include <cmath>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include <unistd.h>

struct mlq_weight_s {
    int device;
    int qtype;
    int M;
    int K;
    int nb;
    size_t n_blocks;
    void* ptr;
    bool owned;
};

struct mlq_gguf_s {
    mlq::GgufIndex index;
};

struct mlq_decoder_s {
    std::unique_ptr<mlq::Decoder> dec;
};

struct mlq_graph_s {
    hipGraph_t graph;
    hipGraphExec_t exec;
    int device;
};

// A validated chain of GEMVs: stage descriptors and barrier words in device
// memory, split into launches (segments) of one kernel variant each.
struct mlq_sequence_s {
    struct Segment {
        int qtype;
        int lpr;
        int stage_begin;
        int nstages;
        int lds_bytes;
        int grid;
        int kmax;  // largest in_features of the segment (pipelined mode)
    };
    int device;
    int mode;
    int nstages;
    unsigned spin_limit;
    std::vector<Segment> segs;
    // Per-stage mode: one grouped GEMV launch per stage.
    struct HostStage {
        mlq::LinearShape shape;  // M = rows of all calls of the stage
        mlq::GemvGroup group;
        const float* x;
    };
    std::vector<HostStage> host_stages;
    void* mem;               // [stage descriptors][SeqSync per segment]
    size_t sync_offset;      // byte offset of the first SeqSync
    size_t sink_offset;      // pipelined mode: byte offset of the chain kernel's sink words
};

namespace {

thread_local std::string g_error;

int fail(int code, const std::string& msg) {
    g_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(MLQ_ERR_HIP, std::string("HIP error in ") + what + ": " + hipGetErrorString(e));
}

#define MLQ_HIP_CHECK(expr)                                   \
    do {                                                      \
        hipError_t mlq_e_ = (expr);                           \
        if (mlq_e_ != hipSuccess) return hip_fail(mlq_e_, #expr); \
    } while (0)

constexpr int kMaxDevices = 64;

// GEMM workspace, one per stream that ran a batched call (grow-only, kept
// until the process ends).
struct Workspace {
    hipStream_t stream;
    void* ptr;
    size_t bytes;
};

// Greedy-pick state of one stream (created on the stream's first pick call,
// kept until the process ends): the fold words, zero between launches, and
// the token word the synchronous entry reads back.
struct PickSlot {
    hipStream_t stream;
    mlq::PickState* state;
    int32_t* token;
};

// Device memory of the no-allocation entry point (mlq_hip_quant_linear_noalloc):
// the batched GEMM's workspace (split-K arrival counters, partial tiles, split
// x) for callers that cannot allocate.  Each GPU the library runs on holds its
// own copy until the process ends; host code uses the per-device address from
// hipGetSymbolAddress (DeviceState::scratch), never the array's name.
constexpr size_t kScratchBytes = size_t(48) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct DeviceState {
    std::once_flag once;
    hipError_t init_err = hipSuccess;
    hipStream_t stream = nullptr;
    void* scratch = nullptr;   // this device's address of `scratch` (zeroed at set-up)
    std::mutex mu;             // guards the host-pointer staging buffers
    void* stage = nullptr;     // x and y staging for host-pointer calls
    size_t stage_bytes = 0;
    std::mutex ws_mu;          // guards the GEMM workspaces and the pick states
    std::vector<Workspace> ws;
    // Workspaces replaced by a larger one.  A graph recorded before the growth
    // still holds the old buffer's address (split-K counters, partials, split
    // x), so a retired buffer is kept until the process ends.
    std::vector<void*> retired_ws;
    std::vector<PickSlot> picks;
    std::mutex pin_mu;         // guards the pinned stage of file uploads
    void* pin[2] = {nullptr, nullptr};
    hipEvent_t pin_done[2] = {nullptr, nullptr};
};

DeviceState g_dev[kMaxDevices];

const char* caller_for(int qtype) {
    switch (qtype) {
        case MLQ_Q8_0: return "hip_q8_0_linear";
        case MLQ_Q4_0: return "hip_q4_0_linear";
        case MLQ_Q4_1: return "hip_q4_1_linear";
        default: return "hip_quant_linear";
    }
}

const char* type_name(int qtype) {
    switch (qtype) {
        case MLQ_Q8_0: return "Q8_0";
        case MLQ_Q4_0: return "Q4_0";
        case MLQ_Q4_1: return "Q4_1";
        default: return "F32";
    }
}

int ensure_device(int device) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if (device < 0 || device >= count || device >= kMaxDevices) {
        return fail(MLQ_ERR_DEVICE, "HIP device " + std::to_string(device) + " is not available (" +
                                        std::to_string(count) + " visible)");
    }
    DeviceState& st = g_dev[device];
    std::call_once(st.once, [&] {
        st.init_err = hipSetDevice(device);
        if (st.init_err == hipSuccess) {
            // Default priority, non-blocking with respect to the null stream.
            st.init_err = hipStreamCreateWithFlags(&st.stream, hipStreamNonBlocking);
        }
        if (st.init_err == hipSuccess) {
            // This device's copy of the no-allocation scratch: its address,
            // then its split-K counters (and the rest) cleared once; every
            // GEMM launch leaves the counters at zero again.
            st.init_err = hipGetSymbolAddress(&st.scratch, HIP_SYMBOL(scratch));
        }
        if (st.init_err == hipSuccess) st.init_err = hipMemsetAsync(st.scratch, 0, kScratchBytes, st.stream);
        if (st.init_err == hipSuccess) st.init_err = hipStreamSynchronize(st.stream);
    });
    if (st.init_err != hipSuccess) return hip_fail(st.init_err, "device init");
    e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    return MLQ_OK;
}

hipStream_t resolve_stream(int device, void* stream) {
    return stream != nullptr ? static_cast<hipStream_t>(stream) : g_dev[device].stream;
}

// Checks that [p, p + bytes) lies inside one device allocation on `device`
// (device or managed memory).  A host pointer handed over as a device pointer,
// or a buffer shorter than the shape implies, would make a kernel fault, so
// every entry point that takes caller pointers runs this before launching.
int check_device_ptr(const void* p, int device, const char* caller, const char* what,
                     size_t bytes) {
    if (p == nullptr) return fail(MLQ_ERR_INVALID, std::string(caller) + ": " + what + " pointer is null");
    hipPointerAttribute_t attr;
    std::memset(&attr, 0, sizeof attr);
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();  // clear the sticky error of a failed lookup
        return fail(MLQ_ERR_DEVICE, std::string(caller) + ": " + what + " is not a HIP device pointer");
    }
    if (attr.type != hipMemoryTypeDevice && attr.type != hipMemoryTypeManaged) {
        return fail(MLQ_ERR_DEVICE, std::string(caller) + ": " + what + " is not a HIP device pointer");
    }
    if (attr.device != device) {
        return fail(MLQ_ERR_DEVICE, std::string(caller) + ": " + what +
                                        " tensor is on a different HIP device");
    }
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    e = hipMemGetAddressRange(&base, &size, const_cast<void*>(p));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(MLQ_ERR_DEVICE, std::string(caller) + ": " + what + " allocation extent is unknown");
    }
    const uintptr_t start = reinterpret_cast<uintptr_t>(p);
    const uintptr_t end = reinterpret_cast<uintptr_t>(base) + size;
    if (start + bytes > end) {
        return fail(MLQ_ERR_LIMIT, std::string(caller) + ": " + what + " buffer is too small: needs " +
                                       std::to_string(bytes) + " bytes, the allocation holds " +
                                       std::to_string(end - start) + " from this pointer");
    }
    return MLQ_OK;
}

// src/cuda_quant.cu:214-243 for the device-weight linear.
int validate_linear(int qtype, int M, int K, size_t n_blocks, int rows) {
    const char* caller = caller_for(qtype);
    if (qtype != MLQ_Q8_0 && qtype != MLQ_Q4_0 && qtype != MLQ_Q4_1) {
        return fail(MLQ_ERR_INVALID, std::string(caller) + ": unsupported quant type " + std::to_string(qtype));
    }
    if (rows <= 0 || K <= 0 || M <= 0) {
        return fail(MLQ_ERR_SHAPE, std::string(caller) + ": empty tensors are not supported");
    }
    const int nb = (K + mlq::kQK - 1) / mlq::kQK;
    const size_t expected = static_cast<size_t>(M) * nb;
    if (n_blocks != expected) {
        return fail(MLQ_ERR_SHAPE, std::string(caller) + ": block count mismatch: expected " +
                                       std::to_string(expected) + ", got " + std::to_string(n_blocks));
    }
    // Indices inside the kernels are 32-bit for rows and dwords per row.
    if (static_cast<long long>(nb) * mlq::block_bytes(qtype) >= (1ll << 31) || rows > 65535) {
        return fail(MLQ_ERR_LIMIT, std::string(caller) + ": shape exceeds the kernel limits");
    }
    return MLQ_OK;
}

// Ends the capture on `s` and instantiates what it recorded; a failed launch
// inside the capture (launch_rc) discards the graph.
int end_capture(hipStream_t s, int device, int launch_rc, mlq_graph_t* out) {
    hipGraph_t graph = nullptr;
    hipError_t end_err = hipStreamEndCapture(s, &graph);
    if (launch_rc != MLQ_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return launch_rc;
    }
    if (end_err != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        return hip_fail(end_err, "hipStreamEndCapture");
    }
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return hip_fail(e, "hipGraphInstantiate");
    }
    *out = new mlq_graph_s{graph, exec, device};
    return MLQ_OK;
}

bool capturing(hipStream_t s) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// Returns a workspace of at least `bytes` for `stream` on `device`.  Growing
// allocates a new buffer and retires the old one without freeing it: graphs
// recorded on the stream keep using the buffer they were recorded with.
int stream_workspace(int device, hipStream_t stream, size_t bytes, void** out) {
    DeviceState& st = g_dev[device];
    std::lock_guard<std::mutex> lock(st.ws_mu);
    for (Workspace& w : st.ws) {
        if (w.stream != stream) continue;
        if (w.bytes < bytes) {
            if (capturing(stream)) {
                return fail(MLQ_ERR_INVALID, "the stream's batched-call workspace must grow, which cannot happen "
                                             "under graph capture: make the largest batched call once first");
            }
            void* p = nullptr;
            MLQ_HIP_CHECK(hipMalloc(&p, bytes));
            // The split-K arrival counters start at zero; every launch leaves
            // them so.  Cleared on the workspace's own stream, ahead of its kernels.
            MLQ_HIP_CHECK(hipMemsetAsync(p, 0, bytes, stream));
            st.retired_ws.push_back(w.ptr);
            w.ptr = p;
            w.bytes = bytes;
        }
        *out = w.ptr;
        return MLQ_OK;
    }
    if (capturing(stream)) {
        return fail(MLQ_ERR_INVALID, "the stream's batched-call workspace is created by a first call outside "
                                     "graph capture");
    }
    void* p = nullptr;
    MLQ_HIP_CHECK(hipMalloc(&p, bytes));
    MLQ_HIP_CHECK(hipMemsetAsync(p, 0, bytes, stream));
    st.ws.push_back(Workspace{stream, p, bytes});
    *out = p;
    return MLQ_OK;
}

int stream_pick(int device, hipStream_t stream, const char* caller, PickSlot* out) {
    DeviceState& st = g_dev[device];
    std::lock_guard<std::mutex> lock(st.ws_mu);
    for (const PickSlot& p : st.picks) {
        if (p.stream == stream) {
            *out = p;
            return MLQ_OK;
        }
    }
    if (capturing(stream)) {
        return fail(MLQ_ERR_INVALID, std::string(caller) +
                                         ": the stream's pick state is created by a first call outside graph capture");
    }
    void* mem = nullptr;
    const size_t bytes = sizeof(mlq::PickState) + 128;
    MLQ_HIP_CHECK(hipMalloc(&mem, bytes));
    MLQ_HIP_CHECK(hipMemsetAsync(mem, 0, bytes, stream));
    PickSlot p{stream, static_cast<mlq::PickState*>(mem),
               reinterpret_cast<int32_t*>(static_cast<char*>(mem) + sizeof(mlq::PickState))};
    st.picks.push_back(p);
    *out = p;
    return MLQ_OK;
}

int dispatch(int device, const mlq::LinearShape& s, const void* w, const float* x, float* y,
             hipStream_t stream) {
    hipError_t e;
    if (s.rows > 1 && mlq::gemm_supported(s)) {
        const size_t need = mlq::gemm_workspace_bytes(s);
        void* ws = nullptr;
        int rc = stream_workspace(device, stream, need, &ws);
        if (rc != MLQ_OK) return rc;
        e = mlq::launch_gemm(s, w, x, y, ws, need, stream);
    } else {
        e = mlq::launch_gemv(s, w, x, y, stream);
    }
    if (e != hipSuccess) return hip_fail(e, caller_for(s.qtype));
    return MLQ_OK;
}

int grow_stage(DeviceState& st, size_t bytes) {
    if (st.stage_bytes >= bytes) return MLQ_OK;
    if (st.stage != nullptr) {
        MLQ_HIP_CHECK(hipStreamSynchronize(st.stream));
        MLQ_HIP_CHECK(hipFree(st.stage));
        st.stage = nullptr;
        st.stage_bytes = 0;
    }
    size_t cap = 1 << 20;
    while (cap < bytes) cap <<= 1;
    MLQ_HIP_CHECK(hipMalloc(&st.stage, cap));
    st.stage_bytes = cap;
    return MLQ_OK;
}

}  // namespace

extern "C" {

const char* mlq_hip_last_error(void) { return g_error.c_str(); }

int mlq_hip_built(void) { return 1; }

int mlq_hip_device_count(int* count) {
    if (count == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_device_count: null output");
    *count = 0;
    hipError_t e = hipGetDeviceCount(count);
    if (e == hipErrorNoDevice) {
        *count = 0;
        (void)hipGetLastError();
        return MLQ_OK;
    }
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    return MLQ_OK;
}

int mlq_hip_device_info(int device, char* buf, size_t len) {
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    hipDeviceProp_t p;
    MLQ_HIP_CHECK(hipGetDeviceProperties(&p, device));
    if (buf != nullptr && len > 0) {
        std::snprintf(buf, len, "HIP device %d: %s (%s), %d CUs, %.1f GiB HBM, LDS %zu KiB/CU",
                      device, p.name, p.gcnArchName, p.multiProcessorCount,
                      static_cast<double>(p.totalGlobalMem) / (1024.0 * 1024.0 * 1024.0),
                      static_cast<size_t>(p.maxSharedMemoryPerMultiProcessor) / 1024);
    }
    return MLQ_OK;
}

int mlq_hip_device_props(int device, mlq_device_props* out) {
    if (out == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_device_props: null output");
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    hipDeviceProp_t p;
    MLQ_HIP_CHECK(hipGetDeviceProperties(&p, device));
    std::memset(out, 0, sizeof *out);
    std::snprintf(out->name, sizeof out->name, "%s", p.name[0] != 0 ? p.name : p.gcnArchName);
    std::snprintf(out->arch, sizeof out->arch, "%s", p.gcnArchName);
    out->major = p.major;
    out->minor = p.minor;
    out->total_memory_bytes = p.totalGlobalMem;
    out->compute_units = p.multiProcessorCount;
    MLQ_HIP_CHECK(hipDriverGetVersion(&out->driver_version));
    MLQ_HIP_CHECK(hipRuntimeGetVersion(&out->runtime_version));
    return MLQ_OK;
}

int mlq_hip_init(int device) { return ensure_device(device); }

int mlq_hip_upload_weight(int device, int qtype, const void* host_blocks, size_t n_blocks,
                          int out_features, int in_features, mlq_weight_t* out) {
    if (out == nullptr) return fail(MLQ_ERR_INVALID, "HIP weight upload: null output handle");
    *out = nullptr;
    if (qtype != MLQ_Q8_0 && qtype != MLQ_Q4_0 && qtype != MLQ_Q4_1) {
        return fail(MLQ_ERR_INVALID, "HIP weight upload: unsupported quant type " + std::to_string(qtype));
    }
    if (out_features <= 0 || in_features <= 0) {
        return fail(MLQ_ERR_SHAPE, std::string("HIP weight upload: expected 2D ") + type_name(qtype) + " weight");
    }
    if (host_blocks == nullptr || n_blocks == 0) {
        return fail(MLQ_ERR_SHAPE, std::string("HIP weight upload: empty ") + type_name(qtype) + " data");
    }
    const int nb = (in_features + mlq::kQK - 1) / mlq::kQK;
    const size_t expected = static_cast<size_t>(out_features) * nb;
    if (n_blocks != expected) {
        return fail(MLQ_ERR_SHAPE, std::string("HIP weight upload: ") + type_name(qtype) +
                                       " block count mismatch, expected " + std::to_string(expected) +
                                       ", got " + std::to_string(n_blocks));
    }
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    const size_t bytes = n_blocks * static_cast<size_t>(mlq::block_bytes(qtype));
    void* ptr = nullptr;
    MLQ_HIP_CHECK(hipMalloc(&ptr, bytes));
    hipError_t e = hipMemcpy(ptr, host_blocks, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(ptr);
        return hip_fail(e, "hipMemcpy(weight)");
    }
    *out = new mlq_weight_s{device, qtype, out_features, in_features, nb, n_blocks, ptr, true};
    return MLQ_OK;
}

int mlq_hip_wrap_weight(int device, int qtype, const void* device_blocks, size_t n_blocks,
                        int out_features, int in_features, mlq_weight_t* out) {
    if (out == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_wrap_weight: null output handle");
    *out = nullptr;
    const char* caller = caller_for(qtype);
    if (device_blocks == nullptr) {
        return fail(MLQ_ERR_INVALID, std::string(caller) + ": device weight pointer is null");
    }
    int rc = validate_linear(qtype, out_features, in_features, n_blocks, 1);
    if (rc != MLQ_OK) return rc;
    rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    rc = check_device_ptr(device_blocks, device, caller, "device weight",
                          n_blocks * static_cast<size_t>(mlq::block_bytes(qtype)));
    if (rc != MLQ_OK) return rc;
    const int nb = (in_features + mlq::kQK - 1) / mlq::kQK;
    *out = new mlq_weight_s{device, qtype, out_features, in_features, nb, n_blocks,
                            const_cast<void*>(device_blocks), false};
    return MLQ_OK;
}

int mlq_hip_free_weight(mlq_weight_t w) {
    if (w == nullptr) return MLQ_OK;
    if (w->owned && w->ptr != nullptr) {
        (void)hipSetDevice(w->device);
        hipError_t e = hipFree(w->ptr);
        delete w;
        if (e != hipSuccess) return hip_fail(e, "hipFree(weight)");
        return MLQ_OK;
    }
    delete w;
    return MLQ_OK;
}

int mlq_hip_weight_info(mlq_weight_t w, int* qtype, int* out_features, int* in_features,
                        size_t* n_blocks, const void** device_blocks, int* device) {
    if (w == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_weight_info: null handle");
    if (qtype) *qtype = w->qtype;
    if (out_features) *out_features = w->M;
    if (in_features) *in_features = w->K;
    if (n_blocks) *n_blocks = w->n_blocks;
    if (device_blocks) *device_blocks = w->ptr;
    if (device) *device = w->device;
    return MLQ_OK;
}

int mlq_hip_quant_linear_device(int device, int qtype, const void* device_blocks, size_t n_blocks,
                                int out_features, int in_features, const float* x, int rows,
                                float* y, void* stream) {
    const char* caller = caller_for(qtype);
    if (device_blocks == nullptr) {
        return fail(MLQ_ERR_INVALID, std::string(caller) + ": device weight pointer is null");
    }
    int rc = validate_linear(qtype, out_features, in_features, n_blocks, rows);
    if (rc != MLQ_OK) return rc;
    rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    const size_t wbytes = n_blocks * static_cast<size_t>(mlq::block_bytes(qtype));
    const size_t xbytes = static_cast<size_t>(rows) * in_features * sizeof(float);
    const size_t ybytes = static_cast<size_t>(rows) * out_features * sizeof(float);
    if ((rc = check_device_ptr(device_blocks, device, caller, "device weight", wbytes)) != MLQ_OK) return rc;
    if ((rc = check_device_ptr(x, device, caller, "input", xbytes)) != MLQ_OK) return rc;
    if ((rc = check_device_ptr(y, device, caller, "output", ybytes)) != MLQ_OK) return rc;
    mlq::LinearShape s{qtype, out_features, in_features, (in_features + 31) / 32, rows};
    return dispatch(device, s, device_blocks, x, y, resolve_stream(device, stream));
}

int mlq_hip_quant_linear_noalloc(mlq_weight_t w, const float* x, int rows, float* y, void* stream) {
    if (w == nullptr) return fail(MLQ_ERR_INVALID, "hip_quant_linear: null weight handle");
    const char* caller = caller_for(w->qtype);
    int rc = validate_linear(w->qtype, w->M, w->K, w->n_blocks, rows);
    if (rc != MLQ_OK) return rc;
    rc = ensure_device(w->device);
    if (rc != MLQ_OK) return rc;
    const size_t xb = static_cast<size_t>(rows) * w->K * sizeof(float);
    const size_t yb = static_cast<size_t>(rows) * w->M * sizeof(float);
    if ((rc = check_device_ptr(x, w->device, caller, "input", xb)) != MLQ_OK) return rc;
    if ((rc = check_device_ptr(y, w->device, caller, "output", yb)) != MLQ_OK) return rc;
    mlq::LinearShape s{w->qtype, w->M, w->K, w->nb, rows};
    const hipStream_t st = resolve_stream(w->device, stream);
    hipError_t e;
    if (rows > 1 && mlq::gemm_supported(s)) {
        const size_t need = mlq::gemm_workspace_bytes(s);
        if (need > kScratchBytes) {
            return fail(MLQ_ERR_LIMIT, std::string(caller) + ": the no-allocation entry point has " +
                                           std::to_string(kScratchBytes) + " bytes of scratch; " +
                                           std::to_string(rows) + " rows of this weight need " +
                                           std::to_string(need) + " (use mlq_hip_quant_linear)");
        }
        e = mlq::launch_gemm(s, w->ptr, x, y, g_dev[w->device].scratch, need, st);
    } else {
        e = mlq::launch_gemv(s, w->ptr, x, y, st);  // no scratch
    }
    if (e != hipSuccess) return hip_fail(e, caller);
    return MLQ_OK;
}

int mlq_hip_quant_linear(mlq_weight_t w, const float* x, int rows, float* y, int flags,
                         void* stream) {
    if (w == nullptr) return fail(MLQ_ERR_INVALID, "hip_quant_linear: null weight handle");
    const char* caller = caller_for(w->qtype);
    if (flags & ~(MLQ_X_ON_DEVICE | MLQ_Y_ON_DEVICE | MLQ_ASYNC)) {
        return fail(MLQ_ERR_INVALID, std::string(caller) + ": unknown flags");
    }
    if (x == nullptr) return fail(MLQ_ERR_INVALID, std::string(caller) + ": input pointer is null");
    if (y == nullptr) return fail(MLQ_ERR_INVALID, std::string(caller) + ": output pointer is null");
    int rc = validate_linear(w->qtype, w->M, w->K, w->n_blocks, rows);
    if (rc != MLQ_OK) return rc;
    rc = ensure_device(w->device);
    if (rc != MLQ_OK) return rc;
    DeviceState& st = g_dev[w->device];
    hipStream_t s = resolve_stream(w->device, stream);
    mlq::LinearShape shape{w->qtype, w->M, w->K, w->nb, rows};
    const size_t xb = static_cast<size_t>(rows) * w->K * sizeof(float);
    const size_t yb = static_cast<size_t>(rows) * w->M * sizeof(float);

    const bool xd = flags & MLQ_X_ON_DEVICE;
    const bool yd = flags & MLQ_Y_ON_DEVICE;
    if (xd && (rc = check_device_ptr(x, w->device, caller, "input", xb)) != MLQ_OK) return rc;
    if (yd && (rc = check_device_ptr(y, w->device, caller, "output", yb)) != MLQ_OK) return rc;
    if (xd && yd) {
        if ((rc = dispatch(w->device, shape, w->ptr, x, y, s)) != MLQ_OK) return rc;
        if (!(flags & MLQ_ASYNC)) MLQ_HIP_CHECK(hipStreamSynchronize(s));
        return MLQ_OK;
    }
    // Host x and/or y: stage through the device's buffer (x first, 256-B aligned y).
    std::lock_guard<std::mutex> lock(st.mu);
    const size_t xoff = 0;
    const size_t yoff = (xb + 255) & ~static_cast<size_t>(255);
    if ((rc = grow_stage(st, yoff + yb)) != MLQ_OK) return rc;
    char* base = static_cast<char*>(st.stage);
    const float* xdev = x;
    float* ydev = y;
    if (!xd) {
        MLQ_HIP_CHECK(hipMemcpyAsync(base + xoff, x, xb, hipMemcpyHostToDevice, s));
        xdev = reinterpret_cast<const float*>(base + xoff);
    }
    if (!yd) ydev = reinterpret_cast<float*>(base + yoff);
    if ((rc = dispatch(w->device, shape, w->ptr, xdev, ydev, s)) != MLQ_OK) return rc;
    if (!yd) MLQ_HIP_CHECK(hipMemcpyAsync(y, ydev, yb, hipMemcpyDeviceToHost, s));
    MLQ_HIP_CHECK(hipStreamSynchronize(s));
    return MLQ_OK;
}

int mlq_hip_quant_linear_many(const mlq_linear_call* calls, int n, void* stream) {
    if (calls == nullptr || n <= 0) return fail(MLQ_ERR_INVALID, "mlq_hip_quant_linear_many: no calls");
    const int device = calls[0].w != nullptr ? calls[0].w->device : -1;
    for (int i = 0; i < n; ++i) {
        const mlq_linear_call& c = calls[i];
        if (c.w == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_quant_linear_many: null weight handle");
        if (c.w->device != device) {
            return fail(MLQ_ERR_DEVICE, "mlq_hip_quant_linear_many: weights on different devices");
        }
        int rc = validate_linear(c.w->qtype, c.w->M, c.w->K, c.w->n_blocks, c.rows);
        if (rc != MLQ_OK) return rc;
    }
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    for (int i = 0; i < n; ++i) {
        const char* caller = caller_for(calls[i].w->qtype);
        const mlq_weight_s* w = calls[i].w;
        const size_t xb = static_cast<size_t>(calls[i].rows) * w->K * sizeof(float);
        const size_t yb = static_cast<size_t>(calls[i].rows) * w->M * sizeof(float);
        if ((rc = check_device_ptr(calls[i].x, device, caller, "input", xb)) != MLQ_OK) return rc;
        if ((rc = check_device_ptr(calls[i].y, device, caller, "output", yb)) != MLQ_OK) return rc;
    }
    hipStream_t s = resolve_stream(device, stream);
    for (int i = 0; i < n; ++i) {
        const mlq_linear_call& c = calls[i];
        mlq::LinearShape shape{c.w->qtype, c.w->M, c.w->K, c.w->nb, c.rows};
        if ((rc = dispatch(device, shape, c.w->ptr, c.x, c.y, s)) != MLQ_OK) return rc;
    }
    return MLQ_OK;
}

namespace {

// Validates a fused call list (same x, rows, in_features and quant type;
// outputs disjoint from x and from each other) into its GEMV group.
int fused_group(const mlq_linear_call* calls, int n, const char* caller, mlq::GemvGroup& g, long long& rows,
                int& device) {
    if (calls == nullptr || n <= 0) return fail(MLQ_ERR_INVALID, std::string(caller) + ": no calls");
    if (n > mlq::kGroupMaxCalls) {
        return fail(MLQ_ERR_LIMIT, std::string(caller) + ": " + std::to_string(n) + " calls (at most " +
                                       std::to_string(mlq::kGroupMaxCalls) + ")");
    }
    if (calls[0].w == nullptr) return fail(MLQ_ERR_INVALID, std::string(caller) + ": null weight handle");
    const mlq_weight_s* w0 = calls[0].w;
    device = w0->device;
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    g = mlq::GemvGroup{};
    rows = 0;
    const int nrows = calls[0].rows;
    for (int i = 0; i < n; ++i) {
        const mlq_linear_call& c = calls[i];
        const std::string at = std::string(caller) + ": call " + std::to_string(i);
        if (c.w == nullptr) return fail(MLQ_ERR_INVALID, at + ": null weight handle");
        if (c.w->device != device) return fail(MLQ_ERR_DEVICE, at + ": weight on a different device");
        if (c.x != calls[0].x || c.w->K != w0->K || c.w->qtype != w0->qtype || c.rows != nrows) {
            return fail(MLQ_ERR_INVALID, at + ": differs from call 0 in input, rows, in_features or quant type");
        }
        if ((rc = validate_linear(c.w->qtype, c.w->M, c.w->K, c.w->n_blocks, c.rows)) != MLQ_OK) return rc;
        const char* lin = caller_for(c.w->qtype);
        const size_t xb = static_cast<size_t>(c.rows) * c.w->K * sizeof(float);
        const size_t yb = static_cast<size_t>(c.rows) * c.w->M * sizeof(float);
        if ((rc = check_device_ptr(c.x, device, lin, "input", xb)) != MLQ_OK) return rc;
        if ((rc = check_device_ptr(c.y, device, lin, "output", yb)) != MLQ_OK) return rc;
        const uintptr_t ylo = reinterpret_cast<uintptr_t>(c.y), yhi = ylo + yb;
        const uintptr_t xlo = reinterpret_cast<uintptr_t>(c.x), xhi = xlo + xb;
        if (ylo < xhi && xlo < yhi) return fail(MLQ_ERR_INVALID, at + ": output overlaps the input");
        for (int j = 0; j < i; ++j) {
            const uintptr_t olo = reinterpret_cast<uintptr_t>(calls[j].y);
            const uintptr_t ohi = olo + static_cast<size_t>(nrows) * calls[j].w->M * sizeof(float);
            if (ylo < ohi && olo < yhi) {
                return fail(MLQ_ERR_INVALID, at + ": output overlaps the output of call " + std::to_string(j));
            }
        }
        g.W[i] = c.w->ptr;
        g.y[i] = c.y;
        g.row_begin[i] = static_cast<int>(rows);
        rows += c.w->M;
    }
    if (rows > (1ll << 30)) return fail(MLQ_ERR_LIMIT, std::string(caller) + ": too many rows");
    g.ncalls = n;
    return MLQ_OK;
}

}  // namespace

int mlq_hip_quant_linear_fused_f32(const mlq_linear_call* calls, int n, void* stream) {
    static const char* caller = "mlq_hip_quant_linear_fused_f32";
    mlq::GemvGroup g;
    long long rows = 0;
    int device = 0;
    int rc = fused_group(calls, n, caller, g, rows, device);
    if (rc != MLQ_OK) return rc;
    const mlq_weight_s* w0 = calls[0].w;
    if (calls[0].rows != 1) return fail(MLQ_ERR_INVALID, std::string(caller) + ": one token row only");
    if (w0->nb % 2 != 0) return fail(MLQ_ERR_INVALID, std::string(caller) + ": needs an even block count");
    mlq::LinearShape shape{w0->qtype, static_cast<int>(rows), w0->K, w0->nb, 1};
    const hipError_t e = mlq::launch_gemv_f32(shape, g, static_cast<const float*>(calls[0].x),
                                              resolve_stream(device, stream));
    if (e != hipSuccess) return hip_fail(e, caller);
    return MLQ_OK;
}

int mlq_hip_quant_linear_fused(const mlq_linear_call* calls, int n, void* stream) {
    static const char* caller = "mlq_hip_quant_linear_fused";
    mlq::GemvGroup g;
    long long rows = 0;
    int device = 0;
    int rc = fused_group(calls, n, caller, g, rows, device);
    if (rc != MLQ_OK) return rc;
    const mlq_weight_s* w0 = calls[0].w;
    const int nrows = calls[0].rows;
    hipStream_t s = resolve_stream(device, stream);
    if (nrows > 1) {
        // Batched rows: one grouped GEMM launch where the shapes allow it (at
        // most three weights, each but the last a whole number of row tiles),
        // else one GEMM (or GEMV batch) per call.
        mlq::LinearShape total{w0->qtype, static_cast<int>(rows), w0->K, w0->nb, nrows};
        int M[3] = {0, 0, 0};
        for (int i = 0; i < n && i < 3; ++i) M[i] = calls[i].w->M;
        // The workspace is sized (and grown) only for a group that will launch.
        if (n <= 3 && mlq::gemm_supported(total) && mlq::gemm_group_supported(total, n, M, calls[0].x)) {
            const void* wd[3];
            float* yd[3];
            for (int i = 0; i < n; ++i) wd[i] = calls[i].w->ptr, yd[i] = calls[i].y;
            const size_t need = mlq::gemm_workspace_bytes(total);
            void* ws = nullptr;
            if ((rc = stream_workspace(device, s, need, &ws)) != MLQ_OK) return rc;
            const hipError_t e = mlq::launch_gemm_group(total, n, wd, yd, M, calls[0].x, ws, need, s);
            if (e != hipErrorNotSupported) {
                if (e != hipSuccess) return hip_fail(e, caller);
                return MLQ_OK;
            }
        }
        for (int i = 0; i < n; ++i) {
            const mlq_linear_call& c = calls[i];
            mlq::LinearShape shape{c.w->qtype, c.w->M, c.w->K, c.w->nb, c.rows};
            if ((rc = dispatch(device, shape, c.w->ptr, c.x, c.y, s)) != MLQ_OK) return rc;
        }
        return MLQ_OK;
    }
    g.ncalls = n;
    mlq::LinearShape shape{w0->qtype, static_cast<int>(rows), w0->K, w0->nb, 1};
    hipError_t e = mlq::launch_gemv_group(shape, g, calls[0].x, s);
    if (e != hipSuccess) return hip_fail(e, caller);
    return MLQ_OK;
}

namespace {

// The group of a measurement launch (mlq_hip_stream_floor / _probe): calls
// validated as for a fused launch, weights only.
int floor_group(const mlq_linear_call* calls, int n, void* sink, const char* caller, mlq::GemvGroup& g,
                mlq::LinearShape& shape, int& device) {
    if (calls == nullptr || n <= 0) return fail(MLQ_ERR_INVALID, std::string(caller) + ": no calls");
    if (n > mlq::kGroupMaxCalls) {
        return fail(MLQ_ERR_LIMIT, std::string(caller) + ": " + std::to_string(n) + " calls (at most " +
                                       std::to_string(mlq::kGroupMaxCalls) + ")");
    }
    if (calls[0].w == nullptr) return fail(MLQ_ERR_INVALID, std::string(caller) + ": null weight handle");
    const mlq_weight_s* w0 = calls[0].w;
    device = w0->device;
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    if ((rc = check_device_ptr(sink, device, caller, "sink", size_t(mlq::kFloorSinkWords) * 4)) != MLQ_OK) return rc;
    if (w0->nb % 2 != 0) return fail(MLQ_ERR_INVALID, std::string(caller) + ": needs an even block count");
    g = mlq::GemvGroup{};
    long long rows = 0;
    for (int i = 0; i < n; ++i) {
        const mlq_linear_call& c = calls[i];
        const std::string at = std::string(caller) + ": call " + std::to_string(i);
        if (c.w == nullptr) return fail(MLQ_ERR_INVALID, at + ": null weight handle");
        if (c.w->device != device) return fail(MLQ_ERR_DEVICE, at + ": weight on a different device");
        if (c.w->K != w0->K || c.w->qtype != w0->qtype) {
            return fail(MLQ_ERR_INVALID, at + ": differs from call 0 in in_features or quant type");
        }
        g.W[i] = c.w->ptr;
        g.row_begin[i] = static_cast<int>(rows);
        rows += c.w->M;
    }
    if (rows > (1ll << 30)) return fail(MLQ_ERR_LIMIT, std::string(caller) + ": too many rows");
    g.ncalls = n;
    shape = mlq::LinearShape{w0->qtype, static_cast<int>(rows), w0->K, w0->nb, 1};
    return MLQ_OK;
}

}  // namespace

int mlq_hip_stream_floor(const mlq_linear_call* calls, int n, void* sink, void* stream) {
    static const char* caller = "mlq_hip_stream_floor";
    mlq::GemvGroup g;
    mlq::LinearShape shape;
    int device = 0;
    const int rc = floor_group(calls, n, sink, caller, g, shape, device);
    if (rc != MLQ_OK) return rc;
    hipError_t e = mlq::launch_stream_floor(shape, g, static_cast<uint32_t*>(sink), resolve_stream(device, stream));
    if (e != hipSuccess) return hip_fail(e, caller);
    return MLQ_OK;
}

int mlq_hip_stream_probe(const mlq_linear_call* calls, int n, int mode, void* sink, void* stream) {
    static const char* caller = "mlq_hip_stream_probe";
    if (mode != MLQ_PROBE_EMPTY && mode != MLQ_PROBE_LOAD) {
        return fail(MLQ_ERR_INVALID, std::string(caller) + ": unknown mode " + std::to_string(mode));
    }
    mlq::GemvGroup g;
    mlq::LinearShape shape;
    int device = 0;
    const int rc = floor_group(calls, n, sink, caller, g, shape, device);
    if (rc != MLQ_OK) return rc;
    const int m = mode == MLQ_PROBE_EMPTY ? mlq::kProbeEmpty : mlq::kProbeLoad;
    hipError_t e = mlq::launch_stream_probe(shape, g, m, static_cast<uint32_t*>(sink), resolve_stream(device, stream));
    if (e != hipSuccess) return hip_fail(e, caller);
    return MLQ_OK;
}

namespace {

// Shared front of the two greedy-pick entries: validates, then launches the
// picking GEMV with the token going to `token` (or to the stream's own word
// when `token` is null).
int launch_pick(mlq_weight_t w, const float* x, float* y, int32_t* token, void* stream, PickSlot* slot,
                hipStream_t* used) {
    if (w == nullptr) return fail(MLQ_ERR_INVALID, "hip_quant_linear_argmax: null weight handle");
    const char* caller = caller_for(w->qtype);
    if (x == nullptr) return fail(MLQ_ERR_INVALID, std::string(caller) + ": input pointer is null");
    int rc = validate_linear(w->qtype, w->M, w->K, w->n_blocks, 1);
    if (rc != MLQ_OK) return rc;
    if ((rc = ensure_device(w->device)) != MLQ_OK) return rc;
    const size_t xb = static_cast<size_t>(w->K) * sizeof(float);
    const size_t yb = static_cast<size_t>(w->M) * sizeof(float);
    if ((rc = check_device_ptr(x, w->device, caller, "input", xb)) != MLQ_OK) return rc;
    if (y != nullptr && (rc = check_device_ptr(y, w->device, caller, "output", yb)) != MLQ_OK) return rc;
    if (token != nullptr && (rc = check_device_ptr(token, w->device, caller, "token", sizeof(int32_t))) != MLQ_OK) {
        return rc;
    }
    const hipStream_t s = resolve_stream(w->device, stream);
    if ((rc = stream_pick(w->device, s, caller, slot)) != MLQ_OK) return rc;
    const mlq::LinearShape shape{w->qtype, w->M, w->K, w->nb, 1};
    const hipError_t e =
        mlq::launch_gemv_pick(shape, w->ptr, x, y, slot->state, token != nullptr ? token : slot->token, s);
    if (e != hipSuccess) return hip_fail(e, caller);
    *used = s;
    return MLQ_OK;
}

}  // namespace

int mlq_hip_quant_linear_argmax(mlq_weight_t w, const float* x, float* y, int32_t* token, void* stream) {
    if (token == nullptr) return fail(MLQ_ERR_INVALID, "hip_quant_linear_argmax: token pointer is null");
    PickSlot slot{};
    hipStream_t s = nullptr;
    return launch_pick(w, x, y, token, stream, &slot, &s);
}

int mlq_hip_sample_greedy(mlq_weight_t w, const float* x, float* y, int* token, void* stream) {
    if (token == nullptr) return fail(MLQ_ERR_INVALID, "hip_sample_greedy: token pointer is null");
    PickSlot slot{};
    hipStream_t s = nullptr;
    int rc = launch_pick(w, x, y, nullptr, stream, &slot, &s);
    if (rc != MLQ_OK) return rc;
    int32_t t = -1;
    MLQ_HIP_CHECK(hipMemcpyAsync(&t, slot.token, sizeof t, hipMemcpyDeviceToHost, s));
    MLQ_HIP_CHECK(hipStreamSynchronize(s));
    if (t < 0) return fail(MLQ_ERR_INVALID, "sampler: logits must be finite");
    *token = t;
    return MLQ_OK;
}

int mlq_hip_quantize(int device, int qtype, const float* src, int rows, int row_len,
                     void* device_blocks, void* stream) {
    if (qtype != MLQ_Q8_0 && qtype != MLQ_Q4_0 && qtype != MLQ_Q4_1) {
        return fail(MLQ_ERR_INVALID, "mlq_hip_quantize: unsupported quant type " + std::to_string(qtype));
    }
    if (rows <= 0 || row_len <= 0) return fail(MLQ_ERR_SHAPE, "mlq_hip_quantize: empty tensors are not supported");
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    const size_t nb = (static_cast<size_t>(row_len) + mlq::kQK - 1) / mlq::kQK;
    const size_t sbytes = static_cast<size_t>(rows) * row_len * sizeof(float);
    const size_t dbytes = static_cast<size_t>(rows) * nb * mlq::block_bytes(qtype);
    if ((rc = check_device_ptr(src, device, "mlq_hip_quantize", "source", sbytes)) != MLQ_OK) return rc;
    if ((rc = check_device_ptr(device_blocks, device, "mlq_hip_quantize", "block", dbytes)) != MLQ_OK) return rc;
    hipError_t e = mlq::launch_quantize(qtype, src, rows, row_len, device_blocks, resolve_stream(device, stream));
    if (e != hipSuccess) return hip_fail(e, "quantize_kernel");
    return MLQ_OK;
}

int mlq_hip_malloc(int device, size_t bytes, void** out) {
    if (out == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_malloc: null output");
    *out = nullptr;
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    MLQ_HIP_CHECK(hipMalloc(out, bytes == 0 ? 1 : bytes));
    return MLQ_OK;
}

int mlq_hip_free(void* ptr) {
    if (ptr == nullptr) return MLQ_OK;
    MLQ_HIP_CHECK(hipFree(ptr));
    return MLQ_OK;
}

// Copies and fills run on the library's stream for the current device and
// wait for it, so they are ordered after every launch the library made there
// (that stream does not synchronize with the null stream).
int mlq_hip_memcpy_htod(void* dst, const void* src, size_t bytes) {
    int dev = 0;
    MLQ_HIP_CHECK(hipGetDevice(&dev));
    int rc = ensure_device(dev);
    if (rc == MLQ_OK) rc = check_device_ptr(dst, dev, "mlq_hip_memcpy_htod", "destination", bytes);
    if (rc != MLQ_OK) return rc;
    hipStream_t s = g_dev[dev].stream;
    MLQ_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
    MLQ_HIP_CHECK(hipStreamSynchronize(s));
    return MLQ_OK;
}

int mlq_hip_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    int dev = 0;
    MLQ_HIP_CHECK(hipGetDevice(&dev));
    int rc = ensure_device(dev);
    if (rc == MLQ_OK) rc = check_device_ptr(src, dev, "mlq_hip_memcpy_dtoh", "source", bytes);
    if (rc != MLQ_OK) return rc;
    hipStream_t s = g_dev[dev].stream;
    MLQ_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
    MLQ_HIP_CHECK(hipStreamSynchronize(s));
    return MLQ_OK;
}

int mlq_hip_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream) {
    int dev = 0;
    MLQ_HIP_CHECK(hipGetDevice(&dev));
    int rc = ensure_device(dev);
    if (rc == MLQ_OK) rc = check_device_ptr(dst, dev, "mlq_hip_memcpy_dtod", "destination", bytes);
    if (rc == MLQ_OK) rc = check_device_ptr(src, dev, "mlq_hip_memcpy_dtod", "source", bytes);
    if (rc != MLQ_OK) return rc;
    MLQ_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, resolve_stream(dev, stream)));
    return MLQ_OK;
}

int mlq_hip_memset(void* ptr, int value, size_t bytes) {
    int dev = 0;
    MLQ_HIP_CHECK(hipGetDevice(&dev));
    int rc = ensure_device(dev);
    if (rc == MLQ_OK) rc = check_device_ptr(ptr, dev, "mlq_hip_memset", "destination", bytes);
    if (rc != MLQ_OK) return rc;
    hipStream_t s = g_dev[dev].stream;
    MLQ_HIP_CHECK(hipMemsetAsync(ptr, value, bytes, s));
    MLQ_HIP_CHECK(hipStreamSynchronize(s));
    return MLQ_OK;
}

int mlq_hip_stream(int device, void** stream) {
    if (stream == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_stream: null output");
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    *stream = g_dev[device].stream;
    return MLQ_OK;
}

int mlq_hip_stream_create(int device, void** stream) {
    if (stream == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_stream_create: null output");
    *stream = nullptr;
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    MLQ_HIP_CHECK(hipSetDevice(device));
    hipStream_t s = nullptr;
    MLQ_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));  // default priority
    *stream = s;
    return MLQ_OK;
}

int mlq_hip_stream_destroy(void* stream) {
    if (stream == nullptr) return MLQ_OK;
    MLQ_HIP_CHECK(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    MLQ_HIP_CHECK(hipStreamDestroy(static_cast<hipStream_t>(stream)));
    return MLQ_OK;
}

int mlq_hip_synchronize(void* stream) {
    if (stream == nullptr) {
        MLQ_HIP_CHECK(hipDeviceSynchronize());
    } else {
        MLQ_HIP_CHECK(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    }
    return MLQ_OK;
}

int mlq_hip_event_create(void** ev) {
    if (ev == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_event_create: null output");
    hipEvent_t e;
    MLQ_HIP_CHECK(hipEventCreate(&e));
    *ev = e;
    return MLQ_OK;
}

int mlq_hip_event_destroy(void* ev) {
    if (ev != nullptr) MLQ_HIP_CHECK(hipEventDestroy(static_cast<hipEvent_t>(ev)));
    return MLQ_OK;
}

int mlq_hip_event_record(void* ev, void* stream) {
    int dev = 0;
    MLQ_HIP_CHECK(hipGetDevice(&dev));
    MLQ_HIP_CHECK(hipEventRecord(static_cast<hipEvent_t>(ev),
                                 stream ? static_cast<hipStream_t>(stream) : g_dev[dev].stream));
    return MLQ_OK;
}

int mlq_hip_event_elapsed_ms(void* start, void* stop, float* ms) {
    if (ms == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_event_elapsed_ms: null output");
    MLQ_HIP_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
    MLQ_HIP_CHECK(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
    return MLQ_OK;
}

int mlq_hip_graph_capture_many(const mlq_linear_call* calls, int n, void* stream, mlq_graph_t* out) {
    if (out == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_graph_capture_many: null output");
    *out = nullptr;
    if (calls == nullptr || n <= 0 || calls[0].w == nullptr) {
        return fail(MLQ_ERR_INVALID, "mlq_hip_graph_capture_many: no calls");
    }
    const int device = calls[0].w->device;
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    // Validate everything before capture starts; nothing below may fail midway
    // except HIP itself.
    for (int i = 0; i < n; ++i) {
        const mlq_linear_call& c = calls[i];
        if (c.w == nullptr || c.w->device != device) {
            return fail(MLQ_ERR_INVALID, "mlq_hip_graph_capture_many: bad weight handle");
        }
        if ((rc = validate_linear(c.w->qtype, c.w->M, c.w->K, c.w->n_blocks, c.rows)) != MLQ_OK) return rc;
        const char* caller = caller_for(c.w->qtype);
        const size_t xb = static_cast<size_t>(c.rows) * c.w->K * sizeof(float);
        const size_t yb = static_cast<size_t>(c.rows) * c.w->M * sizeof(float);
        if ((rc = check_device_ptr(c.x, device, caller, "input", xb)) != MLQ_OK) return rc;
        if ((rc = check_device_ptr(c.y, device, caller, "output", yb)) != MLQ_OK) return rc;
    }
    hipStream_t s = resolve_stream(device, stream);
    // Batched calls need the stream's GEMM workspace; size it for the largest
    // before capture (no allocation may happen inside a capture).  All batched
    // nodes of the graph run in stream order and share it.
    size_t ws_need = 0;
    for (int i = 0; i < n; ++i) {
        const mlq_linear_call& c = calls[i];
        mlq::LinearShape shape{c.w->qtype, c.w->M, c.w->K, c.w->nb, c.rows};
        if (c.rows > 1 && mlq::gemm_supported(shape)) {
            ws_need = std::max(ws_need, mlq::gemm_workspace_bytes(shape));
        }
    }
    if (ws_need > 0) {
        void* ws = nullptr;
        if ((rc = stream_workspace(device, s, ws_need, &ws)) != MLQ_OK) return rc;
    }
    MLQ_HIP_CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int launch_rc = MLQ_OK;
    for (int i = 0; i < n && launch_rc == MLQ_OK; ++i) {
        const mlq_linear_call& c = calls[i];
        mlq::LinearShape shape{c.w->qtype, c.w->M, c.w->K, c.w->nb, c.rows};
        launch_rc = dispatch(device, shape, c.w->ptr, c.x, c.y, s);
    }
    return end_capture(s, device, launch_rc, out);
}

int mlq_hip_graph_launch(mlq_graph_t g, void* stream) {
    if (g == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_graph_launch: null graph");
    int rc = ensure_device(g->device);
    if (rc != MLQ_OK) return rc;
    MLQ_HIP_CHECK(hipGraphLaunch(g->exec, resolve_stream(g->device, stream)));
    return MLQ_OK;
}

int mlq_hip_graph_destroy(mlq_graph_t g) {
    if (g == nullptr) return MLQ_OK;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
    return MLQ_OK;
}

int mlq_hip_graph_begin(int device, void* stream) {
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    MLQ_HIP_CHECK(hipStreamBeginCapture(resolve_stream(device, stream), hipStreamCaptureModeThreadLocal));
    return MLQ_OK;
}

int mlq_hip_graph_end(int device, void* stream, mlq_graph_t* out) {
    if (out == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_graph_end: null output");
    *out = nullptr;
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    return end_capture(resolve_stream(device, stream), device, MLQ_OK, out);
}

int mlq_hip_fill_normal(float* device_dst, size_t n, uint64_t seed, float mean, float stddev,
                        void* stream) {
    int dev = 0;
    MLQ_HIP_CHECK(hipGetDevice(&dev));
    int rc = ensure_device(dev);
    if (rc != MLQ_OK) return rc;
    if (n == 0) return MLQ_OK;
    if ((rc = check_device_ptr(device_dst, dev, "mlq_hip_fill_normal", "destination", n * sizeof(float))) != MLQ_OK) return rc;
    hipError_t e = mlq::launch_fill_normal(device_dst, n, seed, mean, stddev, resolve_stream(dev, stream));
    if (e != hipSuccess) return hip_fail(e, "fill_normal_kernel");
    return MLQ_OK;
}

// ---- device forward ops (include/mini_llama/cuda_ops.h, cuda_attention.h,
// cuda_matmul.h).  Every pointer is checked to lie inside a device allocation
// on `device` of at least the size the shape implies before the launch.

int mlq_hip_rmsnorm(int device, const float* x, const float* weight, int n, float eps, float* y, void* stream) {
    const char* caller = "mlq_hip_rmsnorm";
    if (n <= 0) return fail(MLQ_ERR_SHAPE, std::string(caller) + ": empty tensor");
    if (!std::isfinite(eps) || eps <= 0.0f) return fail(MLQ_ERR_INVALID, std::string(caller) + ": eps must be finite and positive");
    int rc = ensure_device(device);
    const size_t b = static_cast<size_t>(n) * sizeof(float);
    if (rc == MLQ_OK) rc = check_device_ptr(x, device, caller, "input", b);
    if (rc == MLQ_OK) rc = check_device_ptr(weight, device, caller, "weight", b);
    if (rc == MLQ_OK) rc = check_device_ptr(y, device, caller, "output", b);
    if (rc != MLQ_OK) return rc;
    hipError_t e = mlq::launch_op_rmsnorm(x, weight, n, eps, y, resolve_stream(device, stream));
    return e == hipSuccess ? MLQ_OK : hip_fail(e, "op_rmsnorm_kernel");
}

static int elementwise_entry(int op, const char* caller, int device, const float* a, const float* b, size_t n, float* y,
                void* stream) {
    if (n == 0) return MLQ_OK;
    int rc = ensure_device(device);
    const size_t bytes = n * sizeof(float);
    if (rc == MLQ_OK) rc = check_device_ptr(a, device, caller, "input", bytes);
    if (rc == MLQ_OK && op != mlq::kOpSilu) rc = check_device_ptr(b, device, caller, "second input", bytes);
    if (rc == MLQ_OK) rc = check_device_ptr(y, device, caller, "output", bytes);
    if (rc != MLQ_OK) return rc;
    hipError_t e = mlq::launch_op_elementwise(op, a, b, n, y, resolve_stream(device, stream));
    return e == hipSuccess ? MLQ_OK : hip_fail(e, "op_elementwise_kernel");
}

int mlq_hip_silu(int device, const float* x, size_t n, float* y, void* stream) {
    return elementwise_entry(mlq::kOpSilu, "mlq_hip_silu", device, x, nullptr, n, y, stream);
}

int mlq_hip_mul(int device, const float* a, const float* b, size_t n, float* y, void* stream) {
    return elementwise_entry(mlq::kOpMul, "mlq_hip_mul", device, a, b, n, y, stream);
}

int mlq_hip_add(int device, const float* a, const float* b, size_t n, float* y, void* stream) {
    return elementwise_entry(mlq::kOpAdd, "mlq_hip_add", device, a, b, n, y, stream);
}

int mlq_hip_softmax(int device, const float* x, int n, float* y, void* stream) {
    const char* caller = "mlq_hip_softmax";
    if (n <= 0) return fail(MLQ_ERR_SHAPE, std::string(caller) + ": empty tensor");
    int rc = ensure_device(device);
    const size_t b = static_cast<size_t>(n) * sizeof(float);
    if (rc == MLQ_OK) rc = check_device_ptr(x, device, caller, "input", b);
    if (rc == MLQ_OK) rc = check_device_ptr(y, device, caller, "output", b);
    if (rc != MLQ_OK) return rc;
    hipError_t e = mlq::launch_op_softmax(x, n, y, resolve_stream(device, stream));
    return e == hipSuccess ? MLQ_OK : hip_fail(e, "op_softmax_kernel");
}

int mlq_hip_embedding(int device, const float* table, int vocab, int dim, int token, float* y, void* stream) {
    const char* caller = "mlq_hip_embedding";
    if (vocab <= 0 || dim <= 0) return fail(MLQ_ERR_SHAPE, std::string(caller) + ": embedding shape must be positive");
    if (token < 0 || token >= vocab) return fail(MLQ_ERR_LIMIT, std::string(caller) + ": token id out of range");
    int rc = ensure_device(device);
    if (rc == MLQ_OK) {
        rc = check_device_ptr(table, device, caller, "embedding", static_cast<size_t>(vocab) * dim * sizeof(float));
    }
    if (rc == MLQ_OK) rc = check_device_ptr(y, device, caller, "output", static_cast<size_t>(dim) * sizeof(float));
    if (rc != MLQ_OK) return rc;
    hipError_t e = mlq::launch_op_embedding(table, dim, token, y, resolve_stream(device, stream));
    return e == hipSuccess ? MLQ_OK : hip_fail(e, "op_embedding_kernel");
}

int mlq_hip_rope(int device, float* x, int n_heads, int head_dim, int pos, float theta, int neox, void* stream) {
    const char* caller = "mlq_hip_rope";
    if (n_heads <= 0 || head_dim <= 0 || head_dim % 2 != 0) {
        return fail(MLQ_ERR_SHAPE, std::string(caller) + ": invalid head shape");
    }
    if (pos < 0) return fail(MLQ_ERR_LIMIT, std::string(caller) + ": position must be non-negative");
    if (!std::isfinite(theta) || theta <= 0.0f) {
        return fail(MLQ_ERR_INVALID, std::string(caller) + ": theta must be finite and positive");
    }
    int rc = ensure_device(device);
    if (rc == MLQ_OK) {
        rc = check_device_ptr(x, device, caller, "input", static_cast<size_t>(n_heads) * head_dim * sizeof(float));
    }
    if (rc != MLQ_OK) return rc;
    hipError_t e = mlq::launch_op_rope(x, n_heads, head_dim, pos, theta, neox != 0, resolve_stream(device, stream));
    return e == hipSuccess ? MLQ_OK : hip_fail(e, "op_rope_kernel");
}

int mlq_hip_attention_decode(int device, const float* q, const float* keys, const float* values, int n_layers,
                             int layer, int max_seq_len, int n_heads, int n_kv_heads, int head_dim, int pos,
                             float* out, void* stream) {
    const char* caller = "mlq_hip_attention_decode";
    if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || n_layers <= 0 || max_seq_len <= 0) {
        return fail(MLQ_ERR_SHAPE, std::string(caller) + ": head counts, head_dim and cache extents must be positive");
    }
    if (n_heads % n_kv_heads != 0) {
        return fail(MLQ_ERR_SHAPE, std::string(caller) + ": n_heads must be divisible by n_kv_heads");
    }
    if (head_dim > mlq::kOpAttnMaxHeadDim) {
        return fail(MLQ_ERR_LIMIT, std::string(caller) + ": head_dim above " +
                                       std::to_string(mlq::kOpAttnMaxHeadDim) + " is not supported");
    }
    if (layer < 0 || layer >= n_layers) return fail(MLQ_ERR_LIMIT, std::string(caller) + ": layer out of range");
    if (pos < 0 || pos >= max_seq_len) return fail(MLQ_ERR_LIMIT, std::string(caller) + ": position out of range");
    int rc = ensure_device(device);
    const size_t cache = static_cast<size_t>(n_layers) * max_seq_len * n_kv_heads * head_dim * sizeof(float);
    const size_t qb = static_cast<size_t>(n_heads) * head_dim * sizeof(float);
    if (rc == MLQ_OK) rc = check_device_ptr(q, device, caller, "query", qb);
    if (rc == MLQ_OK) rc = check_device_ptr(keys, device, caller, "key cache", cache);
    if (rc == MLQ_OK) rc = check_device_ptr(values, device, caller, "value cache", cache);
    if (rc == MLQ_OK) rc = check_device_ptr(out, device, caller, "output", qb);
    if (rc != MLQ_OK) return rc;
    hipError_t e = mlq::launch_op_attention_decode(q, keys, values, layer, max_seq_len, n_heads, n_kv_heads, head_dim,
                                                   pos, out, resolve_stream(device, stream));
    return e == hipSuccess ? MLQ_OK : hip_fail(e, "op_attention_decode_kernel");
}

int mlq_hip_matmul_f32(int device, const float* a, const float* b, int m, int k, int n, int b_transposed, float* c,
                       void* stream) {
    const char* caller = "mlq_hip_matmul_f32";
    if (m <= 0 || k <= 0 || n <= 0) return fail(MLQ_ERR_SHAPE, std::string(caller) + ": empty tensors are not supported");
    int rc = ensure_device(device);
    if (rc == MLQ_OK) rc = check_device_ptr(a, device, caller, "A", static_cast<size_t>(m) * k * sizeof(float));
    if (rc == MLQ_OK) rc = check_device_ptr(b, device, caller, "B", static_cast<size_t>(k) * n * sizeof(float));
    if (rc == MLQ_OK) rc = check_device_ptr(c, device, caller, "C", static_cast<size_t>(m) * n * sizeof(float));
    if (rc != MLQ_OK) return rc;
    hipError_t e = mlq::launch_op_matmul_f32(a, b, m, k, n, b_transposed != 0, c, resolve_stream(device, stream));
    return e == hipSuccess ? MLQ_OK : hip_fail(e, "op_matmul_f32_kernel");
}

int mlq_hip_kernel_name(int qtype, int rows, int out_features, int in_features, char* buf,
                        size_t len) {
    if (buf == nullptr || len == 0) return fail(MLQ_ERR_INVALID, "mlq_hip_kernel_name: null buffer");
    mlq::LinearShape s{qtype, out_features, in_features, (in_features + 31) / 32, rows};
    const char* name = (rows > 1 && mlq::gemm_supported(s)) ? mlq::gemm_kernel_name(s)
                                                               : mlq::gemv_kernel_name(s);
    std::snprintf(buf, len, "%s", name);
    return MLQ_OK;
}

}  // extern "C"

// ---- sequences --------------------------------------------------------------

namespace {

struct Range {
    uintptr_t lo;
    uintptr_t hi;
};

bool overlaps(const Range& a, const Range& b) { return a.lo < b.hi && b.lo < a.hi; }

Range range_of(const void* p, size_t bytes) {
    const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
    return Range{lo, lo + bytes};
}

constexpr unsigned kDefaultSpinLimit = 1u << 20;

}  // namespace

extern "C" {

int mlq_hip_sequence_create(const mlq_linear_call* calls, int n, const int* stage, int mode,
                            mlq_sequence_t* out) {
    static const char* caller = "mlq_hip_sequence_create";
    if (out == nullptr) return fail(MLQ_ERR_INVALID, std::string(caller) + ": null output");
    *out = nullptr;
    if (calls == nullptr || n <= 0) return fail(MLQ_ERR_INVALID, std::string(caller) + ": no calls");
    if (mode != MLQ_SEQ_PERSISTENT && mode != MLQ_SEQ_PER_STAGE && mode != MLQ_SEQ_INDEPENDENT &&
        mode != MLQ_SEQ_PIPELINED && mode != MLQ_SEQ_LDS_RING) {
        return fail(MLQ_ERR_INVALID, std::string(caller) + ": unknown mode " + std::to_string(mode));
    }
    if (calls[0].w == nullptr) return fail(MLQ_ERR_INVALID, std::string(caller) + ": null weight handle");
    const int device = calls[0].w->device;
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;

    std::vector<Range> wr(n), xr(n), yr(n);
    for (int i = 0; i < n; ++i) {
        const mlq_linear_call& c = calls[i];
        const std::string at = std::string(caller) + ": call " + std::to_string(i);
        if (c.w == nullptr) return fail(MLQ_ERR_INVALID, at + ": null weight handle");
        if (c.w->device != device) return fail(MLQ_ERR_DEVICE, at + ": weight on a different device");
        if (c.rows != 1) {
            return fail(MLQ_ERR_INVALID, at + ": rows=" + std::to_string(c.rows) +
                                             "; a sequence runs GEMV calls (rows == 1)");
        }
        if ((rc = validate_linear(c.w->qtype, c.w->M, c.w->K, c.w->n_blocks, 1)) != MLQ_OK) return rc;
        if (!mlq::sequence_supported(c.w->qtype, c.w->K)) {
            return fail(MLQ_ERR_LIMIT, at + ": in_features=" + std::to_string(c.w->K) +
                                           " needs an even block count and at most 15360 elements");
        }
        if (mode == MLQ_SEQ_PIPELINED && c.w->K % mlq::kQK != 0) {
            return fail(MLQ_ERR_LIMIT, at + ": in_features=" + std::to_string(c.w->K) +
                                           "; MLQ_SEQ_PIPELINED needs in_features % 32 == 0");
        }
        if (mode == MLQ_SEQ_LDS_RING) {
            if (mlq::sequence_lpr(c.w->K) != 64) {
                return fail(MLQ_ERR_LIMIT, at + ": in_features=" + std::to_string(c.w->K) +
                                               "; MLQ_SEQ_LDS_RING needs rows summed in 64-lane groups");
            }
            if (c.w->n_blocks * static_cast<size_t>(mlq::block_bytes(c.w->qtype)) >= (static_cast<size_t>(1) << 31)) {
                return fail(MLQ_ERR_LIMIT, at + ": weight of 2 GiB or more; MLQ_SEQ_LDS_RING addresses a weight "
                                               "with 31-bit offsets");
            }
        }
        const char* lin = caller_for(c.w->qtype);
        const size_t xb = static_cast<size_t>(c.w->K) * sizeof(float);
        const size_t yb = static_cast<size_t>(c.w->M) * sizeof(float);
        if ((rc = check_device_ptr(c.x, device, lin, "input", xb)) != MLQ_OK) return rc;
        if ((rc = check_device_ptr(c.y, device, lin, "output", yb)) != MLQ_OK) return rc;
        wr[i] = range_of(c.w->ptr, c.w->n_blocks * static_cast<size_t>(mlq::block_bytes(c.w->qtype)));
        xr[i] = range_of(c.x, xb);
        yr[i] = range_of(c.y, yb);
    }
    // Outputs never overlap weights (the kernel requests weights of later
    // stages before earlier outputs are written).
    for (int i = 0; i < n; ++i) {
        for (int j = 0; j < n; ++j) {
            if (overlaps(yr[i], wr[j])) {
                return fail(MLQ_ERR_INVALID, std::string(caller) + ": output of call " + std::to_string(i) +
                                                 " overlaps the weight of call " + std::to_string(j));
            }
            if (mode == MLQ_SEQ_INDEPENDENT && overlaps(yr[i], xr[j])) {
                return fail(MLQ_ERR_INVALID, std::string(caller) + ": output of call " + std::to_string(i) +
                                                 " overlaps the input of call " + std::to_string(j) +
                                                 "; MLQ_SEQ_INDEPENDENT needs independent calls");
            }
        }
    }

    // Stages: runs of equal stage ids (or single calls).
    std::vector<mlq::SeqStageDesc> descs;
    std::vector<int> stage_first;
    for (int i = 0; i < n;) {
        int j = i + 1;
        if (stage != nullptr) {
            while (j < n && stage[j] == stage[i]) ++j;
        }
        if (j - i > mlq::kSeqMaxCalls) {
            return fail(MLQ_ERR_LIMIT, std::string(caller) + ": stage starting at call " + std::to_string(i) +
                                           " has " + std::to_string(j - i) + " calls (at most " +
                                           std::to_string(mlq::kSeqMaxCalls) + ")");
        }
        const mlq_weight_s* w0 = calls[i].w;
        mlq::SeqStageDesc d;
        std::memset(&d, 0, sizeof d);
        d.x = calls[i].x;
        d.K = w0->K;
        d.nb = w0->nb;
        d.np = w0->nb / 2;
        const int lpr = mlq::sequence_lpr(w0->K);
        d.nch = (d.np + lpr - 1) / lpr;
        d.ncalls = j - i;
        long long rows = 0;
        for (int k = i; k < j; ++k) {
            const mlq_linear_call& c = calls[k];
            if (c.x != calls[i].x || c.w->K != w0->K || c.w->qtype != w0->qtype) {
                return fail(MLQ_ERR_INVALID, std::string(caller) + ": call " + std::to_string(k) +
                                                 " differs from call " + std::to_string(i) +
                                                 " of its stage in input, in_features or quant type");
            }
            if (overlaps(yr[k], xr[k])) {
                return fail(MLQ_ERR_INVALID, std::string(caller) + ": output of call " + std::to_string(k) +
                                                 " overlaps its stage's input");
            }
            for (int m = i; m < k; ++m) {
                if (overlaps(yr[k], yr[m])) {
                    return fail(MLQ_ERR_INVALID, std::string(caller) + ": outputs of calls " + std::to_string(m) +
                                                     " and " + std::to_string(k) + " of one stage overlap");
                }
            }
            d.call[k - i] = mlq::SeqCallDesc{c.w->ptr, c.y, c.w->M, static_cast<int>(rows)};
            rows += c.w->M;
        }
        if (rows > (1ll << 30)) return fail(MLQ_ERR_LIMIT, std::string(caller) + ": stage has too many rows");
        d.rows = static_cast<int>(rows);
        const int sub = 64 / lpr;
        d.items = (d.rows + sub - 1) / sub;
        descs.push_back(d);
        stage_first.push_back(i);
        i = j;
    }
    std::vector<mlq_sequence_s::HostStage> host_stages;
    for (size_t k = 0; k < descs.size(); ++k) {
        const mlq::SeqStageDesc& d = descs[k];
        mlq_sequence_s::HostStage hs;
        hs.shape = mlq::LinearShape{calls[stage_first[k]].w->qtype, d.rows, d.K, d.nb, 1};
        hs.group = mlq::GemvGroup{};
        for (int c = 0; c < d.ncalls; ++c) {
            hs.group.W[c] = d.call[c].W;
            hs.group.y[c] = d.call[c].y;
            hs.group.row_begin[c] = d.call[c].row_begin;
        }
        hs.group.ncalls = d.ncalls;
        hs.x = d.x;
        host_stages.push_back(hs);
    }

    // Segments: runs of stages with one kernel variant; one per stage in
    // per-stage mode.
    auto seq = new mlq_sequence_s;
    seq->device = device;
    seq->mode = mode;
    seq->nstages = static_cast<int>(descs.size());
    seq->spin_limit = kDefaultSpinLimit;
    seq->mem = nullptr;
    seq->host_stages = std::move(host_stages);
    for (int s = 0; s < seq->nstages; ++s) {
        const mlq_weight_s* w0 = calls[stage_first[s]].w;
        const int lpr = mlq::sequence_lpr(w0->K);
        const int lds = mlq::sequence_stage_lds_bytes(w0->qtype, w0->K);
        bool extend = !seq->segs.empty() && mode != MLQ_SEQ_PER_STAGE;
        if (extend) {
            const auto& last = seq->segs.back();
            extend = last.qtype == w0->qtype && last.lpr == lpr;
        }
        if (extend) {
            auto& last = seq->segs.back();
            last.nstages += 1;
            last.lds_bytes = std::max(last.lds_bytes, lds);
            last.kmax = std::max(last.kmax, w0->K);
            descs[s].barrier = mode == MLQ_SEQ_PERSISTENT || mode == MLQ_SEQ_PIPELINED || mode == MLQ_SEQ_LDS_RING ? 1 : 0;
        } else {
            seq->segs.push_back(mlq_sequence_s::Segment{w0->qtype, lpr, s, 1, lds, 0, w0->K});
            descs[s].barrier = 0;
        }
    }
    for (auto& g : seq->segs) {
        int nslots = 0;
        if (mode == MLQ_SEQ_PIPELINED) g.lds_bytes = mlq::chain_lds_bytes(g.qtype, g.kmax);
        if (mode == MLQ_SEQ_LDS_RING) {
            g.lds_bytes = mlq::ring_lds_bytes(g.qtype, g.kmax, &nslots);
            if (nslots < 8) {  // two slots per loader wave at least
                delete seq;
                return fail(MLQ_ERR_LIMIT, std::string(caller) + ": in_features=" + std::to_string(g.kmax) +
                                               " leaves too little LDS for MLQ_SEQ_LDS_RING's weight ring");
            }
        }
        hipError_t e = mode == MLQ_SEQ_PIPELINED  ? mlq::chain_grid(g.qtype, g.lpr, g.lds_bytes, device, &g.grid)
                       : mode == MLQ_SEQ_LDS_RING ? mlq::ring_grid(g.qtype, g.lds_bytes, device, &g.grid)
                                                  : mlq::sequence_grid(g.qtype, g.lpr, g.lds_bytes, device, &g.grid);
        if (e != hipSuccess) {
            delete seq;
            return hip_fail(e, "sequence occupancy");
        }
        for (int k = g.stage_begin; k < g.stage_begin + g.nstages; ++k) {
            // A stage reads x coherently when an earlier stage of the same
            // launch writes where it reads.
            descs[k].coherent = 0;
            if (mode == MLQ_SEQ_PERSISTENT || mode == MLQ_SEQ_PIPELINED || mode == MLQ_SEQ_LDS_RING) {
                for (int e2 = g.stage_begin; e2 < k; ++e2)
                    for (int c = stage_first[e2]; c < stage_first[e2] + descs[e2].ncalls; ++c)
                        if (overlaps(yr[c], xr[stage_first[k]])) descs[k].coherent = 1;
            }
        }
    }
    const size_t table_bytes = descs.size() * sizeof(mlq::SeqStageDesc);
    seq->sync_offset = (table_bytes + 255) & ~static_cast<size_t>(255);
    const size_t sync_end = seq->sync_offset + seq->segs.size() * sizeof(mlq::SeqSync);
    seq->sink_offset = (sync_end + 255) & ~static_cast<size_t>(255);
    const size_t total = seq->sink_offset + (mode == MLQ_SEQ_PIPELINED ? mlq::chain_sink_bytes() : 0);
    hipError_t e = hipMalloc(&seq->mem, total);
    if (e == hipSuccess) e = hipMemset(seq->mem, 0, total);
    if (e == hipSuccess) e = hipMemcpy(seq->mem, descs.data(), table_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        if (seq->mem) (void)hipFree(seq->mem);
        delete seq;
        return hip_fail(e, "sequence upload");
    }
    *out = seq;
    return MLQ_OK;
}

int mlq_hip_ring_stamps(uint64_t* host, size_t words) {
    static const char* caller = "mlq_hip_ring_stamps";
    if (host == nullptr) return fail(MLQ_ERR_INVALID, std::string(caller) + ": null output");
    if (words != MLQ_RING_STAMP_WORDS) {
        return fail(MLQ_ERR_INVALID, std::string(caller) + ": words=" + std::to_string(words) + ", expected " +
                                         std::to_string(MLQ_RING_STAMP_WORDS));
    }
    static_assert(MLQ_RING_STAMP_WORDS == mlq::kRingStampWgs * mlq::kRingStampStages * mlq::kRingStampSlots,
                  "stamp layout");
    hipError_t e = mlq::ring_stamps_copy(host, words * sizeof(uint64_t));
    if (e == hipErrorNotSupported) {
        return fail(MLQ_ERR_NOT_BUILT, std::string(caller) + ": the library was built without the timestamps "
                                                             "(make stamps builds libmlq_hip_stamps.so)");
    }
    if (e != hipSuccess) return hip_fail(e, caller);
    return MLQ_OK;
}

int mlq_hip_sequence_launch(mlq_sequence_t seq, void* stream) {
    if (seq == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_sequence_launch: null sequence");
    int rc = ensure_device(seq->device);
    if (rc != MLQ_OK) return rc;
    hipStream_t s = resolve_stream(seq->device, stream);
    if (seq->mode == MLQ_SEQ_PER_STAGE) {
        for (const auto& hs : seq->host_stages) {
            hipError_t e = mlq::launch_gemv_group(hs.shape, hs.group, hs.x, s);
            if (e != hipSuccess) return hip_fail(e, mlq::gemv_kernel_name(hs.shape));
        }
        return MLQ_OK;
    }
    auto* table = static_cast<const mlq::SeqStageDesc*>(seq->mem);
    auto* syncs = reinterpret_cast<mlq::SeqSync*>(static_cast<char*>(seq->mem) + seq->sync_offset);
    for (size_t i = 0; i < seq->segs.size(); ++i) {
        const auto& g = seq->segs[i];
        if (seq->mode == MLQ_SEQ_PIPELINED) {
            float* sink = reinterpret_cast<float*>(static_cast<char*>(seq->mem) + seq->sink_offset);
            hipError_t e = mlq::launch_chain(g.qtype, g.lpr, table + g.stage_begin, g.nstages, syncs + i, g.grid,
                                             g.lds_bytes, seq->spin_limit, g.kmax, sink, s);
            if (e != hipSuccess) return hip_fail(e, mlq::chain_kernel_name(g.qtype, g.lpr));
            continue;
        }
        if (seq->mode == MLQ_SEQ_LDS_RING) {
            hipError_t e = mlq::launch_ring(g.qtype, table + g.stage_begin, g.nstages, syncs + i, g.grid, g.lds_bytes,
                                            seq->spin_limit, g.kmax, s);
            if (e != hipSuccess) return hip_fail(e, mlq::ring_kernel_name(g.qtype));
            continue;
        }
        hipError_t e = mlq::launch_sequence(g.qtype, g.lpr, table + g.stage_begin, g.nstages, syncs + i, g.grid,
                                            g.lds_bytes, seq->spin_limit, s);
        if (e != hipSuccess) return hip_fail(e, mlq::sequence_kernel_name(g.qtype, g.lpr));
    }
    return MLQ_OK;
}

int mlq_hip_sequence_status(mlq_sequence_t seq, int* barrier_timeouts) {
    if (seq == nullptr || barrier_timeouts == nullptr) {
        return fail(MLQ_ERR_INVALID, "mlq_hip_sequence_status: null argument");
    }
    int rc = ensure_device(seq->device);
    if (rc != MLQ_OK) return rc;
    *barrier_timeouts = 0;
    auto* syncs = reinterpret_cast<mlq::SeqSync*>(static_cast<char*>(seq->mem) + seq->sync_offset);
    for (size_t i = 0; i < seq->segs.size(); ++i) {
        unsigned err = 0;
        MLQ_HIP_CHECK(hipMemcpy(&err, &syncs[i].error[0], sizeof err, hipMemcpyDeviceToHost));
        if (err != 0) {
            ++*barrier_timeouts;
            MLQ_HIP_CHECK(hipMemset(&syncs[i].error[0], 0, sizeof(unsigned)));
        }
    }
    MLQ_HIP_CHECK(hipDeviceSynchronize());
    return MLQ_OK;
}

int mlq_hip_sequence_set_spin_limit(mlq_sequence_t seq, unsigned polls) {
    if (seq == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_sequence_set_spin_limit: null sequence");
    seq->spin_limit = polls;
    return MLQ_OK;
}

int mlq_hip_sequence_info(mlq_sequence_t seq, int* stages, int* launches, int* grid) {
    if (seq == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_sequence_info: null sequence");
    if (stages) *stages = seq->nstages;
    if (launches) {
        *launches = seq->mode == MLQ_SEQ_PER_STAGE ? seq->nstages : static_cast<int>(seq->segs.size());
    }
    if (grid) *grid = seq->segs.empty() ? 0 : seq->segs[0].grid;
    return MLQ_OK;
}

int mlq_hip_sequence_destroy(mlq_sequence_t seq) {
    if (seq == nullptr) return MLQ_OK;
    (void)hipSetDevice(seq->device);
    hipError_t e = hipSuccess;
    if (seq->mem) {
        e = hipDeviceSynchronize();
        hipError_t f = hipFree(seq->mem);
        if (e == hipSuccess) e = f;
    }
    delete seq;
    if (e != hipSuccess) return hip_fail(e, "mlq_hip_sequence_destroy");
    return MLQ_OK;
}

namespace {

constexpr size_t kPinChunk = size_t(16) << 20;

// Host threads for the host half of file uploads.  A piece's copy from the
// file mapping into the pinned stage is split into slices that the calling
// thread and the workers copy at once, so the page faults on the mapping and
// the copy itself run on several cores (one core copies a page-cache-warm
// mapping at ~15 GB/s).  One copy at a time; the workers sleep in between.
class CopyPool {
public:
    // Never destroyed: a forked child holds copies of the parent's
    // std::thread objects (their threads do not exist there), and destroying
    // a joinable std::thread terminates the process.  At exit the workers are
    // blocked on the condition variable and end with the process.
    static CopyPool& get() {
        static CopyPool* pool = new CopyPool;
        return *pool;
    }

    void copy(void* dst, const void* src, size_t n) {
        const unsigned parts = static_cast<unsigned>(workers_.size()) + 1;
        // (a forked child has none of the workers)
        if (parts == 1 || n < kMinSlice * parts || getpid() != owner_) {
            std::memcpy(dst, src, n);
            return;
        }
        std::lock_guard<std::mutex> one(job_mu_);
        {
            std::lock_guard<std::mutex> l(mu_);
            job_ = Job{static_cast<char*>(dst), static_cast<const char*>(src), n, parts};
            pending_ = parts - 1;
            ++generation_;
        }
        wake_.notify_all();
        run_slice(job_, 0);
        std::unique_lock<std::mutex> l(mu_);
        done_.wait(l, [&] { return pending_ == 0; });
    }

private:
    struct Job {
        char* dst;
        const char* src;
        size_t n;
        unsigned parts;
    };
    static constexpr size_t kMinSlice = size_t(1) << 20;

    CopyPool() : owner_(getpid()) {
        const unsigned hw = std::thread::hardware_concurrency();
        const unsigned n = std::min(7u, hw > 1 ? hw / 2 : 0u);
        // A thread that cannot be started leaves the pool smaller (at worst
        // empty: every copy then runs on the calling thread).
        for (unsigned i = 0; i < n; ++i) {
            try {
                workers_.emplace_back([this, i] { loop(i + 1); });
            } catch (const std::exception&) {
                break;
            }
        }
    }

    // Slice i of the job, 4 KiB aligned.
    static void run_slice(const Job& j, unsigned i) {
        const size_t per = ((j.n + j.parts - 1) / j.parts + 4095) & ~size_t(4095);
        const size_t b = std::min(j.n, per * i), e = std::min(j.n, b + per);
        if (e > b) std::memcpy(j.dst + b, j.src + b, e - b);
    }

    void loop(unsigned slice) {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> l(mu_);
        for (;;) {
            wake_.wait(l, [&] { return generation_ != seen; });
            seen = generation_;
            const Job j = job_;
            l.unlock();
            run_slice(j, slice);
            l.lock();
            if (--pending_ == 0) done_.notify_one();
        }
    }

    const pid_t owner_;
    std::vector<std::thread> workers_;
    std::mutex job_mu_;  // one copy at a time
    std::mutex mu_;
    std::condition_variable wake_, done_;
    Job job_{};
    unsigned pending_ = 0;
    uint64_t generation_ = 0;
};

// Copies `bytes` from host memory that is not pinned (a file mapping) into
// device memory: 16 MiB pieces go through two pinned buffers in turn, so the
// host copy of one piece (split over CopyPool's threads) overlaps the DMA of
// the other.  Synchronous.
int upload_from_host(int device, void* dst, const uint8_t* src, uint64_t bytes) {
    DeviceState& st = g_dev[device];
    std::lock_guard<std::mutex> lock(st.pin_mu);
    for (int b = 0; b < 2; ++b) {
        if (st.pin[b] == nullptr) {
            MLQ_HIP_CHECK(hipHostMalloc(&st.pin[b], kPinChunk, hipHostMallocDefault));
            MLQ_HIP_CHECK(hipEventCreateWithFlags(&st.pin_done[b], hipEventDisableTiming));
        }
    }
    const hipStream_t s = st.stream;
    uint64_t k = 0;
    for (uint64_t off = 0; off < bytes; off += kPinChunk, ++k) {
        const int b = static_cast<int>(k & 1);
        const size_t n = static_cast<size_t>(std::min<uint64_t>(kPinChunk, bytes - off));
        if (k >= 2) MLQ_HIP_CHECK(hipEventSynchronize(st.pin_done[b]));
        CopyPool::get().copy(st.pin[b], src + off, n);
        MLQ_HIP_CHECK(hipMemcpyAsync(static_cast<char*>(dst) + off, st.pin[b], n, hipMemcpyHostToDevice, s));
        MLQ_HIP_CHECK(hipEventRecord(st.pin_done[b], s));
    }
    MLQ_HIP_CHECK(hipStreamSynchronize(s));
    return MLQ_OK;
}

int copy_out(const std::string& v, char* buf, size_t cap, const char* caller, const char* what) {
    if (buf == nullptr) return MLQ_OK;
    if (v.size() + 1 > cap) {
        return fail(MLQ_ERR_LIMIT, std::string(caller) + ": " + what + " needs " + std::to_string(v.size() + 1) +
                                       " bytes, the buffer holds " + std::to_string(cap));
    }
    std::memcpy(buf, v.c_str(), v.size() + 1);
    return MLQ_OK;
}

}  // namespace

int mlq_hip_gguf_open(const char* path, mlq_gguf_t* out) {
    if (out == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_gguf_open: null output");
    *out = nullptr;
    if (path == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_gguf_open: null path");
    mlq_gguf_t g = new mlq_gguf_s;
    if (!g->index.open(path)) {
        const std::string msg = g->index.error;
        delete g;
        return fail(MLQ_ERR_INVALID, msg);
    }
    *out = g;
    return MLQ_OK;
}

int mlq_hip_gguf_close(mlq_gguf_t g) {
    delete g;
    return MLQ_OK;
}

int mlq_hip_gguf_header(mlq_gguf_t g, uint32_t* version, uint64_t* n_tensors, uint64_t* n_metadata,
                        uint64_t* data_offset) {
    if (g == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_gguf_header: null file");
    if (version) *version = g->index.version;
    if (n_tensors) *n_tensors = g->index.n_tensors;
    if (n_metadata) *n_metadata = g->index.n_metadata;
    if (data_offset) *data_offset = g->index.data_offset;
    return MLQ_OK;
}

int mlq_hip_gguf_metadata(mlq_gguf_t g, uint64_t i, char* key, size_t key_cap, uint32_t* type, char* value,
                          size_t value_cap) {
    static const char* caller = "mlq_hip_gguf_metadata";
    if (g == nullptr) return fail(MLQ_ERR_INVALID, std::string(caller) + ": null file");
    if (i >= g->index.metadata.size()) return fail(MLQ_ERR_INVALID, std::string(caller) + ": index out of range");
    const mlq::GgufMeta& m = g->index.metadata[i];
    int rc = copy_out(m.key, key, key_cap, caller, "key");
    if (rc == MLQ_OK) rc = copy_out(m.value, value, value_cap, caller, "value");
    if (rc == MLQ_OK && type) *type = m.type;
    return rc;
}

int mlq_hip_gguf_tensor(mlq_gguf_t g, uint64_t i, char* name, size_t name_cap, uint32_t* n_dims, uint64_t* dims,
                        uint32_t* ggml_type, uint64_t* offset, uint64_t* nbytes) {
    static const char* caller = "mlq_hip_gguf_tensor";
    if (g == nullptr) return fail(MLQ_ERR_INVALID, std::string(caller) + ": null file");
    if (i >= g->index.tensors.size()) return fail(MLQ_ERR_INVALID, std::string(caller) + ": index out of range");
    const mlq::GgufTensor& t = g->index.tensors[i];
    int rc = copy_out(t.name, name, name_cap, caller, "name");
    if (rc != MLQ_OK) return rc;
    if (n_dims) *n_dims = static_cast<uint32_t>(t.dims.size());
    if (dims) {
        for (size_t d = 0; d < 8; ++d) dims[d] = d < t.dims.size() ? t.dims[d] : 0;
    }
    if (ggml_type) *ggml_type = t.type;
    if (offset) *offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return MLQ_OK;
}

int mlq_hip_gguf_find(mlq_gguf_t g, const char* name, uint64_t* index) {
    if (g == nullptr || name == nullptr || index == nullptr) {
        return fail(MLQ_ERR_INVALID, "mlq_hip_gguf_find: null argument");
    }
    const int64_t i = g->index.find(name);
    if (i < 0) return fail(MLQ_ERR_INVALID, std::string("Missing tensor: ") + name);
    *index = static_cast<uint64_t>(i);
    return MLQ_OK;
}

int mlq_hip_gguf_tensor_data(mlq_gguf_t g, uint64_t i, const void** data, uint64_t* nbytes) {
    if (g == nullptr || data == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_gguf_tensor_data: null argument");
    if (i >= g->index.tensors.size()) return fail(MLQ_ERR_INVALID, "mlq_hip_gguf_tensor_data: index out of range");
    const mlq::GgufTensor& t = g->index.tensors[i];
    *data = g->index.tensor_data(t);
    if (nbytes) *nbytes = t.nbytes;
    return MLQ_OK;
}

int mlq_hip_gguf_upload_weight(mlq_gguf_t g, const char* name, int device, mlq_weight_t* out) {
    if (out == nullptr) return fail(MLQ_ERR_INVALID, "HIP weight upload: null output handle");
    *out = nullptr;
    if (g == nullptr || name == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_gguf_upload_weight: null argument");
    const int64_t i = g->index.find(name);
    if (i < 0) return fail(MLQ_ERR_INVALID, std::string("Missing tensor: ") + name);
    const mlq::GgufTensor& t = g->index.tensors[static_cast<size_t>(i)];
    int qtype = 0;
    switch (t.type) {
        case mlq::kGgmlQ8_0: qtype = MLQ_Q8_0; break;
        case mlq::kGgmlQ4_0: qtype = MLQ_Q4_0; break;
        case mlq::kGgmlQ4_1: qtype = MLQ_Q4_1; break;
        default:
            return fail(MLQ_ERR_INVALID, std::string("HIP weight upload: ") + name + " is " +
                                             mlq::ggml_type_label(t.type) +
                                             "; only Q8_0, Q4_0 and Q4_1 linear weights are uploaded");
    }
    // A 2-D tensor [ne0, ne1] holds ne1 rows of ne0 values: W is [out = ne1, in = ne0].
    if (t.dims.size() != 2 || t.dims[0] > static_cast<uint64_t>(INT32_MAX) ||
        t.dims[1] > static_cast<uint64_t>(INT32_MAX)) {
        return fail(MLQ_ERR_SHAPE, std::string("HIP weight upload: expected 2D ") + type_name(qtype) + " weight");
    }
    const int M = static_cast<int>(t.dims[1]);
    const int K = static_cast<int>(t.dims[0]);
    const size_t bb = static_cast<size_t>(mlq::block_bytes(qtype));
    const size_t n_blocks = static_cast<size_t>(t.nbytes / bb);
    const int nb = (K + mlq::kQK - 1) / mlq::kQK;
    const size_t expected = static_cast<size_t>(M) * nb;
    if (n_blocks != expected) {
        return fail(MLQ_ERR_SHAPE, std::string("HIP weight upload: ") + type_name(qtype) +
                                       " block count mismatch, expected " + std::to_string(expected) + ", got " +
                                       std::to_string(n_blocks));
    }
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    void* ptr = nullptr;
    MLQ_HIP_CHECK(hipMalloc(&ptr, t.nbytes));
    if ((rc = upload_from_host(device, ptr, g->index.tensor_data(t), t.nbytes)) != MLQ_OK) {
        (void)hipFree(ptr);
        return rc;
    }
    *out = new mlq_weight_s{device, qtype, M, K, nb, n_blocks, ptr, true};
    return MLQ_OK;
}

int mlq_hip_decoder_open(const char* gguf_path, int device, int max_seq_len, mlq_decoder_t* out) {
    if (out == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_decoder_open: null output");
    *out = nullptr;
    if (gguf_path == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_decoder_open: null path");
    int rc = ensure_device(device);
    if (rc != MLQ_OK) return rc;
    try {
        std::unique_ptr<mlq::Decoder> d = mlq::Decoder::from_gguf(gguf_path, device, max_seq_len);
        *out = new mlq_decoder_s{std::move(d)};
    } catch (const std::exception& e) {
        return fail(MLQ_ERR_INVALID, e.what());
    }
    return MLQ_OK;
}

int mlq_hip_decoder_config(mlq_decoder_t d, mlq_decoder_config* out) {
    if (d == nullptr || out == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_decoder_config: null argument");
    const mlq::DecoderConfig& c = d->dec->config();
    *out = mlq_decoder_config{c.n_layers, c.dim, c.hidden_dim, c.n_heads, c.n_kv_heads, c.head_dim,
                              c.vocab_size, c.max_seq_len, c.rope_theta, c.rms_norm_eps, c.rope_neox};
    return MLQ_OK;
}

int mlq_hip_decoder_forward(mlq_decoder_t d, int token, int pos, float* logits) {
    if (d == nullptr || logits == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_decoder_forward: null argument");
    try {
        d->dec->forward(token, pos, logits);
    } catch (const std::out_of_range& e) {
        return fail(MLQ_ERR_SHAPE, e.what());
    } catch (const std::exception& e) {
        return fail(MLQ_ERR_INVALID, e.what());
    }
    return MLQ_OK;
}

int mlq_hip_decoder_prefill(mlq_decoder_t d, const int* tokens, int n, int start_pos, float* logits) {
    if (d == nullptr || tokens == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_decoder_prefill: null argument");
    try {
        d->dec->prefill(tokens, n, start_pos, logits);
    } catch (const std::out_of_range& e) {
        return fail(MLQ_ERR_SHAPE, e.what());
    } catch (const std::exception& e) {
        return fail(MLQ_ERR_INVALID, e.what());
    }
    return MLQ_OK;
}

int mlq_hip_decoder_generate(mlq_decoder_t d, const int* prompt, int n_prompt, int n_new, int* out_tokens) {
    if (d == nullptr || prompt == nullptr || (n_new > 0 && out_tokens == nullptr)) {
        return fail(MLQ_ERR_INVALID, "mlq_hip_decoder_generate: null argument");
    }
    try {
        d->dec->generate(prompt, n_prompt, n_new, out_tokens);
    } catch (const std::out_of_range& e) {
        return fail(MLQ_ERR_SHAPE, e.what());
    } catch (const std::exception& e) {
        return fail(MLQ_ERR_INVALID, e.what());
    }
    return MLQ_OK;
}

int mlq_hip_decoder_close(mlq_decoder_t d) {
    delete d;
    return MLQ_OK;
}

int mlq_hip_graph_capture_sequence(mlq_sequence_t seq, void* stream, mlq_graph_t* out) {
    if (out == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_graph_capture_sequence: null output");
    *out = nullptr;
    if (seq == nullptr) return fail(MLQ_ERR_INVALID, "mlq_hip_graph_capture_sequence: null sequence");
    int rc = ensure_device(seq->device);
    if (rc != MLQ_OK) return rc;
    hipStream_t s = resolve_stream(seq->device, stream);
    MLQ_HIP_CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    const int launch_rc = mlq_hip_sequence_launch(seq, s);
    return end_capture(s, seq->device, launch_rc, out);
}

}  // extern "C"

// Shared helpers of the drop-in: the reference's device-backend interfaces
// (include/mini_llama/cuda_*.h, backend.h) implemented on the MI355X HIP
// library through its C ABI (include/mlq_hip.h).  Nothing in the drop-in
// includes a HIP or CUDA header; every device operation is a C ABI call.
#pragma once

#include "mlq_hip.h"

#include <stdexcept>
#include <string>

namespace mini_llama {
namespace hipdrop {

// The device the calling thread selected last (cudaSetDevice's per-thread
// current device, src/cuda_runtime.cpp:187-218).
int& current_device();

[[noreturn]] inline void throw_hip(const std::string& what) {
    throw std::runtime_error("HIP runtime error in " + what + ": " + mlq_hip_last_error());
}

inline void check(int rc, const char* what) {
    if (rc != MLQ_OK) throw_hip(what);
}

// The library's stream of `device`: every launch of the drop-in is issued
// there, in call order, so a kernel always sees the buffers written by the
// calls before it.
inline void* stream_of(int device) {
    void* s = nullptr;
    check(mlq_hip_stream(device, &s), "mlq_hip_stream");
    return s;
}

// Waits for everything issued on `device`'s library stream (the reference's
// calls return after their kernels finish).
inline void sync_device(int device) { check(mlq_hip_synchronize(stream_of(device)), "mlq_hip_synchronize"); }

// A C ABI failure as the reference's std::runtime_error, prefixed with the
// reference function's name unless the library's message already carries one.
[[noreturn]] inline void throw_op(const char* caller) {
    const std::string msg = mlq_hip_last_error();
    if (msg.rfind(caller, 0) == 0) throw std::runtime_error(msg);
    throw std::runtime_error(std::string(caller) + ": " + msg);
}

}  // namespace hipdrop
}  // namespace mini_llama

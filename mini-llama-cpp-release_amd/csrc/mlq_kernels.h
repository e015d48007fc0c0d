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

// Batched prefill GEMM for rows > 1 (MFMA).  Needs a device workspace of
// gemm_workspace_bytes(s) bytes (split x, scales, split-K partials) that no
// other launch uses concurrently.  Returns hipErrorNotSupported when the shape
// has no MFMA path (the caller runs the GEMV kernels per row instead).
bool gemm_supported(const LinearShape& s);
size_t gemm_workspace_bytes(const LinearShape& s);
hipError_t launch_gemm(const LinearShape& s, const void* w, const float* x, float* y, void* ws,
                       size_t ws_bytes, hipStream_t stream);
const char* gemm_kernel_name(const LinearShape& s);

// Device quantizer and synthetic-data generator.
hipError_t launch_quantize(int qtype, const float* src, int rows, int row_len, void* dst,
                           hipStream_t stream);
hipError_t launch_fill_normal(float* dst, size_t n, uint64_t seed, float mean, float stddev,
                              hipStream_t stream);

}  // namespace mlq

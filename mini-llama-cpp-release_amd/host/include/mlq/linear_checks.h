// Shape checks and the host bias add of a quantized linear call, shared by
// the two C++ layers over the C ABI: the mlq:: host layer (host/src/hip_quant.cpp)
// and the drop-in of the reference's device interface (dropin/hip_quant.cpp).
//
// Order and texts of the reference's checks, src/cuda_quant.cu:150-243:
// W 2-D, x 1-D or 2-D, no empty extents, in_features equal, block count
// rows * ceil(in / 32); then the bias of src/cuda_quant.cu:139-148.
// Header-only and plain C++17 (no HIP types), so either layer compiles it
// with the host compiler.
#pragma once

#include <cstddef>
#include <stdexcept>
#include <string>
#include <vector>

namespace mlq {
namespace checks {

inline int in_features_of(const std::vector<int>& xs, const std::string& xstr, const char* caller) {
    if (xs.size() == 1) return xs[0];
    if (xs.size() == 2) return xs[1];
    throw std::runtime_error(std::string(caller) + ": expected x shape [in_features] or [batch, in_features], got " +
                             xstr);
}

inline void linear_shape(const std::vector<int>& xs, const std::string& xstr, const std::vector<int>& ws,
                         size_t block_count, const char* caller) {
    if (ws.size() != 2) {
        throw std::runtime_error(std::string(caller) + ": expected W shape [out_features, in_features]");
    }
    const int in = in_features_of(xs, xstr, caller);
    if (in <= 0 || ws[0] <= 0 || ws[1] <= 0) {
        throw std::runtime_error(std::string(caller) + ": empty tensors are not supported");
    }
    if (ws[1] != in) {
        throw std::runtime_error(std::string(caller) + ": dimension mismatch x=" + xstr + " W=[" +
                                 std::to_string(ws[0]) + ", " + std::to_string(ws[1]) + "]");
    }
    const size_t expected = static_cast<size_t>(ws[0]) * static_cast<size_t>((in + 31) / 32);
    if (block_count != expected) {
        throw std::runtime_error(std::string(caller) + ": block count mismatch: expected " +
                                 std::to_string(expected) + ", got " + std::to_string(block_count));
    }
}

// y [rows][cols] += bias [cols] on the host, after the download.
inline void add_bias(float* y, const std::vector<int>& bias_shape, const float* bias, int rows, int cols,
                     const char* caller) {
    if (bias_shape.size() != 1 || bias_shape[0] != cols) {
        throw std::runtime_error(std::string(caller) + ": expected bias shape [out_features]");
    }
    for (int r = 0; r < rows; ++r) {
        for (int c = 0; c < cols; ++c) y[static_cast<size_t>(r) * cols + c] += bias[c];
    }
}

}  // namespace checks
}  // namespace mlq

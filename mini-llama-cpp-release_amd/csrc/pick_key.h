// Ordering key of a greedy pick (argmax of y, first index on ties), shared by
// the fused lm_head pick and the decoder's pick over F32 logits.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mlq {

// A row's key orders by value, then by lower row: the float's bits mapped to
// an unsigned order (-0 taken as +0, since the two compare equal) above the
// complemented row.  A value that is not finite gives the all-ones key, which
// decodes to -1.
__device__ __forceinline__ unsigned long long pick_key(float v, int row) {
    uint32_t b = __builtin_bit_cast(uint32_t, v);
    if ((b & 0x7F800000u) == 0x7F800000u) return ~0ull;
    b = b == 0x80000000u ? 0u : b;
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return (static_cast<unsigned long long>(ord) << 32) | static_cast<uint32_t>(~static_cast<uint32_t>(row));
}

__device__ __forceinline__ int32_t pick_token(unsigned long long k) {
    return k == ~0ull ? -1 : static_cast<int32_t>(~static_cast<uint32_t>(k));
}

}  // namespace mlq

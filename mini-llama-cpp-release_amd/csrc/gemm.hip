// Batched prefill GEMM (rows > 1).  The MFMA kernel is not in this file yet;
// until it is, batched calls run the GEMV kernels once per x row.
#include "mlq_kernels.h"

namespace mlq {

bool gemm_supported(const LinearShape&) { return false; }

hipError_t launch_gemm(const LinearShape&, const void*, const float*, float*, hipStream_t) {
    return hipErrorNotSupported;
}

const char* gemm_kernel_name(const LinearShape&) { return "none"; }

}  // namespace mlq

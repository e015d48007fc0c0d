// Backend selection with `--backend hip` (src/backend.cpp:8-79 plus the CLI
// messages of src/main.cpp:560-568 and scripts/test_backend_cli.py:58-113).
#include "mlq/backend.h"

#include "mlq/hip_runtime.h"
#include "mlq_hip.h"

#include <stdexcept>

namespace mlq {

bool parse_backend_kind(const std::string& text, BackendKind& kind) {
    if (text == "cpu") {
        kind = BackendKind::Cpu;
        return true;
    }
    if (text == "cuda") {
        kind = BackendKind::Cuda;
        return true;
    }
    if (text == "hip") {
        kind = BackendKind::Hip;
        return true;
    }
    return false;
}

std::string backend_kind_name(BackendKind kind) {
    switch (kind) {
        case BackendKind::Cpu: return "cpu";
        case BackendKind::Cuda: return "cuda";
        case BackendKind::Hip: return "hip";
    }
    return "unknown";
}

bool hip_backend_built() { return hip_runtime_built(); }

bool hip_backend_available(int device_id) {
    int n = 0;
    if (mlq_hip_device_count(&n) != MLQ_OK) return false;
    return device_id >= 0 && device_id < n;
}

void validate_backend(const BackendConfig& config) {
    if (config.kind == BackendKind::Cpu) {
        if (config.device_id_set) {
            throw std::runtime_error("--device can only be used with --backend hip.");
        }
        return;
    }
    if (config.kind == BackendKind::Hip) {
        if (!hip_backend_built()) {
            throw std::runtime_error("HIP backend was not built. Build libmlq_hip.so for gfx950 with hipcc.");
        }
        if (!hip_backend_available(config.device_id)) {
            throw std::runtime_error("HIP device " + std::to_string(config.device_id) +
                                     " is not available: " + hip_device_summary(config.device_id));
        }
        return;
    }
    if (config.kind == BackendKind::Cuda) {
        throw std::runtime_error("CUDA backend was not built. This build targets HIP (--backend hip).");
    }
    throw std::runtime_error("unknown backend");
}

std::string backend_execution_note(const BackendConfig& config) {
    if (config.kind == BackendKind::Cpu) return "compute: cpu";
    if (config.kind == BackendKind::Hip) {
        return "compute: hip quantized linear (Q8_0/Q4_0/Q4_1, gfx950 GEMV and MFMA GEMM kernels)";
    }
    return "compute: cuda";
}

std::string invalid_backend_message() { return "Invalid --backend value. Supported values: cpu, cuda, hip."; }

std::string invalid_device_message() { return "Invalid --device value. Expected a non-negative integer."; }

}  // namespace mlq

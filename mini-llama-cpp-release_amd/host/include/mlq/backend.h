// Backend selection with the HIP backend added (include/mini_llama/backend.h:7-29,
// src/backend.cpp:8-79).  `--backend hip` parses to BackendKind::Hip; the CUDA
// kind is kept so the enum stays a superset of the reference's.
#pragma once

#include <string>

namespace mlq {

enum class BackendKind { Cpu, Cuda, Hip };

struct BackendConfig {
    BackendKind kind = BackendKind::Cpu;
    int device_id = 0;
    bool device_id_set = false;
};

bool parse_backend_kind(const std::string& text, BackendKind& kind);
std::string backend_kind_name(BackendKind kind);

bool hip_backend_built();
bool hip_backend_available(int device_id = 0);

// Throws when the requested backend cannot run in this build or on this host.
void validate_backend(const BackendConfig& config);

// Explains which execution path is active.
std::string backend_execution_note(const BackendConfig& config);

// The CLI's messages for bad flag values (src/main.cpp:562, 567).
std::string invalid_backend_message();
std::string invalid_device_message();

}  // namespace mlq

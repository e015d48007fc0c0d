// C++ parity test of the HIP quantized linear, laid out like the reference's
// tests/test_cuda_quant.cpp: the same deterministic pattern tensors (:51-58),
// the same shapes ({5,13} + bias, {32,64} with x [3,64], {17,65} for Q4_1,
// :293-420), the same closeness rule (abs <= 1e-3 or rel <= 1e-3 against
// max(1, |y|), :23-36), and all three call forms (host weight, device weight,
// device input).  The expected values come from the CPU oracle (oracle/oracle.cpp,
// linked into this test only).
//
//   test_hip_quant cpu       backend selection, shape validation, no device needed
//   test_hip_quant q8_0|q4|forms|all   parity on device 0
#include "mlq/backend.h"
#include "mlq/hip_quant.h"

#include <cmath>
#include <cstring>
#include <iostream>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

extern "C" {
long long mlq_oracle_quantize(int qtype, const float* src, int rows, int row_len, void* out, int threads);
int mlq_oracle_linear(int qtype, const float* x, int rows, int K, const void* blocks, size_t n_blocks, int M,
                      float* y, int threads, char* err, size_t err_len);
}

using namespace mlq;

namespace {

void require(bool ok, const std::string& msg) {
    if (!ok) throw std::runtime_error(msg);
}

bool close_enough(float actual, float expected) {
    const float abs_err = std::fabs(actual - expected);
    const float scale = std::max(1.0f, std::fabs(expected));
    return abs_err <= 1e-3f || abs_err / scale <= 1e-3f;
}

void require_close(const Tensor& actual, const Tensor& expected, const std::string& label) {
    require(actual.shape == expected.shape, label + ": shape mismatch");
    for (size_t i = 0; i < actual.size(); ++i) {
        if (!close_enough(actual.data[i], expected.data[i])) {
            throw std::runtime_error(label + ": value mismatch at " + std::to_string(i) + ", actual=" +
                                     std::to_string(actual.data[i]) + ", expected=" + std::to_string(expected.data[i]));
        }
    }
}

Tensor pattern(const std::vector<int>& shape, float scale, float shift) {
    Tensor t(shape);
    for (size_t i = 0; i < t.size(); ++i) {
        const int bucket = static_cast<int>((i * 19 + 7) % 31);
        t.data[i] = static_cast<float>(bucket - 15) * scale + shift;
    }
    return t;
}

template <typename Block>
std::vector<Block> quantize(QuantType t, const Tensor& w) {
    const int k = w.shape.back();
    const int rows = static_cast<int>(w.size()) / k;
    std::vector<Block> out(static_cast<size_t>(rows) * ((k + 31) / 32));
    require(mlq_oracle_quantize(static_cast<int>(t), w.data.data(), rows, k, out.data(), 1) ==
                static_cast<long long>(out.size()),
            "oracle quantize failed");
    return out;
}

template <typename Block>
Tensor cpu_linear(QuantType t, const Tensor& x, const std::vector<Block>& w, const std::vector<int>& ws) {
    const int k = ws[1];
    const int rows = static_cast<int>(x.size()) / k;
    Tensor y(x.ndim() == 1 ? std::vector<int>{ws[0]} : std::vector<int>{rows, ws[0]});
    char err[256];
    require(mlq_oracle_linear(static_cast<int>(t), x.data.data(), rows, k, w.data(), w.size(), ws[0],
                              y.data.data(), 1, err, sizeof err) == 0,
            err);
    return y;
}

template <typename Block, typename HostFn, typename DevWFn, typename DevInFn>
void check_format(QuantType t, const char* name, const std::vector<int>& w2shape, HostFn host_fn,
                  DevWFn devw_fn, DevInFn devin_fn) {
    Tensor w1 = pattern({5, 13}, 0.037f, -0.11f);
    Tensor x1 = pattern({13}, 0.071f, 0.03f);
    Tensor b1 = pattern({5}, 0.013f, -0.02f);
    auto q1 = quantize<Block>(t, w1);
    Tensor expected1 = cpu_linear(t, x1, q1, w1.shape);
    require_close(host_fn(x1, q1, w1.shape, nullptr, 0), expected1, std::string(name) + " 1D no bias");
    Tensor expected_bias = expected1;
    for (int i = 0; i < 5; ++i) expected_bias.data[i] += b1.data[i];
    require_close(host_fn(x1, q1, w1.shape, &b1, 0), expected_bias, std::string(name) + " 1D bias");

    Tensor w2 = pattern(w2shape, 0.019f, 0.04f);
    Tensor x2 = pattern({3, w2shape[1]}, 0.029f, -0.06f);
    auto q2 = quantize<Block>(t, w2);
    Tensor expected2 = cpu_linear(t, x2, q2, w2.shape);
    require_close(host_fn(x2, q2, w2.shape, nullptr, 0), expected2, std::string(name) + " 2D batch");

    HipDeviceBuffer wd(q2.size() * sizeof(Block), 0);
    wd.upload(q2.data(), q2.size() * sizeof(Block));
    require_close(devw_fn(x2, wd.data(), q2.size(), w2.shape, nullptr, 0), expected2,
                  std::string(name) + " device weight");
    HipTensor xd = hip_tensor_from_host(x2, 0);
    require_close(devin_fn(xd, wd.data(), q2.size(), w2.shape, 0).download(), expected2,
                  std::string(name) + " device input");

    // validation mirrors src/cuda_quant.cu:214-243
    bool threw = false;
    try {
        (void)devw_fn(x2, wd.data(), q2.size() - 1, w2.shape, nullptr, 0);
    } catch (const std::exception& e) {
        threw = std::string(e.what()).find("block count mismatch: expected") != std::string::npos;
    }
    require(threw, std::string(name) + ": block count mismatch not reported");
    threw = false;
    try {
        (void)devw_fn(x2, nullptr, q2.size(), w2.shape, nullptr, 0);
    } catch (const std::exception& e) {
        threw = std::string(e.what()).find("device weight pointer is null") != std::string::npos;
    }
    require(threw, std::string(name) + ": null weight not reported");
}

void test_cpu_side() {
    BackendKind k;
    require(parse_backend_kind("hip", k) && k == BackendKind::Hip, "parse hip");
    require(parse_backend_kind("cpu", k) && k == BackendKind::Cpu, "parse cpu");
    require(!parse_backend_kind("metal", k), "metal must be rejected");
    require(invalid_backend_message().find("Invalid --backend value") == 0, "invalid backend message");
    require(invalid_device_message().find("Invalid --device value") == 0, "invalid device message");
    BackendConfig cfg;
    cfg.device_id_set = true;
    bool threw = false;
    try {
        validate_backend(cfg);
    } catch (const std::exception& e) {
        threw = std::string(e.what()) == "--device can only be used with --backend hip.";
    }
    require(threw, "cpu backend must reject --device");
    require(backend_execution_note(BackendConfig{}) == "compute: cpu", "cpu note");
    BackendConfig hip_cfg;
    hip_cfg.kind = BackendKind::Hip;
    require(backend_execution_note(hip_cfg).find("compute: hip quantized linear") == 0, "hip note");
    require(hip_quant_built(), "HIP kernels must be built into libmlq_hip.so");
    // host-side shape validation answers before any device work
    Tensor x({3, 7});
    std::vector<BlockQ4_0> w(4);
    threw = false;
    try {
        (void)hip_q4_0_linear(x, w, {4, 8});
    } catch (const std::exception& e) {
        threw = std::string(e.what()) == "hip_q4_0_linear: dimension mismatch x=[3, 7] W=[4, 8]";
    }
    require(threw, "dimension mismatch message");
    threw = false;
    try {
        (void)hip_q8_0_linear(Tensor({2, 2, 2}), std::vector<BlockQ8_0>(1), {1, 2});
    } catch (const std::exception& e) {
        threw = std::string(e.what()).find("expected x shape [in_features] or [batch, in_features]") !=
                std::string::npos;
    }
    require(threw, "rank message");
    threw = false;
    try {
        (void)Tensor({0});
    } catch (const std::runtime_error&) {
        threw = true;
    }
    require(threw, "zero dimension must be rejected");
}

void test_forms() {
    // forward_linear_device-style use: upload once, call on a device input
    Tensor w = pattern({300, 4096}, 0.0007f, 0.0001f);
    QuantizedTensor qt;
    qt.type = QuantType::Q4_0;
    qt.shape = w.shape;
    qt.q4_0_data = quantize<BlockQ4_0>(QuantType::Q4_0, w);
    HipUploadedWeight up = hip_upload_linear_weight(qt, "layers.0.wq", 0);
    Tensor x = pattern({4096}, 0.05f, 0.01f);
    Tensor expected = cpu_linear(QuantType::Q4_0, x, qt.q4_0_data, qt.shape);
    HipTensor xd = hip_tensor_from_host(x, 0);
    require_close(hip_linear_device(xd, up, 0).download(), expected, "uploaded weight forward");
    QuantizedTensor bad = qt;
    bad.q4_0_data.pop_back();
    bool threw = false;
    try {
        (void)hip_upload_linear_weight(bad, "layers.0.wk", 0);
    } catch (const std::exception& e) {
        threw = std::string(e.what()).find("HIP weight upload: Q4_0 block count mismatch for layers.0.wk") == 0;
    }
    require(threw, "upload block count message");

    // Greedy sampling on the device (compute_logits_device + sample_greedy):
    // the first maximum of the logits, and the sampler's error on Inf/NaN.
    Tensor wl = pattern({1000, 4096}, 0.0009f, 0.0003f);
    QuantizedTensor lm;
    lm.type = QuantType::Q4_0;
    lm.shape = wl.shape;
    lm.q4_0_data = quantize<BlockQ4_0>(QuantType::Q4_0, wl);
    HipUploadedWeight lmw = hip_upload_linear_weight(lm, "lm_head", 0);
    Tensor logits = hip_linear_device(xd, lmw, 0).download();
    int first_max = 0;
    for (size_t i = 1; i < logits.data.size(); ++i) {
        if (logits.data[i] > logits.data[first_max]) first_max = static_cast<int>(i);
    }
    const int token = hip_sample_greedy_device(xd, lmw, 0);
    require(token == first_max, "greedy token is the first maximum of the device logits");
    Tensor cpu_logits = cpu_linear(QuantType::Q4_0, x, lm.q4_0_data, lm.shape);
    float cpu_max = cpu_logits.data[0];
    for (float v : cpu_logits.data) cpu_max = v > cpu_max ? v : cpu_max;
    require(cpu_max - cpu_logits.data[token] <= 1e-3f * (1.0f + std::fabs(cpu_max)),
            "greedy token is a maximum of the CPU logits within tolerance");
    Tensor xinf = x;
    xinf.data[3] = std::numeric_limits<float>::infinity();
    HipTensor xinf_d = hip_tensor_from_host(xinf, 0);
    threw = false;
    try {
        (void)hip_sample_greedy_device(xinf_d, lmw, 0);
    } catch (const std::exception& e) {
        threw = std::string(e.what()) == "sampler: logits must be finite";
    }
    require(threw, "non-finite logits message");
}

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc >= 2 ? argv[1] : "all";
    try {
        test_cpu_side();
        if (mode == "cpu") {
            std::cout << "PASS hip_quant_cpu_side\n";
            return 0;
        }
        validate_backend(BackendConfig{BackendKind::Hip, 0, true});
        if (mode == "q8_0" || mode == "all") {
            check_format<BlockQ8_0>(QuantType::Q8_0, "hip_q8_0_linear", {32, 64}, hip_q8_0_linear,
                                    hip_q8_0_linear_device_weight, hip_q8_0_linear_device_input);
            std::cout << "PASS hip_quant_q8_0\n";
        }
        if (mode == "q4" || mode == "all") {
            check_format<BlockQ4_0>(QuantType::Q4_0, "hip_q4_0_linear", {32, 64}, hip_q4_0_linear,
                                    hip_q4_0_linear_device_weight, hip_q4_0_linear_device_input);
            check_format<BlockQ4_1>(QuantType::Q4_1, "hip_q4_1_linear", {17, 65}, hip_q4_1_linear,
                                    hip_q4_1_linear_device_weight, hip_q4_1_linear_device_input);
            std::cout << "PASS hip_quant_q4\n";
        }
        if (mode == "forms" || mode == "all") {
            test_forms();
            std::cout << "PASS hip_quant_forms\n";
        }
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "FAIL " << mode << ": " << e.what() << "\n";
        return 1;
    }
}

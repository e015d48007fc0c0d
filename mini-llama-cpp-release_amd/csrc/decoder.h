// Device-resident decode step of a llama / qwen2 model over the quantized
// linears (internal interface between decoder.hip and mlq_abi.hip).
//
// Mirrors forward_token (src/forward.cpp:865-903) with every op on the
// device: embedding lookup, per layer RMSNorm -> q/k/v (+ bias) -> RoPE ->
// KV-cache write -> attention -> o -> residual -> RMSNorm -> gate/up ->
// SwiGLU -> down -> residual, then the final RMSNorm and the lm_head.  The
// token and position a step uses live in device memory, so one step is a
// fixed sequence of launches that can be recorded once and replayed per
// token, with the greedy pick of one step feeding the next.
#pragma once

#include "mlq_kernels.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace mlq {

struct DecoderConfig {
    int n_layers = 0;
    int dim = 0;
    int hidden_dim = 0;
    int n_heads = 0;
    int n_kv_heads = 0;
    int head_dim = 0;
    int vocab_size = 0;
    int max_seq_len = 0;
    float rope_theta = 10000.0f;
    float rms_norm_eps = 1e-5f;
    int rope_neox = 0;  // RopeType::NeoX (general.architecture == "qwen2")
};

// State words of one decoder in device memory.
struct DecodeState {
    int32_t pos;     // position of the step about to run
    int32_t token;   // its input token
    int32_t next;    // greedy pick of the last step (-1: a logit was not finite)
    int32_t error;   // bit 0: token out of range, 1: position out of range, 2: non-finite logits
    int32_t n_prompt;
    int32_t n_out;
    int32_t pad[2];
};

constexpr int kDecodeErrToken = 1;
constexpr int kDecodeErrPos = 2;
constexpr int kDecodeErrLogits = 4;

class Decoder {
public:
    // Loads a model the way load_gguf_model does (src/gguf_loader.cpp:320-456:
    // config from metadata, tensor names, F32 norms / embedding / biases with
    // quantized ones dequantized, tied lm_head) and places it on `device`.
    // max_seq_len > 0 bounds the KV cache below the model's context length.
    // Throws std::runtime_error with the loader's messages.
    static std::unique_ptr<Decoder> from_gguf(const std::string& path, int device, int max_seq_len);
    ~Decoder();

    const DecoderConfig& config() const { return cfg_; }
    int device() const { return device_; }

    // forward_token with ctx.pos = pos: logits [vocab] to host memory.
    void forward(int token, int pos, float* logits_host);
    // Greedy generation: the prompt at positions 0..n_prompt-1, then n_new
    // tokens each picked from the previous step's logits (first maximum) and
    // fed back on the device.  One upload, one download, no host work per
    // token.  Throws on a device-side error (bad prompt token, position past
    // the cache, non-finite logits).
    void generate(const int* prompt, int n_prompt, int n_new, int* out);
    // forward_batch (src/batch.cpp:33-52) over tokens at positions
    // start..start+n-1, all rows of a layer at once (the MFMA GEMM for the
    // linears); logits of the last token to host memory (when not null).
    void prefill(const int* tokens, int n, int start, float* logits_host);

    // Rows per batched pass: the GEMM at 512 token rows does 17 % more work per
    // µs than at 256 (4096 x 4096 Q4_0: 66.8 against 2 x 40.1 us).
    static constexpr int kPrefillRows = 512;

private:
    Decoder() = default;
    void enqueue_step(hipStream_t s, bool pick, bool advance);
    void check(hipError_t e, const char* what);

    struct Linear {
        int qtype = 0;   // 0 = F32 [M][K] floats, else MLQ_Q8_0 / Q4_0 / Q4_1 blocks
        int M = 0;
        int K = 0;
        void* data = nullptr;
    };
    struct Layer {
        float* attn_norm = nullptr;
        float* ffn_norm = nullptr;
        float* bq = nullptr;
        float* bk = nullptr;
        float* bv = nullptr;
        Linear wq, wk, wv, wo, w_gate, w_up, w_down;
    };

    void linear_group(hipStream_t s, const Linear* const* ws, float* const* ys, int n, const float* x);
    bool launch_attention_rope(hipStream_t s, int layer);
    void launch_norm(hipStream_t s, const float* delta, const float* w);
    void linear_rows(hipStream_t s, const Linear& w, const float* X, float* Y, int rows);
    // Up to three linears over the same X (q/k/v, gate/up) as one grouped GEMM
    // launch when the shapes allow it, else one linear_rows each.
    void linear_rows_group(hipStream_t s, int n, const Linear* const* w, const float* X, float* const* Y, int rows);
    void ensure_workspace(hipStream_t s, size_t need);
    // A prefill GEMM (1-3 linears over one x) whose producer writes the split
    // x straight into the workspace (gemm_split_x).
    struct SplitTarget {
        int ng = 0;
        const void* w[3] = {};
        int M[3] = {};
        LinearShape shape{};
        GemmSplitX sx{};
    };
    bool split_target(int ng, const Linear* const* w, int rows, SplitTarget& t) const;
    void gemm_split(hipStream_t s, const SplitTarget& t, float* const* Y);
    void norm_into(hipStream_t s, const SplitTarget* t, float* X, const float* D, const float* w, int n);
    void linear_fused(hipStream_t s, const Linear* const* ws, float* const* ys, int n, const float* x,
                      const float* norm_w, bool acc);
    void enqueue_prefill(hipStream_t s, const int32_t* tokens, int n, int start);
    bool prefill_batched() const;
    void ensure_prefill();
    void ensure_io(size_t need);

    DecoderConfig cfg_;
    int device_ = 0;
    hipStream_t stream_ = nullptr;
    std::vector<void*> allocs_;
    float* embedding_ = nullptr;  // [vocab][dim]
    float* final_norm_ = nullptr;
    Linear lm_head_;
    std::vector<Layer> layers_;
    // Activations and cache.
    float *x_ = nullptr, *h_ = nullptr, *q_ = nullptr, *k_ = nullptr, *v_ = nullptr, *att_ = nullptr;
    float *proj_ = nullptr, *gate_ = nullptr, *up_ = nullptr, *act_ = nullptr, *ff_ = nullptr;
    float* logits_ = nullptr;
    float* scores_ = nullptr;    // [n_heads][max_seq_len]
    float* kcache_ = nullptr;    // [n_layers][max_seq_len][n_kv_heads][head_dim]
    float* vcache_ = nullptr;
    DecodeState* state_ = nullptr;
    int32_t* io_ = nullptr;      // prompt tokens then generated tokens
    size_t io_cap_ = 0;
    void* pick_ = nullptr;       // PickState
    float* attn_part_ = nullptr;     // [n_heads][attn_splits_][head_dim + 2]: split attention states
    unsigned* attn_cnt_ = nullptr;   // [n_heads] arrival counts of the split attention
    int attn_splits_ = 1;
    // Batched prefill: activations of kPrefillRows rows and the GEMM workspace.
    float *X_ = nullptr, *H_ = nullptr, *Q_ = nullptr, *K_ = nullptr, *V_ = nullptr, *ATT_ = nullptr;
    float *PROJ_ = nullptr, *GATE_ = nullptr, *UP_ = nullptr, *ACT_ = nullptr, *FF_ = nullptr;
    void* ws_ = nullptr;
    size_t ws_bytes_ = 0;
    hipGraphExec_t graph_ = nullptr;
    // generate() keeps at most kGenerateInflight recorded steps queued: the
    // event after step i is waited for before step i + kGenerateInflight.
    static constexpr int kGenerateInflight = 8;
    hipEvent_t inflight_[kGenerateInflight] = {};
};

}  // namespace mlq

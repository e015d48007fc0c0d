// mlq reference shim -- TEST INFRASTRUCTURE ONLY.
//
// A C-ABI over the reference's own CPU quant functions, compiled by
// oracle/Makefile (target `ref`) from the sources where they lie under
// /root/reference, into oracle/_ref/libmlq_ref.so.  It exists to (1) generate
// the golden vectors in tests/golden/ and (2) serve as the "reference" CPU
// baseline in bench.py.  The product never links it.
//
// Nothing from the reference is copied here: the reference headers are found
// through -I at build time, and the Q4_1 quantizer, which exists only as a
// test-local function in tests/test_cuda_quant.cpp:129-180, is reached by
// including that test's translation unit (with its main() renamed) below.

#define main mlq_ref_unused_test_main
#include "tests/test_cuda_quant.cpp"
#undef main

#include "mini_llama/context.h"
#include "mini_llama/forward.h"
#include "mini_llama/gguf.h"
#include "mini_llama/sampler.h"
#include "mini_llama/gguf_loader.h"
#include "mini_llama/model.h"
#include "mini_llama/ops.h"
#include "mini_llama/quant.h"
#include "mini_llama/thread_pool.h"

#include <cstdio>
#include <memory>
#include <cstring>
#include <string>
#include <vector>

namespace {

using namespace mini_llama;

Tensor make_tensor(const float* src, int rows, int cols, bool as_1d) {
    Tensor t(as_1d ? std::vector<int>{cols} : std::vector<int>{rows, cols}, 0.0f);
    std::memcpy(t.data.data(), src, sizeof(float) * t.data.size());
    return t;
}

template <typename Block>
std::vector<Block> blocks_from(const void* src, size_t n) {
    std::vector<Block> v(n);
    std::memcpy(v.data(), src, n * sizeof(Block));
    return v;
}

}  // namespace

extern "C" {

// The reference fp16 encoders are file-local; they are observed through
// one-element blocks.  A one-element Q4_1 block has range 0, so its m field is
// exactly fp16(v) from the test copy of the codec (tests/test_cuda_quant.cpp:60-96,
// identical to src/quant.cpp:19-55) for every v except +Inf and NaN, which that
// routine maps to 0.  A one-element Q8_0 block has d = fp16(|v| / 127) from the
// product copy (src/quant.cpp:141-142).
uint16_t mlq_ref_fp16_probe_q4_1(float v) {
    Tensor t({1}, v);
    std::vector<BlockQ4_1> b = quantize_to_q4_1_for_test(t);
    return b.empty() ? 0 : b[0].m;
}

uint16_t mlq_ref_fp16_probe_q8_0(float v) {
    Tensor t({1}, v);
    std::vector<BlockQ8_0> b = quantize_to_q8_0(t);
    return b.empty() ? 0 : b[0].d;
}

long long mlq_ref_quantize(int qtype, const float* src, int rows, int row_len, void* out) {
    Tensor t = make_tensor(src, rows, row_len, rows == 1);
    size_t n = 0;
    if (qtype == 1) {
        std::vector<BlockQ8_0> b = quantize_to_q8_0(t);
        n = b.size();
        std::memcpy(out, b.data(), n * sizeof(BlockQ8_0));
    } else if (qtype == 2) {
        std::vector<BlockQ4_0> b = quantize_to_q4_0(t);
        n = b.size();
        std::memcpy(out, b.data(), n * sizeof(BlockQ4_0));
    } else if (qtype == 3) {
        std::vector<BlockQ4_1> b = quantize_to_q4_1_for_test(t);
        n = b.size();
        std::memcpy(out, b.data(), n * sizeof(BlockQ4_1));
    } else {
        return -1;
    }
    return static_cast<long long>(n);
}

int mlq_ref_dequantize(int qtype, const void* blocks, int rows, int row_len, float* dst) {
    const int nb = (row_len + 31) / 32;
    const size_t n = static_cast<size_t>(rows) * nb;
    std::vector<int> shape = rows == 1 ? std::vector<int>{row_len} : std::vector<int>{rows, row_len};
    Tensor y;
    if (qtype == 1) {
        y = dequantize_from_q8_0(blocks_from<BlockQ8_0>(blocks, n), shape);
    } else if (qtype == 2) {
        y = dequantize_from_q4_0(blocks_from<BlockQ4_0>(blocks, n), shape);
    } else if (qtype == 3) {
        y = dequantize_from_q4_1(blocks_from<BlockQ4_1>(blocks, n), shape);
    } else {
        return -1;
    }
    std::memcpy(dst, y.data.data(), y.data.size() * sizeof(float));
    return 0;
}

// y = linear(x, W) through the reference's dispatch (src/ops.cpp:197-209) with
// the global thread count set to `threads` (src/thread_pool.cpp:19-21).
int mlq_ref_linear(int qtype, const float* x, int rows, int K, const void* blocks,
                   size_t n_blocks, int M, float* y, int threads, char* err, size_t err_len) {
    try {
        set_thread_count(threads);
        QuantizedTensor w;
        w.shape = {M, K};
        if (qtype == 1) {
            w.type = QuantType::Q8_0;
            w.q8_0_data = blocks_from<BlockQ8_0>(blocks, n_blocks);
        } else if (qtype == 2) {
            w.type = QuantType::Q4_0;
            w.q4_0_data = blocks_from<BlockQ4_0>(blocks, n_blocks);
        } else if (qtype == 3) {
            w.type = QuantType::Q4_1;
            w.q4_1_data = blocks_from<BlockQ4_1>(blocks, n_blocks);
        } else {
            throw std::runtime_error("mlq_ref_linear: unsupported type");
        }
        Tensor xt = make_tensor(x, rows, K, rows == 1);
        Tensor out = linear(xt, w);
        std::memcpy(y, out.data.data(), out.data.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        if (err != nullptr && err_len > 0) std::snprintf(err, err_len, "%s", e.what());
        return -1;
    }
}

// Same, but with the caller's blocks borrowed for many calls: the weight is
// wrapped once so that timing loops measure only linear().
void* mlq_ref_weight_new(int qtype, const void* blocks, size_t n_blocks, int M, int K) {
    QuantizedTensor* w = new QuantizedTensor();
    w->shape = {M, K};
    if (qtype == 1) {
        w->type = QuantType::Q8_0;
        w->q8_0_data = blocks_from<BlockQ8_0>(blocks, n_blocks);
    } else if (qtype == 2) {
        w->type = QuantType::Q4_0;
        w->q4_0_data = blocks_from<BlockQ4_0>(blocks, n_blocks);
    } else if (qtype == 3) {
        w->type = QuantType::Q4_1;
        w->q4_1_data = blocks_from<BlockQ4_1>(blocks, n_blocks);
    } else {
        delete w;
        return nullptr;
    }
    return w;
}

void mlq_ref_weight_free(void* w) { delete static_cast<QuantizedTensor*>(w); }

int mlq_ref_weight_linear(void* w, const float* x, int rows, float* y, int threads) {
    try {
        set_thread_count(threads);
        QuantizedTensor* qt = static_cast<QuantizedTensor*>(w);
        Tensor xt = make_tensor(x, rows, qt->shape[1], rows == 1);
        Tensor out = linear(xt, *qt);
        std::memcpy(y, out.data.data(), out.data.size() * sizeof(float));
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int mlq_ref_argmax(const float* v, int n) {
    Tensor t({n}, 0.0f);
    std::memcpy(t.data.data(), v, sizeof(float) * n);
    return argmax(t);
}

int mlq_ref_hardware_threads(void) {
    set_thread_count(0);
    return get_thread_count();
}

// ---- GGUF: the reference reader (src/gguf.cpp) and loader (src/gguf_loader.cpp)

// Parses `path` with GGUFReader::load; the reader is returned whether or not
// the load succeeded (*ok), so its fields and load_error can be read back.
void* mlq_ref_gguf_load(const char* path, int* ok) {
    GGUFReader* r = new GGUFReader;
    *ok = r->load(path) ? 1 : 0;
    return r;
}

void mlq_ref_gguf_free(void* h) { delete static_cast<GGUFReader*>(h); }

const char* mlq_ref_gguf_error(void* h) { return static_cast<GGUFReader*>(h)->load_error.c_str(); }

void mlq_ref_gguf_header(void* h, uint32_t* version, uint64_t* n_tensors, uint64_t* n_metadata,
                         uint64_t* data_offset, uint64_t* n_meta_read, uint64_t* n_tensors_read) {
    const GGUFReader* r = static_cast<GGUFReader*>(h);
    *version = r->version;
    *n_tensors = r->n_tensors;
    *n_metadata = r->n_metadata;
    *data_offset = r->data_offset;
    *n_meta_read = r->metadata.size();
    *n_tensors_read = r->tensors.size();
}

void mlq_ref_gguf_metadata(void* h, uint64_t i, const char** key, uint32_t* type, const char** value,
                           uint64_t* value_len) {
    const GGUFMetadataKV& kv = static_cast<GGUFReader*>(h)->metadata[i];
    *key = kv.key.c_str();
    *type = kv.type;
    *value = kv.value_str.data();
    *value_len = kv.value_str.size();
}

void mlq_ref_gguf_tensor(void* h, uint64_t i, const char** name, uint32_t* n_dims, uint64_t* dims, uint32_t* type,
                         uint64_t* offset, uint64_t* nbytes) {
    const GGUFTensorInfo& t = static_cast<GGUFReader*>(h)->tensors[i];
    *name = t.name.c_str();
    *n_dims = static_cast<uint32_t>(t.shape.size());
    for (size_t d = 0; d < t.shape.size() && d < 8; ++d) dims[d] = t.shape[d];
    *type = t.type;
    *offset = t.offset;
    uint64_t n = 0;
    *nbytes = gguf_tensor_data_size(t, n) ? n : ~0ull;
}

// read_gguf_tensor_raw into `out` (capacity `cap`); returns the byte count.
long long mlq_ref_gguf_read(const char* path, void* h, uint64_t i, void* out, uint64_t cap) {
    const GGUFReader* r = static_cast<GGUFReader*>(h);
    std::vector<uint8_t> raw = read_gguf_tensor_raw(path, r->tensors[i], r->data_offset);
    if (raw.size() > cap) return -1;
    std::memcpy(out, raw.data(), raw.size());
    return static_cast<long long>(raw.size());
}

const char* mlq_ref_ggml_type_name(uint32_t t) { return ggml_type_name(t); }
const char* mlq_ref_gguf_value_type_name(uint32_t t) { return gguf_value_type_name(t); }

// load_gguf_model; the model is returned whether or not it loaded (*ok).
void* mlq_ref_gguf_model(const char* path, int* ok) {
    MiniLlamaModel* m = new MiniLlamaModel(load_gguf_model(path));
    *ok = m->loaded ? 1 : 0;
    return m;
}

void mlq_ref_model_free(void* h) { delete static_cast<MiniLlamaModel*>(h); }

const char* mlq_ref_model_error(void* h) { return static_cast<MiniLlamaModel*>(h)->load_error.c_str(); }

// A linear weight of a loaded model by the reference's own name ("lm_head",
// "layers.N.wq" ... "layers.N.w_down"): quant type, shape and block bytes.
int mlq_ref_model_linear(void* h, const char* name, int* qtype, int* rows, int* cols, const void** data,
                         uint64_t* nbytes) {
    MiniLlamaModel* m = static_cast<MiniLlamaModel*>(h);
    const std::string n = name;
    const QuantizedTensor* q = nullptr;
    if (n == "lm_head") {
        q = &m->lm_head;
    } else if (n.rfind("layers.", 0) == 0) {
        const size_t dot = n.find('.', 7);
        if (dot == std::string::npos) return -1;
        const int layer = std::stoi(n.substr(7, dot - 7));
        if (layer < 0 || layer >= static_cast<int>(m->layers.size())) return -1;
        LayerWeights& lw = m->layers[layer];
        const std::string op = n.substr(dot + 1);
        if (op == "wq") q = &lw.wq;
        else if (op == "wk") q = &lw.wk;
        else if (op == "wv") q = &lw.wv;
        else if (op == "wo") q = &lw.wo;
        else if (op == "w_gate") q = &lw.w_gate;
        else if (op == "w_up") q = &lw.w_up;
        else if (op == "w_down") q = &lw.w_down;
    }
    if (q == nullptr || q->shape.size() != 2) return -1;
    *qtype = static_cast<int>(q->type);
    *rows = q->shape[0];
    *cols = q->shape[1];
    switch (q->type) {
        case QuantType::Q8_0: *data = q->q8_0_data.data(); *nbytes = q->q8_0_data.size() * sizeof(BlockQ8_0); break;
        case QuantType::Q4_0: *data = q->q4_0_data.data(); *nbytes = q->q4_0_data.size() * sizeof(BlockQ4_0); break;
        case QuantType::Q4_1: *data = q->q4_1_data.data(); *nbytes = q->q4_1_data.size() * sizeof(BlockQ4_1); break;
        default: *data = q->f32_data.data(); *nbytes = q->f32_data.size() * sizeof(float); break;
    }
    return 0;
}

// ---- Decode: load_gguf_model + forward_token (src/forward.cpp:865-903)

struct RefDecoder {
    MiniLlamaModel model;
    std::unique_ptr<MiniLlamaContext> ctx;
};

void* mlq_ref_decoder_open(const char* path, int threads, int* ok) {
    set_thread_count(threads);
    RefDecoder* d = new RefDecoder;
    d->model = load_gguf_model(path);
    *ok = d->model.loaded ? 1 : 0;
    if (d->model.loaded) d->ctx.reset(new MiniLlamaContext(&d->model));
    return d;
}

const char* mlq_ref_decoder_error(void* h) { return static_cast<RefDecoder*>(h)->model.load_error.c_str(); }

void mlq_ref_decoder_free(void* h) { delete static_cast<RefDecoder*>(h); }

void mlq_ref_decoder_config(void* h, int* out) {
    const ModelConfig& c = static_cast<RefDecoder*>(h)->model.config;
    const int v[] = {c.n_layers, c.dim, c.hidden_dim, c.n_heads, c.n_kv_heads, c.head_dim, c.vocab_size,
                     c.max_seq_len, c.rope_type == RopeType::NeoX ? 1 : 0};
    std::memcpy(out, v, sizeof v);
}

// forward_token with ctx.pos = pos; logits to `out`.  Returns 0, or -1 with
// the exception text in err.
int mlq_ref_decoder_forward(void* h, int token, int pos, float* out, char* err, size_t err_len) {
    RefDecoder* d = static_cast<RefDecoder*>(h);
    try {
        d->ctx->pos = pos;
        Tensor logits = forward_token(d->model, *d->ctx, token);
        std::memcpy(out, logits.data.data(), logits.data.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        std::snprintf(err, err_len, "%s", e.what());
        return -1;
    }
}

// forward_batch over tokens at positions start..; logits of the last token.
int mlq_ref_decoder_batch(void* h, const int* tokens, int n, int start, float* out, char* err, size_t err_len) {
    RefDecoder* d = static_cast<RefDecoder*>(h);
    try {
        std::vector<int> toks(tokens, tokens + n);
        Tensor logits = forward_batch(d->model, *d->ctx, MiniBatch::from_tokens(toks, start));
        std::memcpy(out, logits.data.data(), logits.data.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        std::snprintf(err, err_len, "%s", e.what());
        return -1;
    }
}

// Greedy generation as forward_batch over the prompt, then sample_greedy and
// forward_token per new token.
int mlq_ref_decoder_generate(void* h, const int* prompt, int n_prompt, int n_new, int* out, char* err,
                             size_t err_len) {
    RefDecoder* d = static_cast<RefDecoder*>(h);
    try {
        std::vector<int> toks(prompt, prompt + n_prompt);
        Tensor logits = forward_batch(d->model, *d->ctx, MiniBatch::from_tokens(toks, 0));
        int pos = n_prompt;
        for (int i = 0; i < n_new; ++i) {
            const int t = MiniSampler::sample_greedy(logits);
            out[i] = t;
            if (i + 1 < n_new) {
                d->ctx->pos = pos++;
                logits = forward_token(d->model, *d->ctx, t);
            }
        }
        return 0;
    } catch (const std::exception& e) {
        std::snprintf(err, err_len, "%s", e.what());
        return -1;
    }
}

}  // extern "C"

"""Small llama / qwen2 model files in GGUF for the decoder tests (test
infrastructure): the metadata keys and tensor names load_gguf_model reads
(src/gguf_loader.cpp:15-104, 241-310), seeded weights, every linear in a
chosen format (quantized by the oracle, or F32)."""

from __future__ import annotations

import numpy as np

import gguf_writer as gw
import oracle

FMT = {"q8_0": (oracle.Q8_0, gw.GGML_Q8_0), "q4_0": (oracle.Q4_0, gw.GGML_Q4_0),
       "q4_1": (oracle.Q4_1, gw.GGML_Q4_1), "f32": (None, gw.GGML_F32)}


def write_model(orc, path, *, arch="llama", layers=2, dim=128, hidden=352, heads=8, kv_heads=4, vocab=300,
                ctx=64, fmts=("q4_0", "q8_0", "q4_1"), lm="q8_0", emb="f32", biases=False, seed=0,
                scale=0.05, theta=10000.0, eps=1e-5, skip=()):
    """Writes the model; `lm` None ties the output to the embedding; `skip`
    leaves GGUF tensors out (to test the loader's errors)."""
    rng = np.random.default_rng(seed)
    hd = dim // heads
    a = arch
    meta = [("general.architecture", gw.STRING, arch), ("general.name", gw.STRING, "mlq-test"),
            (f"{a}.block_count", gw.U32, layers), (f"{a}.embedding_length", gw.U32, dim),
            (f"{a}.feed_forward_length", gw.U32, hidden), (f"{a}.attention.head_count", gw.U32, heads),
            (f"{a}.attention.head_count_kv", gw.U32, kv_heads), (f"{a}.context_length", gw.U32, ctx),
            (f"{a}.rope.freq_base", gw.F32, theta), (f"{a}.attention.layer_norm_rms_epsilon", gw.F32, eps),
            ("tokenizer.ggml.tokens", gw.ARRAY, (gw.STRING, [f"t{i}" for i in range(vocab)]))]
    tensors = []
    k = [0]

    def add(name, t):
        if name not in skip:
            tensors.append(t)

    def matrix(name, rows, cols, fmt):
        w = (rng.standard_normal((rows, cols)) * scale).astype(np.float32)
        qt, gt = FMT[fmt]
        if qt is None:
            add(name, gw.f32_tensor(name, w))
        else:
            add(name, gw.linear_tensor(name, gt, orc.quantize(qt, w), rows, cols))

    def linear(name, rows, cols):
        fmt = fmts[k[0] % len(fmts)]
        k[0] += 1
        matrix(name, rows, cols, fmt)

    def vec(name, n, mean=1.0, sd=0.1):
        add(name, gw.f32_tensor(name, (mean + sd * rng.standard_normal(n)).astype(np.float32)))

    e = (rng.standard_normal((vocab, dim)) * 0.5).astype(np.float32)
    if emb == "f32":
        add("token_embd.weight", gw.f32_tensor("token_embd.weight", e))
    else:
        qt, gt = FMT[emb]
        add("token_embd.weight", gw.linear_tensor("token_embd.weight", gt, orc.quantize(qt, e), vocab, dim))
    for l in range(layers):
        p = f"blk.{l}."
        vec(p + "attn_norm.weight", dim)
        linear(p + "attn_q.weight", heads * hd, dim)
        linear(p + "attn_k.weight", kv_heads * hd, dim)
        linear(p + "attn_v.weight", kv_heads * hd, dim)
        if biases:
            vec(p + "attn_q.bias", heads * hd, 0.0, 0.05)
            vec(p + "attn_k.bias", kv_heads * hd, 0.0, 0.05)
            vec(p + "attn_v.bias", kv_heads * hd, 0.0, 0.05)
        linear(p + "attn_output.weight", dim, heads * hd)
        vec(p + "ffn_norm.weight", dim)
        linear(p + "ffn_gate.weight", hidden, dim)
        linear(p + "ffn_up.weight", hidden, dim)
        linear(p + "ffn_down.weight", dim, hidden)
    vec("output_norm.weight", dim)
    if lm is not None:
        matrix("output.weight", vocab, dim, lm)
    gw.write(path, meta, tensors, alignment=32)
    return path

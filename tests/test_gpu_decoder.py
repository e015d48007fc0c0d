"""Device-resident decode (mlq_hip_decoder_*) against the reference's own
load_gguf_model + forward_token (src/gguf_loader.cpp, src/forward.cpp:865-903)
and greedy loop (forward_batch + MiniSampler::sample_greedy), compiled into
oracle/_ref, on seeded model files written by tests/model_files.py.

* logits at every position of a token sequence: |gpu - ref| <= TOL * max(1,
  max |ref logits|) with TOL = 1e-3, the north star's bound for one quantized
  linear (the Q4 GEMV alone may differ from the reference by ~1e-4 relative;
  the other ops add the order of parallel sums and a few ulp of the device
  exp / pow / sin / cos).  Measured worst: 8.3e-5;
* greedy generation: the same tokens as the reference (a divergence is only
  accepted where the reference's top two logits lie within that tolerance);
* the recorded, fed-back device loop equals step-by-step forwards with a host
  argmax (first maximum);
* the loader's and the forward's error messages.
Variants cover llama (normal RoPE) and qwen2 (NeoX RoPE, q/k/v biases, tied
lm_head -> F32 GEMV), every linear format including F32, a quantized
embedding, multi-head / grouped / multi-query attention, head_dim 16 and 128
(and 64 / 256 after a batched prefill), and hidden widths of an odd number of
blocks.
"""

import os
import sys

import numpy as np
import pytest

import model_files as mf
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-3

VARIANTS = {
    "llama_mixed": dict(),
    "qwen2_bias_tied": dict(arch="qwen2", biases=True, lm=None, seed=1),
    "q8_embedding_f32_linears": dict(emb="q8_0", lm="q4_1", fmts=("f32", "q4_0"), seed=2),
    "mha_q4_0": dict(heads=4, kv_heads=4, hidden=256, fmts=("q4_0",), lm="q4_0", seed=3),
    "mqa_q8_0_3_layers": dict(heads=8, kv_heads=1, fmts=("q8_0",), lm="q8_0", layers=3, seed=4),
    "head_dim_128": dict(dim=256, heads=2, kv_heads=1, hidden=704, fmts=("q4_1", "q4_0"), lm="q4_0", seed=5),
}


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ref():
    r = oracle.reference()
    if r is None:
        pytest.skip("reference shim not built (oracle/_ref)")
    return r


def model(orc, tmp_path, name):
    return mf.write_model(orc, str(tmp_path / f"{name}.gguf"), **VARIANTS[name])


def close(got, want, label):
    scale = max(1.0, float(np.abs(want).max()))
    err = float(np.abs(got.astype(np.float64) - want).max())
    assert np.isfinite(got).all(), label
    assert err <= TOL * scale, f"{label}: max |diff| {err:.3e} > {TOL * scale:.3e}"
    return err / scale


@pytest.mark.parametrize("name", list(VARIANTS))
def test_logits_match_reference(hip, orc, ref, tmp_path, name):
    path = model(orc, tmp_path, name)
    say(f"decoder {name}")
    dec = hip.Decoder(path)
    rd = ref.decoder(path)
    assert dec.config["vocab_size"] == rd.config["vocab_size"]
    assert dec.config["rope_neox"] == rd.config["rope_neox"]
    rng = np.random.default_rng(7)
    tokens = rng.integers(0, dec.config["vocab_size"], 12).tolist()
    worst = 0.0
    for pos, t in enumerate(tokens):
        worst = max(worst, close(dec.forward(t, pos), rd.forward(t, pos), f"{name} pos {pos}"))
    say(f"  worst relative logit difference {worst:.2e}")
    dec.close()


@pytest.mark.parametrize("name,n_tok", [("head_dim_128", 160), ("mha_q4_0", 560), ("head_dim_128", 1000)])
def test_long_context_logits_match_reference(hip, orc, ref, tmp_path, name, n_tok):
    """Contexts of several attention passes: one pass covers 32 cache rows at
    head_dim 128 and 128 rows at head_dim 32 (256 threads, 4 rows each), so
    these runs take the multi-pass path with its one-pass-ahead requests; past
    128 positions the positions are split over up to 8 workgroups per head
    (2, 5 and 8 splits for caches of 168, 568 and 1008 positions)."""
    path = mf.write_model(orc, str(tmp_path / f"{name}_long.gguf"), **dict(VARIANTS[name], ctx=n_tok + 8))
    say(f"decoder {name} over {n_tok} positions")
    dec = hip.Decoder(path)
    rd = ref.decoder(path)
    rng = np.random.default_rng(11)
    tokens = rng.integers(0, dec.config["vocab_size"], n_tok).tolist()
    worst = 0.0
    for pos, t in enumerate(tokens):
        worst = max(worst, close(dec.forward(t, pos), rd.forward(t, pos), f"{name} pos {pos}"))
    say(f"  worst relative logit difference {worst:.2e}")
    dec.close()


@pytest.mark.parametrize("name", list(VARIANTS))
def test_greedy_generation_matches_reference(hip, orc, ref, tmp_path, name):
    path = model(orc, tmp_path, name)
    prompt, n_new = [3, 1, 4, 1, 5], 16
    dec = hip.Decoder(path)
    got = dec.generate(prompt, n_new)
    want = ref.decoder(path).generate(prompt, n_new)
    if got != want:
        i = next(j for j in range(n_new) if got[j] != want[j])
        # Logits the reference saw before the divergent pick.
        rd = ref.decoder(path)
        toks = prompt + want[:i]
        for pos, t in enumerate(toks):
            logits = rd.forward(t, pos)
        scale = max(1.0, float(np.abs(logits).max()))
        top = np.sort(logits)[-2:]
        say(f"  {name}: divergence allowance used at token {i}: HIP {got[i]}, reference {want[i]}, "
            f"reference top-2 gap {top[1] - top[0]:.3e}, HIP pick's logit {logits[got[i]]:.6g} "
            f"vs max {logits.max():.6g}")
        assert top[1] - top[0] <= TOL * scale, \
            f"{name}: token {i} is {got[i]}, reference {want[i]} (gap {top[1] - top[0]:.3e})"
        # The HIP pick must itself be one of the (near-)maximal logits of the
        # reference, not an arbitrary token.
        assert logits[got[i]] >= logits.max() - TOL * scale, \
            f"{name}: token {i}: HIP picked {got[i]} whose reference logit {logits[got[i]]:.6g} is not near " \
            f"the maximum {logits.max():.6g}"
    dec.close()


def test_device_loop_equals_stepwise_forward(hip, orc, tmp_path):
    """The recorded step, replayed with the pick fed back on the device, gives
    the tokens of step-by-step forwards with a host argmax."""
    path = model(orc, tmp_path, "llama_mixed")
    dec = hip.Decoder(path)
    prompt, n_new = [10, 20, 30], 20
    loop = dec.generate(prompt, n_new)
    toks = list(prompt)
    for pos in range(len(prompt) + n_new - 1):
        logits = dec.forward(toks[pos], pos)
        if pos >= len(prompt) - 1:
            toks.append(int(np.argmax(logits)))
    assert loop == toks[len(prompt):]
    # Again on the same decoder (recorded step reused), then with a longer
    # prompt (buffers grow, the step is recorded again).
    assert dec.generate(prompt, n_new) == loop
    longer = dec.generate(list(range(1, 30)), 30)
    assert len(longer) == 30
    dec.close()


def test_device_loop_long_context(hip, orc, tmp_path):
    """Past 128 positions decode attention splits each head over several
    workgroups that count in on a per-head counter the last one resets: the
    recorded step replayed over a long context (twice) gives the tokens of
    stepwise forwards after the same batched prefill."""
    path = mf.write_model(orc, str(tmp_path / "long.gguf"), **dict(VARIANTS["head_dim_128"], ctx=600))
    dec = hip.Decoder(path)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, dec.config["vocab_size"], 300).tolist()
    n_new = 40
    loop = dec.generate(prompt, n_new)
    assert dec.generate(prompt, n_new) == loop
    dec.prefill(prompt[:-1])
    toks = list(prompt)
    for pos in range(len(prompt) - 1, len(prompt) + n_new - 1):
        toks.append(int(np.argmax(dec.forward(toks[pos], pos))))
    assert loop == toks[len(prompt):]
    dec.close()


def test_forward_and_generate_errors(hip, orc, tmp_path):
    path = model(orc, tmp_path, "llama_mixed")
    dec = hip.Decoder(path, max_seq_len=16)
    assert dec.config["max_seq_len"] == 16
    with pytest.raises(hip.MlqError, match="forward_token token id out of range"):
        dec.forward(300, 0)
    with pytest.raises(hip.MlqError, match="forward_token position out of range"):
        dec.forward(1, 16)
    with pytest.raises(hip.MlqError, match="forward_token position out of range"):
        dec.generate([1, 2, 3], 15)
    with pytest.raises(hip.MlqError, match="forward_token token id out of range"):
        dec.generate([1, -2], 3)
    assert len(dec.generate([1, 2, 3], 14)) == 14  # exactly fills the 16 positions
    dec.close()


@pytest.mark.parametrize("case", ["missing_w_up", "missing_embedding", "no_vocab", "bad_heads"])
def test_loader_errors_match_reference(hip, orc, ref, tmp_path, case):
    kw = {"missing_w_up": dict(skip=("blk.1.ffn_up.weight",)),
          "missing_embedding": dict(skip=("token_embd.weight",)),
          "no_vocab": dict(vocab=0),
          "bad_heads": dict(heads=8, kv_heads=3)}[case]
    if case == "no_vocab":
        path = mf.write_model(orc, str(tmp_path / "m.gguf"), vocab=1)
        data = open(path, "rb").read().replace(b"tokenizer.ggml.tokens", b"tokenizer.ggml.tokenz")
        open(path, "wb").write(data)
    else:
        path = mf.write_model(orc, str(tmp_path / "m.gguf"), **kw)
    with pytest.raises(RuntimeError) as want:
        ref.decoder(path)
    with pytest.raises(hip.MlqError) as got:
        hip.Decoder(path)
    assert got.value.msg == str(want.value)


@pytest.mark.parametrize("name", list(VARIANTS))
def test_batched_prefill_matches_reference(hip, orc, ref, tmp_path, name):
    """mlq_hip_decoder_prefill (every layer over all rows, MFMA GEMMs for the
    linears) against the reference's token-by-token forward_batch: the last
    token's logits, then a continuation step that reads the cache the batch
    wrote, and a second batch at a later start."""
    path = model(orc, tmp_path, name)
    dec = hip.Decoder(path)
    rd = ref.decoder(path)
    rng = np.random.default_rng(11)
    v = dec.config["vocab_size"]
    toks = rng.integers(0, v, 44).tolist()
    worst = close(dec.prefill(toks[:20]), rd.batch(toks[:20]), f"{name} batch 0..19")
    worst = max(worst, close(dec.forward(toks[20], 20), rd.forward(toks[20], 20), f"{name} step 20"))
    worst = max(worst, close(dec.prefill(toks[21:37], 21), rd.batch(toks[21:37], 21), f"{name} batch 21..36"))
    # 7 rows: the attention's last group of four query rows is partial
    worst = max(worst, close(dec.prefill(toks[37:44], 37), rd.batch(toks[37:44], 37), f"{name} batch 37..43"))
    say(f"  worst relative logit difference {worst:.2e}")
    dec.close()


@pytest.mark.parametrize("dim,heads,kv_heads", [(256, 4, 2), (256, 1, 1)], ids=["head_dim_64", "head_dim_256"])
def test_batched_prefill_head_dims(hip, orc, ref, tmp_path, dim, heads, kv_heads):
    """The prefill attention at other head sizes (64: the MFMA kernel; 256:
    the VALU kernel, 32 lanes of two float4s per cache row), over many passes
    of cache rows and a second batch at a later start; then decode steps."""
    path = mf.write_model(orc, str(tmp_path / "hd.gguf"), dim=dim, heads=heads, kv_heads=kv_heads, hidden=352,
                          ctx=256, fmts=("q4_0",), lm="q4_0", seed=12)
    dec = hip.Decoder(path)
    rd = ref.decoder(path)
    toks = np.random.default_rng(13).integers(0, 300, 230).tolist()
    worst = close(dec.prefill(toks[:150]), rd.batch(toks[:150]), f"head_dim {dim // heads} batch 0..149")
    worst = max(worst, close(dec.prefill(toks[150:230], 150), rd.batch(toks[150:230], 150),
                             f"head_dim {dim // heads} batch 150..229"))
    # decode steps after the batches: the single-token attention at this head
    # size, past 128 positions (its positions split over two workgroups)
    for pos, t in ((230, 5), (231, 7)):
        worst = max(worst, close(dec.forward(t, pos), rd.forward(t, pos), f"head_dim {dim // heads} step {pos}"))
    say(f"  head_dim {dim // heads}: worst relative logit difference {worst:.2e}")
    dec.close()


# Row widths of the producers that write a GEMM's split x: the RMSNorm row
# kernel covers `dim`, the SwiGLU row kernel `hidden`, each with C = 1..4
# halves of 16 elements per thread (C = ceil(width / 4096)).
SPLIT_SHAPES = {
    "c1": dict(dim=256, heads=2, kv_heads=1, hidden=768, layers=2),
    "swiglu_c2": dict(dim=256, heads=2, kv_heads=1, hidden=4608, layers=2),
    "swiglu_c3": dict(dim=256, heads=2, kv_heads=1, hidden=11008, layers=2),
    "swiglu_c4": dict(dim=256, heads=2, kv_heads=1, hidden=13824, layers=1),
    "norm_c2": dict(dim=4608, heads=36, kv_heads=4, hidden=352, layers=1),
}


@pytest.mark.parametrize("shape", list(SPLIT_SHAPES))
@pytest.mark.parametrize("fmt", ["q4_0", "q8_0", "q4_1"])
def test_batched_prefill_split_x_written_by_norm_and_swiglu(hip, orc, ref, tmp_path, fmt, shape):
    """Over 128 rows the RMSNorm and SwiGLU row kernels write the q/k/v,
    gate/up and down GEMMs' split x themselves (every linear of one format, so
    q/k/v and gate/up run as grouped GEMMs), at every producer width C = 1..4
    (hidden 768 / 4608 / 11008 / 13824, dim 256 / 4608); then a short batch
    (plain x) reads the cache the long one wrote."""
    kw = SPLIT_SHAPES[shape]
    path = mf.write_model(orc, str(tmp_path / f"split_{fmt}_{shape}.gguf"), ctx=320, fmts=(fmt,), lm=fmt,
                          seed=21, **kw)
    dec = hip.Decoder(path)
    rd = ref.decoder(path)
    toks = np.random.default_rng(22).integers(0, 300, 260).tolist()
    say(f"split-x producers {shape} {fmt}: batch of 200 rows, then 60")
    worst = close(dec.prefill(toks[:200]), rd.batch(toks[:200]), f"{fmt} {shape} batch 0..199")
    worst = max(worst, close(dec.prefill(toks[200:260], 200), rd.batch(toks[200:260], 200),
                             f"{fmt} {shape} batch 200..259"))
    say(f"  {fmt} {shape}: worst relative logit difference {worst:.2e}")
    dec.close()


def test_batched_prefill_longer_than_one_pass(hip, orc, ref, tmp_path):
    """A prompt of more rows than one batched pass holds (chunks of 512)."""
    path = mf.write_model(orc, str(tmp_path / "long.gguf"), ctx=640, vocab=300, layers=2, seed=9)
    dec = hip.Decoder(path)
    rd = ref.decoder(path)
    toks = np.random.default_rng(3).integers(0, 300, 600).tolist()
    close(dec.prefill(toks), rd.batch(toks), "600-token batch")
    got = dec.generate(toks[:300], 8)
    assert got == ref.decoder(path).generate(toks[:300], 8)
    dec.close()

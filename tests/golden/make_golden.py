"""Write the golden vectors in tests/golden/ from the compiled reference.

Run in the build container, where /root/reference exists:

    make -C oracle ref            # builds oracle/_ref/libmlq_ref.so from the reference sources
    python tests/golden/make_golden.py

Everything produced here is data (inputs and the reference's outputs); no
reference source text is stored.  Outputs:

* ``quant_golden.npz`` -- for every case: the f32 weight and input, and for each
  of Q8_0 / Q4_0 / Q4_1 the reference's block bytes (``quantize_to_q8_0``,
  ``quantize_to_q4_0``, the test-local ``quantize_to_q4_1_for_test``), its
  dequantized weights and the bits of its scalar ``linear`` output.  Plus an
  fp16 encoding table observed through one-element Q4_1 blocks.
* ``tiny_linears.npz`` -- the 15 linear weights of the reference's tiny model
  (``models/tiny/model.bin`` read through ``models/tiny/model.json``; hidden_dim
  86 gives tail blocks) with the reference outputs for a pattern input.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, REPO)

import oracle  # noqa: E402

REF_ROOT = os.environ.get("MLQ_REFERENCE", "/root/reference")
OUT = os.path.dirname(os.path.abspath(__file__))
FORMATS = {"q8_0": oracle.Q8_0, "q4_0": oracle.Q4_0, "q4_1": oracle.Q4_1}


def pattern(shape, scale, shift):
    """tests/test_cuda_quant.cpp:51-58: bucket = (i*19+7) % 31; (bucket-15)*scale + shift in f32."""
    n = int(np.prod(shape))
    i = np.arange(n, dtype=np.int64)
    bucket = ((i * 19 + 7) % 31 - 15).astype(np.float32)
    return (bucket * np.float32(scale) + np.float32(shift)).astype(np.float32).reshape(shape)


def cases():
    rng = np.random.default_rng(20260101)
    out = []
    # The reference's own CUDA parity shapes (tests/test_cuda_quant.cpp:297-299, 312-313, 395-396).
    out.append(("pat_5x13", pattern((5, 13), 0.037, -0.11), pattern((13,), 0.071, 0.03)))
    out.append(("pat_32x64", pattern((32, 64), 0.019, 0.04), pattern((3, 64), 0.029, -0.06)))
    out.append(("pat_17x65", pattern((17, 65), 0.019, 0.04), pattern((3, 65), 0.029, -0.06)))
    # tests/test_quant.cpp:17-76, 253-291 inputs.
    out.append(("ramp_1x32", (np.arange(32, dtype=np.float32) * np.float32(0.1)).reshape(1, 32),
                np.ones(32, np.float32)))
    out.append(("ramp_1x100", (np.arange(100, dtype=np.float32) * np.float32(0.05)).reshape(1, 100),
                np.ones(100, np.float32)))
    w = (np.arange(128, dtype=np.float32) * np.float32(0.05) - np.float32(1.0)).reshape(4, 32)
    x = np.arange(32, dtype=np.float32) * np.float32(0.1) - np.float32(0.4)
    out.append(("ramp_4x32", w, x))
    out.append(("zeros_2x64", np.zeros((2, 64), np.float32), np.ones(64, np.float32)))
    # Constant and single-sign blocks: Q4_1 range 0, Q4_0 clamps.
    const = np.full((3, 40), 0.25, np.float32)
    const[1] = -0.5
    out.append(("const_3x40", const, pattern((40,), 0.01, 0.0)))
    # Seeded N(0, 0.02) weights at the BASELINE shapes' K (row strides 8 B aligned at K=896).
    for m, k, rows in [(16, 896, 1), (12, 896, 4), (6, 4096, 1), (4, 4864, 2), (2, 11008, 1),
                       (33, 86, 3), (3, 4095, 2)]:
        wv = (rng.standard_normal((m, k)) * 0.02).astype(np.float32)
        xv = rng.standard_normal((rows, k) if rows > 1 else (k,)).astype(np.float32)
        out.append((f"rand_{m}x{k}_r{rows}", wv, xv))
    # Wide-range weights: scales near fp16 subnormals and near the top of the range.
    wv = (rng.standard_normal((6, 64)) * np.float32(1e-6)).astype(np.float32)
    wv[3] *= np.float32(1e10)
    wv[4] = (rng.standard_normal(64) * np.float32(1e-9)).astype(np.float32)
    out.append(("scales_6x64", wv, rng.standard_normal(64).astype(np.float32)))
    return out


def fp16_table(ref: oracle.Reference):
    """Finite f32 inputs that cover every rounding region of the encoder."""
    rng = np.random.default_rng(7)
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e30, -1e30,
            2.0 ** -14, 2.0 ** -24, 2.0 ** -25, 2.0 ** -26, 3 * 2.0 ** -26, 1.5 * 2.0 ** -24,
            2.0 ** -25 * 1.0000001, 6.1e-5, 1e-8, 1e-45]
    # Exact ties and near-ties at bit 12 for normals and subnormals.
    base = rng.integers(0, 2 ** 31, 4000, dtype=np.int64).astype(np.uint32)
    base &= np.uint32(0x7fffffff)
    for delta in (0x0000, 0x1000, 0x0fff, 0x1001, 0x1fff):
        u = (base & np.uint32(0xffffe000)) | np.uint32(delta)
        vals.extend(u.view(np.float32)[:800].tolist())
    u = rng.integers(0x30000000, 0x48000000, 8000, dtype=np.int64).astype(np.uint32)
    vals.extend(u.view(np.float32).tolist())
    v = np.array(vals, dtype=np.float32)
    v = v[np.isfinite(v)]
    v = np.concatenate([v, -v])
    enc = np.array([ref.fp16_probe_q4_1(float(t)) for t in v], dtype=np.uint16)
    enc_q8 = np.array([ref.fp16_probe_q8_0(float(t)) for t in v[:4000]], dtype=np.uint16)
    return v, enc, enc_q8


def tiny_model(ref: oracle.Reference):
    d = os.path.join(REF_ROOT, "models", "tiny")
    with open(os.path.join(d, "model.json")) as f:
        manifest = json.load(f)
    raw = np.fromfile(os.path.join(d, "model.bin"), dtype=np.uint8)
    store = {}
    names = []
    for t in manifest["tensors"]:
        if len(t["shape"]) != 2 or t["name"] == "token_embedding":
            continue
        arr = raw[t["offset"]:t["offset"] + t["byte_size"]].view(np.float32).reshape(t["shape"]).copy()
        names.append(t["name"])
        key = t["name"].replace(".", "_")
        store[f"{key}__w"] = arr
        m, k = arr.shape
        x = pattern((k,), 0.071, 0.03)
        store[f"{key}__x"] = x
        for fname, qt in FORMATS.items():
            blocks = ref.quantize(qt, arr)
            store[f"{key}__{fname}__blocks"] = blocks
            store[f"{key}__{fname}__y"] = ref.linear(qt, x, blocks, m, threads=1)
    store["names"] = np.array(names)
    return store


def main():
    oracle.build(REF_ROOT)
    ref = oracle.reference()
    if ref is None:
        raise SystemExit("reference shim not built")
    store = {}
    names = []
    for name, w, x in cases():
        names.append(name)
        m, k = w.shape
        store[f"{name}__w"] = w
        store[f"{name}__x"] = x
        for fname, qt in FORMATS.items():
            blocks = ref.quantize(qt, w)
            store[f"{name}__{fname}__blocks"] = blocks
            if m * k <= 4096:
                store[f"{name}__{fname}__deq"] = ref.dequantize(qt, blocks, m, k)
            store[f"{name}__{fname}__y"] = ref.linear(qt, x, blocks, m, threads=1)
            # the threaded path must give the same bits (src/thread_pool.cpp splits by output)
            y4 = ref.linear(qt, x, blocks, m, threads=4)
            assert (y4.view(np.uint32) == store[f"{name}__{fname}__y"].view(np.uint32)).all()
    store["names"] = np.array(names)
    v, enc, enc_q8 = fp16_table(ref)
    store["fp16_in"] = v
    store["fp16_out"] = enc
    store["fp16_q8_probe"] = enc_q8
    np.savez_compressed(os.path.join(OUT, "quant_golden.npz"), **store)
    np.savez_compressed(os.path.join(OUT, "tiny_linears.npz"), **tiny_model(ref))
    for f in ("quant_golden.npz", "tiny_linears.npz"):
        print(f, os.path.getsize(os.path.join(OUT, f)), "bytes")


if __name__ == "__main__":
    main()

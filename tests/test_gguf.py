"""GGUF ingest, CPU side: the library's GGUF index (mlq_hip_gguf_*) against
the reference's own reader and loader, compiled from src/gguf.cpp and
src/gguf_loader.cpp into oracle/_ref (no GPU needed: parsing and the mapping
are host code).

* Known answers of the reference's tests/test_gguf.cpp:68-270 on its fixture
  models/tiny/test.gguf (copied to tests/golden/test.gguf) and on the same
  mutations those tests make: version 2, bad alignment, duplicate key, zero
  dimension, data out of bounds, wrong magic, missing file.
* Differential checks against GGUFReader::load: every prefix of the fixture,
  seeded byte mutations of the header, every metadata value type and
  rendering, quantized / F16 / unknown-type tensors and alignments; the
  tensor bytes the mapping exposes against read_gguf_tensor_raw.
* A whole model file read by load_gguf_model: every linear's bytes and
  [out, in] shape equal what the index maps for the file's tensor.
"""

import os
import shutil
import struct

import numpy as np
import pytest

import gguf_writer as gw
import mlq_hip
import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "test.gguf")
QT_GGML = {oracle.Q8_0: gw.GGML_Q8_0, oracle.Q4_0: gw.GGML_Q4_0, oracle.Q4_1: gw.GGML_Q4_1}


@pytest.fixture(scope="module")
def lib():
    return mlq_hip.load()


@pytest.fixture(scope="module")
def ref():
    r = oracle.reference()
    if r is None:
        pytest.skip("reference shim not built (oracle/_ref)")
    return r


def ours(path):
    try:
        g = mlq_hip.GgufFile(path)
    except mlq_hip.MlqError as e:
        return {"ok": False, "error": e.msg}
    try:
        out = {"ok": True, "error": ""}
        out.update(g.header())
        out["metadata"] = g.metadata()
        out["tensors"] = g.tensors()
        return out
    finally:
        g.close()


def agree(ref, path):
    a, b = ours(path), ref.gguf(path)
    assert (a["ok"], a["error"]) == (b["ok"], b["error"]), f"{path}: ours {a['error']!r}, reference {b['error']!r}"
    if a["ok"]:
        for k in ("version", "n_tensors", "n_metadata", "data_offset"):
            assert a[k] == b[k], k
        assert a["metadata"] == b["metadata"]
        assert a["tensors"] == b["tensors"]
    return a


def mutated(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(bytes(data))
    return str(p)


# ------------------------------------------------------------ known answers
def test_fixture_known_answers(lib):
    g = ours(FIXTURE)
    assert g["ok"], g["error"]
    assert (g["version"], g["n_tensors"], g["n_metadata"]) == (3, 1, 3)
    assert g["metadata"] == [("general.architecture", gw.STRING, "llama"), ("general.name", gw.STRING, "tiny-test"),
                             ("general.alignment", gw.U32, "64")]
    t = g["tensors"][0]
    assert (t["name"], t["dims"], t["type"], t["offset"]) == ("token_embd.weight", [128, 32], gw.GGML_F32, 0)
    assert t["nbytes"] == 128 * 32 * 4
    assert g["data_offset"] > 0 and g["data_offset"] % 64 == 0


def _field_after(data, needle, skip):
    i = bytes(data).find(needle.encode())
    assert i >= 0
    return i + len(needle) + skip


@pytest.mark.parametrize("case", ["version2", "alignment48", "zero_dim", "out_of_bounds", "duplicate_key",
                                  "not_gguf", "missing"])
def test_reference_error_cases(lib, tmp_path, case):
    """The mutations of tests/test_gguf.cpp:142-270 and their exact messages."""
    data = bytearray(open(FIXTURE, "rb").read())
    if case == "version2":
        data[4:8] = struct.pack("<I", 2)
        want = "unsupported GGUF version: 2"
    elif case == "alignment48":
        o = _field_after(data, "general.alignment", 4)
        data[o:o + 4] = struct.pack("<I", 48)
        want = "invalid general.alignment"
    elif case == "zero_dim":
        o = _field_after(data, "token_embd.weight", 4)
        data[o:o + 8] = struct.pack("<Q", 0)
        want = "invalid zero tensor dimension for: token_embd.weight"
    elif case == "out_of_bounds":
        o = _field_after(data, "token_embd.weight", 4 + 8 + 8 + 4)
        data[o:o + 8] = struct.pack("<Q", len(data))
        want = "tensor data outside file bounds: token_embd.weight"
    elif case == "duplicate_key":
        data = gw.build([("general.name", gw.STRING, "first"), ("general.name", gw.STRING, "second")], [])
        want = "duplicate metadata key: general.name"
    elif case == "not_gguf":
        data = open(os.path.join(HERE, "golden", "make_golden.py"), "rb").read()
        want = "invalid GGUF magic"
    path = str(tmp_path / "missing.gguf") if case == "missing" else mutated(tmp_path, case + ".gguf", data)
    if case == "missing":
        want = "failed to open: " + path
    got = ours(path)
    assert not got["ok"] and got["error"] == want


# ------------------------------------------------------- differential checks
def test_every_prefix_agrees(lib, ref, tmp_path):
    """Every truncation of the fixture up to past its data offset, and a few
    inside the data: same verdict and message as the reference reader."""
    data = open(FIXTURE, "rb").read()
    lengths = list(range(0, 300)) + [1000, 8000, len(data) - 1, len(data)]
    for n in lengths:
        agree(ref, mutated(tmp_path, "prefix.gguf", data[:n]))


def rich_file():
    meta = [
        ("u8", gw.U8, 200), ("i8", gw.I8, -7), ("u16", gw.U16, 65535), ("i16", gw.I16, -32768),
        ("u32", gw.U32, 4294967295), ("i32", gw.I32, -2147483648), ("u64", gw.U64, 2 ** 64 - 1),
        ("i64", gw.I64, -2 ** 63), ("bool0", gw.BOOL, 0), ("bool1", gw.BOOL, 1), ("bool2", gw.BOOL, 2),
        ("f_tenth", gw.F32, 0.1), ("f_eps", gw.F32, 1e-5), ("f_big", gw.F32, 3.4028234663852886e38),
        ("f_negzero", gw.F32, -0.0), ("f_inf", gw.F32, float("inf")), ("f_nan", gw.F32, float("nan")),
        ("f_int", gw.F32, 123456789.0), ("d_pi", gw.F64, 3.141592653589793), ("d_tiny", gw.F64, 5e-324),
        ("s_empty", gw.STRING, ""), ("s_utf8", gw.STRING, "héllo wörld"),
        ("arr_str", gw.ARRAY, (gw.STRING, ["a", "bc", ""])), ("arr_i32", gw.ARRAY, (gw.I32, [1, -2, 3])),
        ("arr_empty", gw.ARRAY, (gw.F64, [])),
        ("arr_nested", gw.ARRAY, (gw.ARRAY, [(gw.U8, [1, 2]), (gw.STRING, ["x"])])),
        ("general.alignment", gw.U64, 128),
    ]
    rng = np.random.default_rng(3)
    tensors = [
        ("f16", [48, 3], gw.GGML_F16, rng.standard_normal(144).astype(np.float16).tobytes()),
        ("odd_type", [5], 15, b""),
        ("q8", [64, 2], gw.GGML_Q8_0, rng.integers(0, 256, 4 * 34, dtype=np.uint8).tobytes()),
        ("q4_0", [96, 3], gw.GGML_Q4_0, rng.integers(0, 256, 9 * 18, dtype=np.uint8).tobytes()),
        ("q4_1", [32, 1, 2], gw.GGML_Q4_1, rng.integers(0, 256, 2 * 20, dtype=np.uint8).tobytes()),
        ("f32", [7], gw.GGML_F32, np.arange(7, dtype=np.float32).tobytes()),
    ]
    return gw.build(meta, tensors, alignment=128)


def test_every_value_type_and_tensor_kind_agrees(lib, ref, tmp_path):
    path = mutated(tmp_path, "rich.gguf", rich_file())
    got = agree(ref, path)
    assert got["ok"] and got["data_offset"] % 128 == 0
    names = [t["name"] for t in got["tensors"]]
    g = mlq_hip.GgufFile(path)
    try:
        for i, t in enumerate(got["tensors"]):
            want = ref.gguf_tensor_raw(path, i)
            if t["nbytes"] == 0:
                assert want.size == 0 and g.tensor_bytes(t["name"]).size == 0
                continue
            assert np.array_equal(g.tensor_bytes(t["name"]), want), names[i]
        with pytest.raises(mlq_hip.MlqError, match="Missing tensor: nope"):
            g.find("nope")
    finally:
        g.close()


@pytest.mark.parametrize("align_meta", [(gw.STRING, "64"), (gw.STRING, " 64"), (gw.STRING, "+64"),
                                        (gw.STRING, "64x"), (gw.STRING, "-64"), (gw.F32, 64.0),
                                        (gw.F32, 64.5), (gw.I32, -1), (gw.U32, 0), (gw.U32, 2 ** 20),
                                        (gw.U32, 2 ** 21), (gw.U64, 1), (gw.BOOL, 1)],
                         ids=lambda v: f"{v[0]}:{v[1]!r}")
def test_alignment_rules_agree(lib, ref, tmp_path, align_meta):
    data = gw.build([("general.alignment",) + align_meta],
                    [("t", [32], gw.GGML_Q8_0, bytes(range(34)))], alignment=1)
    # The data section is re-placed by the reader; pad enough bytes after the
    # header that any accepted alignment still finds the tensor inside.
    agree(ref, mutated(tmp_path, "align.gguf", data + b"\0" * (2 ** 21 + 64)))


def test_block_sizes_and_limits_agree(lib, ref, tmp_path):
    cases = [
        [("q4_not_whole", [33], gw.GGML_Q4_0, b"")],                     # numel % 32 != 0
        [("f32_huge", [2 ** 40, 2 ** 40], gw.GGML_F32, b"")],            # byte count overflows
        [("a", [32], gw.GGML_Q8_0, bytes(34)), ("a", [32], gw.GGML_Q8_0, bytes(34))],  # duplicate name
        [("nine_dims", [1] * 9, gw.GGML_F32, b"")],
    ]
    for k, tensors in enumerate(cases):
        agree(ref, mutated(tmp_path, f"lim{k}.gguf", gw.build([], tensors)))
    big = gw.build([], [])
    big = big[:8] + struct.pack("<QQ", 1000001, 0) + big[24:]
    agree(ref, mutated(tmp_path, "many.gguf", big))


def test_seeded_header_mutations_agree(lib, ref, tmp_path):
    """Random byte overwrites in the header of the fixture and of a rich file:
    the index accepts exactly what the reference reader accepts, with the
    same message and the same fields."""
    rng = np.random.default_rng(2024)
    bases = [open(FIXTURE, "rb").read(), rich_file()]
    for it in range(400):
        base = bytearray(bases[it % 2])
        head = 256 if it % 2 == 0 else 700
        for _ in range(int(rng.integers(1, 4))):
            pos = int(rng.integers(0, head))
            base[pos] = int(rng.choice([0, 1, 2, 0x7F, 0x80, 0xFF, int(rng.integers(0, 256))]))
        agree(ref, mutated(tmp_path, "fuzz.gguf", base))


# ------------------------------------------------------- a whole model file
def tiny_model_file(orc, path, lm_qt=oracle.Q8_0):
    """A 2-layer llama-style model (dim 64, 4 heads / 2 kv heads, hidden 96,
    vocab 40) with every linear format; returns {gguf name: (qt, rows, cols,
    blocks)} for the quantized linears."""
    rng = np.random.default_rng(11)
    dim, hidden, vocab, heads, kv_heads = 64, 96, 40, 4, 2
    head_dim = dim // heads
    meta = [("general.architecture", gw.STRING, "llama"), ("general.name", gw.STRING, "tiny-quant"),
            ("llama.block_count", gw.U32, 2), ("llama.embedding_length", gw.U32, dim),
            ("llama.feed_forward_length", gw.U32, hidden), ("llama.attention.head_count", gw.U32, heads),
            ("llama.attention.head_count_kv", gw.U32, kv_heads), ("llama.context_length", gw.U32, 128),
            ("llama.rope.freq_base", gw.F32, 10000.0),
            ("llama.attention.layer_norm_rms_epsilon", gw.F32, 1e-5),
            ("tokenizer.ggml.tokens", gw.ARRAY, (gw.STRING, [f"t{i}" for i in range(vocab)]))]
    tensors, linears = [], {}

    def linear(name, qt, rows, cols):
        w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
        blocks = orc.quantize(qt, w)
        tensors.append(gw.linear_tensor(name, QT_GGML[qt], blocks, rows, cols))
        linears[name] = (qt, rows, cols, blocks)

    tensors.append(gw.f32_tensor("token_embd.weight", rng.standard_normal((vocab, dim)).astype(np.float32)))
    for layer in range(2):
        p = f"blk.{layer}."
        tensors.append(gw.f32_tensor(p + "attn_norm.weight", np.ones(dim, np.float32)))
        linear(p + "attn_q.weight", oracle.Q4_0, heads * head_dim, dim)
        linear(p + "attn_k.weight", oracle.Q8_0, kv_heads * head_dim, dim)
        linear(p + "attn_v.weight", oracle.Q4_1, kv_heads * head_dim, dim)
        linear(p + "attn_output.weight", oracle.Q4_0, dim, heads * head_dim)
        tensors.append(gw.f32_tensor(p + "ffn_norm.weight", np.ones(dim, np.float32)))
        linear(p + "ffn_gate.weight", oracle.Q8_0, hidden, dim)
        linear(p + "ffn_up.weight", oracle.Q4_1, hidden, dim)
        linear(p + "ffn_down.weight", oracle.Q4_0, dim, hidden)
    tensors.append(gw.f32_tensor("output_norm.weight", np.ones(dim, np.float32)))
    linear("output.weight", lm_qt, vocab, dim)
    gw.write(path, meta, tensors, alignment=64)
    return linears


REF_NAME = {"attn_q": "wq", "attn_k": "wk", "attn_v": "wv", "attn_output": "wo", "ffn_gate": "w_gate",
            "ffn_up": "w_up", "ffn_down": "w_down"}


def ref_name(gguf_name):
    if gguf_name == "output.weight":
        return "lm_head"
    _, layer, op, _ = gguf_name.split(".")
    return f"layers.{layer}.{REF_NAME[op]}"


def test_model_file_linears_match_reference_loader(lib, ref, orc, tmp_path):
    path = str(tmp_path / "tiny_quant.gguf")
    linears = tiny_model_file(orc, path)
    agree(ref, path)
    loaded = ref.gguf_model_linears(path, [ref_name(n) for n in linears])
    g = mlq_hip.GgufFile(path)
    try:
        infos = {t["name"]: t for t in g.tensors()}
        for name, (qt, rows, cols, blocks) in linears.items():
            rqt, rrows, rcols, rbytes = loaded[ref_name(name)]
            assert (rqt, rrows, rcols) == (qt, rows, cols), name
            t = infos[name]
            assert (t["dims"][1], t["dims"][0]) == (rows, cols)
            mine = g.tensor_bytes(name)
            assert np.array_equal(mine, rbytes), name
            assert np.array_equal(mine, blocks.ravel()), name
    finally:
        g.close()


def test_upload_rejects_non_linear_tensors(lib, orc, tmp_path):
    """Argument errors are caught before any device work (no GPU here)."""
    path = str(tmp_path / "tiny_quant.gguf")
    tiny_model_file(orc, path)
    g = mlq_hip.GgufFile(path)
    try:
        with pytest.raises(mlq_hip.MlqError, match="token_embd.weight is F32; only Q8_0, Q4_0 and Q4_1"):
            g.upload_weight("token_embd.weight")
        with pytest.raises(mlq_hip.MlqError, match="Missing tensor: blk.9.attn_q.weight"):
            g.upload_weight("blk.9.attn_q.weight")
    finally:
        g.close()


def test_upload_shape_checks(lib, tmp_path):
    """A quantized tensor that is not 2-D, or whose rows are not whole blocks,
    is refused with the upload's messages before any device work."""
    path = mutated(tmp_path, "shapes.gguf", gw.build([], [
        ("vec", [64], gw.GGML_Q8_0, bytes(2 * 34)),
        ("ragged", [48, 2], gw.GGML_Q4_0, bytes(3 * 18)),   # 96 values = 3 blocks, rows of 48 need 2 each
    ]))
    g = mlq_hip.GgufFile(path)
    try:
        with pytest.raises(mlq_hip.MlqError, match="HIP weight upload: expected 2D Q8_0 weight"):
            g.upload_weight("vec")
        with pytest.raises(mlq_hip.MlqError, match="Q4_0 block count mismatch, expected 4, got 3"):
            g.upload_weight("ragged")
    finally:
        g.close()

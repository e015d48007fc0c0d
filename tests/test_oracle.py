"""CPU tests that pin the oracle (oracle/oracle.cpp) before it is trusted.

Each function of the oracle is checked against something other than itself:
golden vectors written by the compiled reference (tests/golden/make_golden.py),
the reference's own known-answer tests (tests/test_quant.cpp), IEEE binary16
semantics computed independently in numpy/float64, fp64 brute force, and
invariants (thread-count invariance, round-trip bounds).  Where the compiled
reference shim is present it is compared live as well.
"""

import numpy as np
import pytest

import oracle
from tolerance import check_close

FMTS = {"q8_0": oracle.Q8_0, "q4_0": oracle.Q4_0, "q4_1": oracle.Q4_1}


def names(golden):
    return [str(n) for n in golden["names"]]


# ---------------------------------------------------------------- layouts
def test_block_sizes(orc):
    # tests/test_quant.cpp:8-12, 174-184; src/gguf.cpp:178-197
    assert oracle.BLOCK_BYTES == {oracle.Q8_0: 34, oracle.Q4_0: 18, oracle.Q4_1: 20}
    f = orc._fn("block_bytes", __import__("ctypes").c_size_t, [__import__("ctypes").c_int])
    assert [f(q) for q in (1, 2, 3)] == [34, 18, 20]
    assert f(0) == 0


# ---------------------------------------------------------------- fp16 codec
def test_fp16_decode_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.fp16_decode(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # NaN payloads survive (exp 31: 0x7f800000 | frac << 13)
    assert np.array_equal(got[nan].view(np.uint32) & 0x7FFFFF, (h[nan].astype(np.uint32) & 0x3FF) << 13)


def rna_binary16(v: np.ndarray) -> np.ndarray:
    """Round-to-nearest, ties-away-from-zero f32 -> binary16, computed from
    exact float64 distances between the neighbouring binary16 values.
    Overflow (|v| >= 65520, i.e. at or past the tie with 65536) gives Inf."""
    v = v.astype(np.float32)
    a = np.abs(v.astype(np.float64))
    # all non-negative finite binary16 values, ascending
    table = np.arange(0x7C00, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float64)
    idx = np.searchsorted(table, a, side="right") - 1  # largest value <= a
    idx = np.clip(idx, 0, len(table) - 1)
    lo = table[idx]
    hi = np.where(idx + 1 < len(table), table[np.minimum(idx + 1, len(table) - 1)], 65536.0)
    pick_hi = (a - lo) >= (hi - a)  # ties go up in magnitude
    bits = np.where(pick_hi, idx + 1, idx).astype(np.uint32)
    bits = np.where(a >= 65520.0, 0x7C00, bits)
    sign = (v.view(np.uint32) >> 16) & 0x8000
    return (bits | sign).astype(np.uint16)


def test_fp16_encode_matches_rna(orc):
    rng = np.random.default_rng(11)
    # every binary16 bucket boundary: midpoints and their f32 neighbours
    h = np.arange(0x7C00, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float64)
    mids = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    probes = [mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(np.inf)),
              h.astype(np.float32),
              np.float32(2.0) ** rng.uniform(-30, 17, 200000).astype(np.float32),
              np.array([0.0, 2 ** -25, 2 ** -26, 3 * 2 ** -26, 65504, 65519.996, 65520, 1e30,
                        np.finfo(np.float32).tiny, 1e-45], np.float32)]
    v = np.concatenate(probes).astype(np.float32)
    v = np.concatenate([v, -v])
    assert np.array_equal(orc.fp16_encode(v), rna_binary16(v))


def test_fp16_encode_special(orc):
    enc = orc.fp16_encode(np.array([np.inf, -np.inf, np.nan, -np.nan, 0.0, -0.0], np.float32))
    # src/quant.cpp:39-41: exponent >= 31 (Inf and NaN) -> signed Inf
    assert list(enc) == [0x7C00, 0xFC00, 0x7C00, 0xFC00, 0x0000, 0x8000]


def test_fp16_encode_golden(orc, golden):
    v = golden["fp16_in"]
    assert np.array_equal(orc.fp16_encode(v), golden["fp16_out"])
    # the product copy of the encoder, observed as Q8_0 d = fp16(|v| / 127)
    v8 = v[:golden["fp16_q8_probe"].size]
    want = golden["fp16_q8_probe"]
    got = orc.fp16_encode((np.abs(v8) / np.float32(127.0)).astype(np.float32))
    got = np.where(np.abs(v8) > 0, got, 0)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- quantizers vs golden
@pytest.mark.parametrize("fmt", list(FMTS))
def test_quantize_golden(orc, golden, fmt):
    qt = FMTS[fmt]
    for n in names(golden):
        w = golden[f"{n}__w"]
        got = orc.quantize(qt, w, threads=3)
        assert np.array_equal(got, golden[f"{n}__{fmt}__blocks"]), f"{n} {fmt} blocks"
        key = f"{n}__{fmt}__deq"
        if key in golden:
            deq = orc.dequantize(qt, got, *w.shape)
            assert np.array_equal(deq.view(np.uint32), golden[key].view(np.uint32)), f"{n} {fmt} deq"


@pytest.mark.parametrize("fmt", list(FMTS))
def test_linear_golden_bits(orc, golden, fmt):
    qt = FMTS[fmt]
    for n in names(golden):
        w = golden[f"{n}__w"]
        x = golden[f"{n}__x"]
        blocks = golden[f"{n}__{fmt}__blocks"]
        want = golden[f"{n}__{fmt}__y"]
        for threads in (1, 4):
            got = orc.linear(qt, x, blocks, w.shape[0], threads=threads)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{n} {fmt} t={threads}"


def test_tiny_model_golden(orc, tiny):
    for n in tiny["names"]:
        key = str(n).replace(".", "_")
        w = tiny[f"{key}__w"]
        x = tiny[f"{key}__x"]
        for fmt, qt in FMTS.items():
            blocks = orc.quantize(qt, w)
            assert np.array_equal(blocks, tiny[f"{key}__{fmt}__blocks"]), f"{n} {fmt}"
            y = orc.linear(qt, x, blocks, w.shape[0])
            assert np.array_equal(y.view(np.uint32), tiny[f"{key}__{fmt}__y"].view(np.uint32))


def test_reference_shim_live(orc):
    """Where the compiled reference exists, compare it live on fresh inputs."""
    ref = oracle.reference()
    if ref is None:
        pytest.skip("oracle/_ref not built")
    rng = np.random.default_rng(5)
    for fmt, qt in FMTS.items():
        for m, k in [(37, 100), (64, 896), (19, 4096)]:
            w = (rng.standard_normal((m, k)) * 0.02).astype(np.float32)
            x = rng.standard_normal((2, k)).astype(np.float32)
            b = orc.quantize(qt, w)
            assert np.array_equal(b, ref.quantize(qt, w))
            assert np.array_equal(orc.linear(qt, x, b, m).view(np.uint32),
                                  ref.linear(qt, x, b, m, threads=2).view(np.uint32))


# ---------------------------------------------------------------- known answers (tests/test_quant.cpp)
def test_q4_1_dequant_known_values(orc):
    # tests/test_quant.cpp:221-236: d = fp16(0.5), m = fp16(-1), byte i = i | (15-i) << 4
    blk = np.zeros((1, 20), np.uint8)
    blk[0, 0:2] = np.array([0x3800], np.uint16).view(np.uint8)
    blk[0, 2:4] = np.array([0xBC00], np.uint16).view(np.uint8)
    blk[0, 4:] = [(i | ((15 - i) << 4)) for i in range(16)]
    out = orc.dequantize(oracle.Q4_1, blk, 1, 32)[0]
    i = np.arange(16)
    assert np.allclose(out[:16], -1.0 + 0.5 * i, atol=1e-6)
    assert np.allclose(out[16:], -1.0 + 0.5 * (15 - i), atol=1e-6)


def test_q4_1_linear_known_answer(orc):
    # tests/test_quant.cpp:238-251: d = 1, m = 0, all nibbles 1, x = 2 -> 64
    blk = np.zeros((1, 20), np.uint8)
    blk[0, 0:2] = np.array([0x3C00], np.uint16).view(np.uint8)
    blk[0, 4:] = 0x11
    y = orc.linear(oracle.Q4_1, np.full(32, 2.0, np.float32), blk, 1)
    assert y[0] == 64.0


def test_roundtrip_bounds(orc):
    # tests/test_quant.cpp:17-41, 55-76, 186-207
    src = (np.arange(32, dtype=np.float32) * np.float32(0.1))
    for qt, bound in ((oracle.Q8_0, 6e-2), (oracle.Q4_0, 3e-1)):
        b = orc.quantize(qt, src)
        assert b.shape[0] == 1
        assert np.abs(orc.dequantize(qt, b, 1, 32)[0] - src).max() < bound
    src = np.arange(100, dtype=np.float32) * np.float32(0.05)
    b = orc.quantize(oracle.Q8_0, src)
    assert b.shape[0] == 4
    assert np.abs(orc.dequantize(oracle.Q8_0, b, 1, 100)[0] - src).max() < 6e-2


def test_zero_blocks(orc):
    # tests/test_quant.cpp:43-53, 209-219; src/quant.cpp:157-159, 261-263
    z = np.zeros(64, np.float32)
    for qt in (oracle.Q8_0, oracle.Q4_0):
        b = orc.quantize(qt, z)
        assert b.shape[0] == 2 and not b.any()
        assert not orc.dequantize(qt, b, 1, 64).any()
    b = orc.quantize(oracle.Q4_1, np.full(32, 0.75, np.float32))
    d, m = b[0, 0:4].view(np.uint16)
    assert d == 0 and m == 0x3A00  # constant block: d = 0, m = fp16(min)


def test_q4_0_vs_f32_linear(orc):
    # tests/test_quant.cpp:253-274
    w = (np.arange(128, dtype=np.float32) * np.float32(0.05) - 1).reshape(4, 32)
    x = np.arange(32, dtype=np.float32) * np.float32(0.1) - np.float32(0.4)
    y = orc.linear(oracle.Q4_0, x, orc.quantize(oracle.Q4_0, w), 4)
    assert np.abs(y - w @ x).max() < 2.0


# ---------------------------------------------------------------- maths
@pytest.mark.parametrize("fmt", list(FMTS))
def test_dequant_closed_form(orc, fmt):
    """Element values follow d*q, d*(n-8), d*n+m from the raw bytes."""
    qt = FMTS[fmt]
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((9, 77)) * 0.05).astype(np.float32)
    b = orc.quantize(qt, w)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    nb = 3
    if qt == oracle.Q8_0:
        q = b[:, 2:].view(np.int8).astype(np.float32)
        deq = d[:, None] * q
    else:
        qs = b[:, 2:] if qt == oracle.Q4_0 else b[:, 4:]
        n = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.float32)
        if qt == oracle.Q4_0:
            deq = d[:, None] * (n - 8)
        else:
            m = b[:, 2:4].copy().view(np.float16).astype(np.float32).ravel()
            deq = (d[:, None] * n).astype(np.float32) + m[:, None]
    deq = deq.reshape(9, nb * 32)[:, :77].astype(np.float32)
    assert np.array_equal(orc.dequantize(qt, b, 9, 77).view(np.uint32), deq.view(np.uint32))
    # quantisation error within half a step (plus the fp16 rounding of m)
    err = np.abs(deq - w)
    step = np.repeat(d.reshape(9, nb), 32, axis=1)[:, :77]
    assert (err <= 0.5 * step * 1.0001 + 1e-3 * (qt == oracle.Q4_1)).all()


@pytest.mark.parametrize("fmt", list(FMTS))
def test_linear_brute_force_fp64(orc, fmt):
    """y equals sum(dequant(W) * x) up to the f32 rounding of a K-term sum."""
    qt = FMTS[fmt]
    rng = np.random.default_rng(4)
    for m, k in [(13, 45), (32, 64), (8, 1000)]:
        w = (rng.standard_normal((m, k)) * 0.02).astype(np.float32)
        x = rng.standard_normal((3, k)).astype(np.float32)
        b = orc.quantize(qt, w)
        deq = orc.dequantize(qt, b, m, k).astype(np.float64)
        exact = x.astype(np.float64) @ deq.T
        y = orc.linear(qt, x, b, m)
        bound = 2 * k * 2.0 ** -24 * (np.abs(x.astype(np.float64)) @ np.abs(deq).T) + 1e-30
        assert (np.abs(y - exact) <= bound).all()


def test_linear_thread_invariance(orc):
    # each output is owned by one thread in a fixed order (src/thread_pool.cpp:23-73)
    rng = np.random.default_rng(8)
    w = (rng.standard_normal((300, 256)) * 0.02).astype(np.float32)
    x = rng.standard_normal((2, 256)).astype(np.float32)
    b = orc.quantize(oracle.Q4_0, w)
    ys = [orc.linear(oracle.Q4_0, x, b, 300, threads=t).view(np.uint32) for t in (1, 2, 3, 8)]
    assert all(np.array_equal(ys[0], y) for y in ys[1:])


def test_linear_rejects_bad_block_count(orc):
    b = orc.quantize(oracle.Q8_0, np.ones((4, 64), np.float32))
    with pytest.raises(RuntimeError, match="block count mismatch: expected 8, got 7"):
        orc.linear(oracle.Q8_0, np.ones(64, np.float32), b[:7], 4)


def test_argmax_first_max(orc):
    assert orc.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert orc.argmax(np.array([-1], np.float32)) == 0


def test_checker_catches_planted_error(orc):
    """The parity checker itself: a one-ulp-scale perturbation passes, a dropped
    block (planted in the oracle's output on the CPU) fails."""
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((64, 4096)) * 0.02).astype(np.float32)
    x = rng.standard_normal(4096).astype(np.float32)
    b = orc.quantize(oracle.Q4_0, w)
    y = orc.linear(oracle.Q4_0, x, b, 64)
    check_close(y * np.float32(1 + 1e-6), y, x, oracle.Q4_0, b, "ulp")
    b2 = b.copy()
    b2[5 * 128 + 7, 0:2] = 0  # zero one block's scale in row 5
    y2 = orc.linear(oracle.Q4_0, x, b2, 64)
    with pytest.raises(AssertionError):
        check_close(y2, y, x, oracle.Q4_0, b, "planted")

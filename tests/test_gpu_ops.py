"""GPU parity of the device forward ops behind the reference's op-by-op device
interfaces (mlq_hip_rmsnorm / silu / mul / add / softmax / embedding / rope /
attention_decode / matmul_f32; include/mini_llama/cuda_ops.h,
cuda_attention.h, cuda_matmul.h), called through the C ABI at decode sizes
(LLaMA-7B: dim 4096, hidden 11008, 32 heads of 128; grouped and multi-query
attention, head_dim 8 / 64 / 128 / 256, positions 0 .. 1500), against float64
numpy restatements of the reference's CPU ops (src/ops.cpp:19-176;
attention: src/forward.cpp:580-600, scores q.k / sqrt(head_dim), softmax,
probability-weighted v).

Tolerances: the elementwise product and sum are one f32 rounding, so
bit-exact; the embedding lookup is a copy, bit-exact; everything else within
a few f32 ulps of the float64 value (relative 1e-5, or absolute 1e-5 of the
output scale), which the reference's own device tests (abs or rel 1e-4,
tests/test_cuda_ops.cpp:16-17) accept as well."""

import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(hip, a):
    return hip.DeviceBuffer.from_array(np.ascontiguousarray(a, np.float32))


def out(hip, n):
    return hip.DeviceBuffer(4 * max(1, n))


def got(hip, buf, n):
    hip.synchronize(hip.stream(0))
    return buf.download(np.float32, n)


def close(y, want, label, rel=1e-5):
    want = np.asarray(want, np.float64)
    scale = max(1.0, float(np.abs(want).max())) if want.size else 1.0
    err = np.abs(y.astype(np.float64) - want)
    bound = np.maximum(rel * np.abs(want), rel * scale)
    assert (err <= bound).all(), f"{label}: max err {err.max():.3e} (bound {bound[np.argmax(err)]:.3e})"


@pytest.mark.parametrize("n", [1, 5, 32, 4096, 11008])
def test_rmsnorm(hip, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    dx, dw, y = dev(hip, x), dev(hip, w), out(hip, n)
    hip._check(hip.load().mlq_hip_rmsnorm(0, dx.ptr, dw.ptr, n, ctypes.c_float(1e-5), y.ptr, None))
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 * x64).mean() + 1e-5) * w
    close(got(hip, y, n), want, f"rmsnorm {n}")


@pytest.mark.parametrize("n", [1, 255, 11008, 1 << 20])
def test_elementwise(hip, n):
    rng = np.random.default_rng(7 + n)
    a = (rng.standard_normal(n) * 4).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    da, db, y = dev(hip, a), dev(hip, b), out(hip, n)
    lib = hip.load()
    hip._check(lib.mlq_hip_mul(0, da.ptr, db.ptr, n, y.ptr, None))
    assert np.array_equal(got(hip, y, n), a * b), "mul"
    hip._check(lib.mlq_hip_add(0, da.ptr, db.ptr, n, y.ptr, None))
    assert np.array_equal(got(hip, y, n), a + b), "add"
    hip._check(lib.mlq_hip_silu(0, da.ptr, n, y.ptr, None))
    a64 = a.astype(np.float64)
    close(got(hip, y, n), a64 / (1.0 + np.exp(-a64)), "silu")


@pytest.mark.parametrize("n", [1, 7, 1000, 32000])
def test_softmax(hip, n):
    x = (np.random.default_rng(n).standard_normal(n) * 3).astype(np.float32)
    dx, y = dev(hip, x), out(hip, n)
    hip._check(hip.load().mlq_hip_softmax(0, dx.ptr, n, y.ptr, None))
    e = np.exp(x.astype(np.float64) - x.max())
    close(got(hip, y, n), e / e.sum(), f"softmax {n}")


def test_embedding(hip):
    vocab, dim = 300, 4096
    t = np.random.default_rng(1).standard_normal((vocab, dim)).astype(np.float32)
    table, y = dev(hip, t), out(hip, dim)
    for tok in (0, 17, vocab - 1):
        hip._check(hip.load().mlq_hip_embedding(0, table.ptr, vocab, dim, tok, y.ptr, None))
        assert np.array_equal(got(hip, y, dim), t[tok])
    rc = hip.load().mlq_hip_embedding(0, table.ptr, vocab, dim, vocab, y.ptr, None)
    assert rc != 0 and "token id out of range" in hip.last_error()


def rope_ref(x, pos, theta, neox):
    """src/ops.cpp:109-141 with the frequency and angle rounded to f32 as there."""
    nh, hd = x.shape
    y = x.astype(np.float64).copy()
    half = hd // 2
    for i in range(half):
        freq = np.float32(1.0) / np.float32(np.power(np.float64(theta), np.float64(np.float32(2 * i) / np.float32(hd))))
        ang = np.float64(np.float32(pos) * np.float32(freq))
        c, s = np.cos(ang), np.sin(ang)
        i0, i1 = (i, i + half) if neox else (2 * i, 2 * i + 1)
        x0, x1 = x[:, i0].astype(np.float64), x[:, i1].astype(np.float64)
        y[:, i0] = x0 * c - x1 * s
        y[:, i1] = x0 * s + x1 * c
    return y


@pytest.mark.parametrize("neox", [0, 1], ids=["normal", "neox"])
@pytest.mark.parametrize("heads,hd,pos", [(4, 8, 3), (32, 128, 0), (32, 128, 1000), (8, 256, 77)])
def test_rope(hip, neox, heads, hd, pos):
    x = np.random.default_rng(hd + pos).standard_normal((heads, hd)).astype(np.float32)
    d = dev(hip, x)
    hip._check(hip.load().mlq_hip_rope(0, d.ptr, heads, hd, pos, ctypes.c_float(10000.0), neox, None))
    # |angle| up to 1000 rad: the f32 angle itself carries ~6e-5 absolute, so
    # the bound is that of the rounding of pos * freq, not of the rotation.
    close(got(hip, d, heads * hd).reshape(heads, hd), rope_ref(x, pos, 10000.0, neox), f"rope {heads}x{hd}@{pos}",
          rel=1e-5 if pos < 100 else 1e-4)


def attention_ref(q, K, V, layer, pos, n_heads, n_kv, hd):
    out = np.zeros((n_heads, hd))
    g = n_heads // n_kv
    for h in range(n_heads):
        kh = h // g
        k = K[layer, : pos + 1, kh].astype(np.float64)
        v = V[layer, : pos + 1, kh].astype(np.float64)
        s = k @ q[h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v
    return out


@pytest.mark.parametrize("n_heads,n_kv,hd,max_seq,pos", [
    (4, 4, 8, 128, 0), (4, 4, 8, 128, 9), (32, 8, 128, 2048, 1500), (32, 32, 128, 256, 255),
    (8, 1, 64, 512, 300), (2, 1, 256, 64, 63), (2, 2, 512, 16, 5)])
def test_attention_decode(hip, n_heads, n_kv, hd, max_seq, pos):
    layers, layer = 2, 1
    rng = np.random.default_rng(n_heads * 1000 + hd + pos)
    K = rng.standard_normal((layers, max_seq, n_kv, hd)).astype(np.float32)
    V = rng.standard_normal((layers, max_seq, n_kv, hd)).astype(np.float32)
    q = rng.standard_normal((n_heads, hd)).astype(np.float32)
    dq, dk, dv, o = dev(hip, q), dev(hip, K), dev(hip, V), out(hip, n_heads * hd)
    say(f"attention {n_heads}/{n_kv} heads of {hd}, position {pos} of {max_seq}")
    hip._check(hip.load().mlq_hip_attention_decode(0, dq.ptr, dk.ptr, dv.ptr, layers, layer, max_seq, n_heads, n_kv,
                                                    hd, pos, o.ptr, None))
    close(got(hip, o, n_heads * hd).reshape(n_heads, hd), attention_ref(q, K, V, layer, pos, n_heads, n_kv, hd),
          f"attention {n_heads}x{hd}@{pos}")


def test_attention_rejects_bad_positions(hip):
    q, kv, o = out(hip, 64), out(hip, 2 * 16 * 64), out(hip, 64)
    lib = hip.load()
    assert lib.mlq_hip_attention_decode(0, q.ptr, kv.ptr, kv.ptr, 2, 0, 16, 1, 1, 64, 16, o.ptr, None) != 0
    assert "position out of range" in hip.last_error()
    assert lib.mlq_hip_attention_decode(0, q.ptr, kv.ptr, kv.ptr, 2, 2, 16, 1, 1, 64, 0, o.ptr, None) != 0
    assert "layer out of range" in hip.last_error()
    # a cache buffer smaller than the extents claim is refused before any launch
    assert lib.mlq_hip_attention_decode(0, q.ptr, kv.ptr, kv.ptr, 2, 0, 32, 1, 1, 64, 0, o.ptr, None) != 0
    assert "too small" in hip.last_error()


@pytest.mark.parametrize("m,k,n", [(1, 32, 86), (5, 13, 7), (64, 96, 40), (128, 4096, 33)])
@pytest.mark.parametrize("bt", [0, 1], ids=["b_kn", "b_nk"])
def test_matmul_f32(hip, m, k, n, bt):
    rng = np.random.default_rng(m + k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k) if bt else (k, n)).astype(np.float32)
    da, db, c = dev(hip, a), dev(hip, b), out(hip, m * n)
    hip._check(hip.load().mlq_hip_matmul_f32(0, da.ptr, db.ptr, m, k, n, bt, c.ptr, None))
    want = a.astype(np.float64) @ (b.astype(np.float64).T if bt else b.astype(np.float64))
    close(got(hip, c, m * n).reshape(m, n), want, f"matmul {m}x{k}x{n}", rel=1e-5 * max(1.0, np.sqrt(k) / 8))


def test_device_props(hip):
    p = hip.device_props(0)
    say(p)
    assert p["arch"].startswith("gfx950") and (p["major"], p["minor"]) == (9, 5)
    assert p["total_memory_bytes"] > 0 and p["compute_units"] > 0
    assert p["driver_version"] > 0 and p["runtime_version"] > 0

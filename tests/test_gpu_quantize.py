"""The device quantizer (mlq_hip_quantize) against the oracle / reference bytes.

Bit-exact: the same f32 weights must give the same block bytes as
quantize_to_q8_0 / quantize_to_q4_0 (src/quant.cpp:112-170, 207-270) and the
Q4_1 test quantizer (tests/test_cuda_quant.cpp:129-180)."""

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

FMTS = {"q8_0": oracle.Q8_0, "q4_0": oracle.Q4_0, "q4_1": oracle.Q4_1}


def device_quantize(hip, qt, w):
    rows, k = w.shape
    nb = (k + 31) // 32
    src = hip.DeviceBuffer.from_array(np.ascontiguousarray(w, np.float32))
    dst = hip.DeviceBuffer(rows * nb * oracle.BLOCK_BYTES[qt])
    dst.fill(0xAB)
    hip.quantize_device(qt, src, rows, k, dst)
    hip.synchronize(hip.stream(0))
    return dst.download(np.uint8).reshape(rows * nb, oracle.BLOCK_BYTES[qt])


@pytest.mark.parametrize("fmt", list(FMTS))
def test_device_quantizer_golden(hip, golden, fmt):
    qt = FMTS[fmt]
    for n in golden["names"]:
        n = str(n)
        w = golden[f"{n}__w"]
        print(f"quantize golden {n} {fmt}", flush=True)
        assert np.array_equal(device_quantize(hip, qt, w), golden[f"{n}__{fmt}__blocks"]), n


@pytest.mark.parametrize("fmt", list(FMTS))
def test_device_quantizer_random_and_special(hip, orc, fmt):
    qt = FMTS[fmt]
    rng = np.random.default_rng(21)
    cases = []
    cases.append((rng.standard_normal((64, 4096), dtype=np.float32) * np.float32(0.02)))
    cases.append((rng.standard_normal((33, 86), dtype=np.float32)))
    w = rng.standard_normal((16, 96), dtype=np.float32)
    w[0] = 0.0                                  # all-zero blocks
    w[1] = 3.0                                  # constant blocks
    w[2, :32] = np.float32(1e-30)               # scale underflows fp16
    w[3] *= np.float32(1e6)                     # scale overflows fp16 -> inf
    w[4, 5] = np.float32(65519.996)             # near the fp16 top
    w[5] = np.round(w[5] * 8) / 8               # exact ties in q
    w[6, ::2] = -w[6, 1::2]
    cases.append(w)
    t = rng.standard_normal((8, 4095), dtype=np.float32)  # tail block of 31
    cases.append(t)
    for w in cases:
        w = np.ascontiguousarray(w, np.float32)
        print(f"quantize {fmt} {w.shape}", flush=True)
        assert np.array_equal(device_quantize(hip, qt, w), orc.quantize(qt, w, threads=4)), w.shape


def test_fill_normal_moments(hip):
    n = 1 << 22
    buf = hip.DeviceBuffer(4 * n)
    hip.fill_normal(buf, n, seed=123, mean=0.0, std=0.02)
    hip.synchronize(hip.stream(0))
    v = buf.download(np.float32)
    assert np.isfinite(v).all()
    assert abs(float(v.mean())) < 1e-4
    assert abs(float(v.std()) - 0.02) < 2e-4
    buf2 = hip.DeviceBuffer(4 * n)
    hip.fill_normal(buf2, n, seed=123, mean=0.0, std=0.02)
    hip.synchronize(hip.stream(0))
    assert np.array_equal(buf2.download(np.float32).view(np.uint32), v.view(np.uint32))


def test_extent_checks_refuse_short_buffers(hip):
    """Buffers shorter than the shape implies are refused on the host, before
    any launch (the C ABI checks every device pointer's allocation extent).
    Buffers are 2 MiB so that allocation rounding cannot hide the overrun."""
    lib = hip.load()
    two_mib = 2 << 20
    buf = hip.DeviceBuffer(two_mib)
    rc = lib.mlq_hip_fill_normal(buf.ptr, two_mib // 4 + 1, 1, 0.0, 1.0, None)
    assert rc == 6 and "buffer is too small" in hip.last_error()
    rows, k = 2048, 1024                      # 8 MiB of f32, 2048*32*18 = 1.1 MiB of blocks
    src = hip.DeviceBuffer(two_mib)           # too short for the source
    dst = hip.DeviceBuffer(two_mib)
    rc = lib.mlq_hip_quantize(0, 2, src.ptr, rows, k, dst.ptr, None)
    assert rc == 6 and "source buffer is too small" in hip.last_error()
    src2 = hip.DeviceBuffer(8 << 20)
    rc = lib.mlq_hip_quantize(0, 1, src2.ptr, rows, k, dst.ptr, None)  # Q8_0 needs 2.1 MiB
    assert rc == 6 and "block buffer is too small" in hip.last_error()
    k = two_mib // 4 + 32
    nb = (k + 31) // 32
    wb = hip.DeviceBuffer(4 * nb * 18)
    x = hip.DeviceBuffer(two_mib)
    y = hip.DeviceBuffer(16)
    rc = lib.mlq_hip_quant_linear_device(0, 2, wb.ptr, 4 * nb, 4, k, x.ptr, 1, y.ptr, None)
    assert rc == 6 and "input buffer is too small" in hip.last_error()

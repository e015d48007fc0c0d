"""mlq_hip_quant_linear_noalloc (the entry point that allocates nothing: the
batched GEMM's workspace comes from the library's fixed scratch array) against
the existing mlq_hip_quant_linear on the same inputs, bit for bit: two calls in
a row with the second smaller, every format, GEMV and GEMM rows; the refusal
of a shape whose GEMM needs more scratch than the array holds; and the first
batched call of a fresh stream made under graph capture, replayed with eager
work in between."""

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

FMTS = {"q8_0": oracle.Q8_0, "q4_0": oracle.Q4_0, "q4_1": oracle.Q4_1}


def weight(hip, qt, m, k, seed):
    nb = (k + 31) // 32
    f = hip.DeviceBuffer(4 * m * k)
    hip.fill_normal(f, m * k, seed, 0.0, 0.02)
    buf = hip.DeviceBuffer(m * nb * hip.BLOCK_BYTES[qt])
    hip.quantize_device(qt, f, m, k, buf)
    f.free()
    return hip.Weight.wrap(qt, buf, m * nb, m, k), buf


def bits(buf):
    return buf.download(np.float32).view(np.uint32)


@pytest.mark.parametrize("fmt", list(FMTS))
def test_noalloc_equals_existing_entry(hip, fmt):
    qt = FMTS[fmt]
    m, k = 4096, 4096
    w, keep = weight(hip, qt, m, k, 11 + qt)
    s = hip.stream_create(0)
    for rows in (64, 16, 1, 512, 3):  # each call after a larger one, then a larger one again
        print(f"noalloc {fmt} {m}x{k} rows={rows}", flush=True)
        x = hip.DeviceBuffer(4 * rows * k)
        # x on the calls' own stream: filled on the device's default stream it
        # could still be in flight when the first call on `s` reads it
        hip.fill_normal(x, rows * k, 100 + rows, 0.0, 1.0, stream=s)
        y_ref, y = hip.DeviceBuffer(4 * rows * m), hip.DeviceBuffer(4 * rows * m)
        w.linear_device(x, y_ref, rows=rows, stream=s)  # existing entry (stream workspace)
        y.fill(0)
        w.linear_noalloc(x, y, rows=rows, stream=s)
        hip.synchronize(s)
        assert np.array_equal(bits(y), bits(y_ref)), f"{fmt} rows={rows}"
        for b in (x, y, y_ref):
            b.free()
    hip.stream_destroy(s)
    w.free()
    keep.free()


def test_noalloc_refuses_shapes_beyond_the_scratch(hip):
    m, k, rows = 4096, 4096, 4096  # the GEMM would need 66 MiB of workspace
    w, keep = weight(hip, oracle.Q4_0, m, k, 5)
    x, y = hip.DeviceBuffer(4 * rows * k), hip.DeviceBuffer(4 * rows * m)
    with pytest.raises(hip.MlqError, match="no-allocation entry point has .* bytes of scratch"):
        w.linear_noalloc(x, y, rows=rows)
    # a shape that fits still runs after the refusal
    w.linear_noalloc(x, y, rows=2048)
    hip.synchronize()
    for b in (x, y, keep):
        b.free()
    w.free()


def test_noalloc_first_call_under_graph_capture(hip):
    """A fresh stream's first batched call recorded in a graph (the existing
    entry refuses this: its workspace is created by a first eager call)."""
    m, k, rows = 4096, 4096, 64
    w, keep = weight(hip, oracle.Q4_0, m, k, 7)
    s = hip.stream_create(0)
    x = hip.DeviceBuffer(4 * rows * k)
    y = hip.DeviceBuffer(4 * rows * m)
    y_ref = hip.DeviceBuffer(4 * rows * m)
    g = hip.Graph.record(lambda: w.linear_noalloc(x, y, rows=rows, stream=s), s, keep=(x, y))
    for rep in range(3):
        hip.fill_normal(x, rows * k, 300 + rep, 0.0, 1.0)
        hip.synchronize()
        y.fill(0)
        print(f"noalloc graph replay {rep}", flush=True)
        g.launch(s)
        hip.synchronize(s)
        w.linear_device(x, y_ref, rows=rows)  # eager work between replays
        hip.synchronize()
        assert np.array_equal(bits(y), bits(y_ref)), f"replay {rep}"
    g.destroy()
    hip.stream_destroy(s)
    for b in (x, y, y_ref, keep):
        b.free()
    w.free()

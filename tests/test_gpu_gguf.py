"""GGUF ingest on the device: weights uploaded from a mapped model file
(mlq_hip_gguf_upload_weight) hold the file's block bytes exactly, and the
linear on them equals the linear on the same blocks uploaded from host memory
(bit for bit) and the CPU oracle (within the parity bound).  Files are written
by tests/gguf_writer.py; the tensor layout the reference loader reads from
such files is checked on the CPU in tests/test_gguf.py."""

import os
import sys

import numpy as np
import pytest

import gguf_writer as gw
import oracle
from tolerance import check_close
from test_gguf import QT_GGML, tiny_model_file

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def device_bytes(hip, w, nbytes):
    import ctypes

    qt, m, k, nblk, ptr, dev = (ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_size_t(),
                                ctypes.c_void_p(), ctypes.c_int())
    hip._check(hip.load().mlq_hip_weight_info(w.h, ctypes.byref(qt), ctypes.byref(m), ctypes.byref(k),
                                               ctypes.byref(nblk), ctypes.byref(ptr), ctypes.byref(dev)))
    out = np.empty(nbytes, np.uint8)
    hip._check(hip.load().mlq_hip_memcpy_dtoh(out.ctypes.data, ptr.value, nbytes))
    return out


@pytest.mark.parametrize("qt", [oracle.Q8_0, oracle.Q4_0, oracle.Q4_1], ids=["q8_0", "q4_0", "q4_1"])
def test_ingest_lm_head_sized_weight(hip, orc, tmp_path, qt):
    """32000 x 4096 (74-139 MB: several 16 MiB pieces through the pinned
    stage) next to a small tensor, at a 4 KiB alignment."""
    m, k = 32000, 4096
    rng = np.random.default_rng(5 + qt)
    w = (rng.standard_normal((m, k), dtype=np.float32) * np.float32(0.02))
    blocks = orc.quantize(qt, w, threads=THREADS)
    small = orc.quantize(qt, w[:7, :64].copy(), threads=THREADS)
    path = str(tmp_path / "lm.gguf")
    gw.write(path, [("general.architecture", gw.STRING, "llama")],
             [gw.linear_tensor("small.weight", QT_GGML[qt], small, 7, 64),
              gw.linear_tensor("output.weight", QT_GGML[qt], blocks, m, k)], alignment=4096)
    g = hip.GgufFile(path)
    say(f"gguf ingest {m}x{k} qt={qt}")
    wt = g.upload_weight("output.weight")
    assert (wt.m, wt.k, wt.qtype) == (m, k, qt)
    assert np.array_equal(device_bytes(hip, wt, blocks.size), blocks.ravel())
    ws = g.upload_weight("small.weight")
    assert np.array_equal(device_bytes(hip, ws, small.size), small.ravel())
    x = rng.standard_normal(k, dtype=np.float32)
    y = wt.linear_host(x)
    host = hip.Weight.upload(qt, blocks, m, k)
    assert np.array_equal(y.view(np.uint32), host.linear_host(x).view(np.uint32))
    check_close(y, orc.linear(qt, x, blocks, m, threads=THREADS), x, qt, blocks, "gguf lm_head")
    for h in (wt, ws, host):
        h.free()
    g.close()


def test_ingest_whole_model_file(hip, orc, tmp_path):
    """Every quantized linear of a 2-layer model file: device bytes equal the
    blocks written, and each linear agrees with the oracle."""
    path = str(tmp_path / "tiny_quant.gguf")
    linears = tiny_model_file(orc, path)
    g = hip.GgufFile(path)
    rng = np.random.default_rng(9)
    for name, (qt, rows, cols, blocks) in linears.items():
        wt = g.upload_weight(name)
        assert (wt.m, wt.k, wt.qtype) == (rows, cols, qt), name
        assert np.array_equal(device_bytes(hip, wt, blocks.size), blocks.ravel()), name
        x = rng.standard_normal(cols, dtype=np.float32)
        check_close(wt.linear_host(x), orc.linear(qt, x, blocks, rows), x, qt, blocks, name)
        wt.free()
    g.close()

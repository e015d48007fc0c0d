"""GPU parity of the batched prefill GEMM (rows > 1, MFMA path) against the oracle.

X f32 N(0,1) with N = 16 / 64 / 512 token rows, W Q8_0
and Q4_0 at 4096x4096 and 11008x4096 (N(0,0.02), reference quantiser); Q4_1
and ragged shapes in addition.  Bound: tests/tolerance.py (BASELINE and the
reference's own criterion)."""

import os
import sys

import numpy as np
import pytest

import oracle
from tolerance import check_close

pytestmark = pytest.mark.gpu

FMTS = {"q8_0": oracle.Q8_0, "q4_0": oracle.Q4_0, "q4_1": oracle.Q4_1}
THREADS = min(16, os.cpu_count() or 1)


def run(hip, orc, qt, m, k, n, seed=0, scale_rows=None):
    rng = np.random.default_rng(500 + m + k + n + seed)
    w = (rng.standard_normal((m, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = rng.standard_normal((n, k), dtype=np.float32)
    if scale_rows is not None:
        x *= np.asarray(scale_rows, np.float32)[:, None]
    blocks = orc.quantize(qt, w, threads=THREADS)
    want = orc.linear(qt, x, blocks, m, threads=THREADS)
    name = hip.kernel_name(qt, n, m, k)
    print(f"gemm qt={qt} M={m} K={k} N={n} kernel={name}", flush=True)
    wt = hip.Weight.upload(qt, blocks, m, k)
    got = wt.linear_host(x)
    wt.free()
    return name, check_close(got, want, x, qt, blocks, f"gemm qt={qt} {m}x{k} N={n}")


@pytest.mark.parametrize("n", [16, 64, 512])
@pytest.mark.parametrize("shape", [(4096, 4096), (11008, 4096)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_gemm_baseline_config4(hip, orc, shape, n):
    for fmt in ("q8_0", "q4_0"):
        name, _ = run(hip, orc, FMTS[fmt], *shape, n)
        assert name.startswith("gemm_mfma"), name


@pytest.mark.parametrize("shape", [(4096, 4096), (4096, 11008)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_gemm_256_tokens_two_splits(hip, orc, shape):
    """256 token rows (x split once, 256 tiles: two K splits and their reduction)."""
    for fmt, qt in FMTS.items():
        name, _ = run(hip, orc, qt, *shape, 256)
        assert "splitk2" in name, name


@pytest.mark.parametrize("m,k,n", [(4096, 4096, 16), (64, 64, 2), (33, 4096, 17), (300, 896, 40),
                                   (4864, 896, 7), (17, 64, 100), (1000, 11008, 3), (520, 4096, 130),
                                   (300, 896, 200), (200, 4096, 96),
                                   # either side of the in-kernel x split (up to 128 token rows)
                                   (300, 4096, 128), (300, 4096, 129),
                                   # 130 blocks per row: not a whole number of 4-block chunks
                                   (300, 4160, 40), (300, 4160, 200)])
def test_gemm_q4_1_and_ragged(hip, orc, m, k, n):
    for fmt, qt in FMTS.items():
        run(hip, orc, qt, m, k, n)


def test_gemm_wide_dynamic_range(hip, orc):
    """Per-token power-of-two scaling keeps the hi/lo split exact across token
    magnitudes from 1e-6 to 1e4 (and an all-zero token)."""
    scales = [1e-6, 1.0, 1e4, 0.0, 3.5, 1e-3, 250.0, 1.0]
    for fmt, qt in FMTS.items():
        run(hip, orc, qt, 512, 4096, len(scales), scale_rows=scales)


def test_gemm_odd_block_count_uses_gemv_rows(hip, orc):
    # K=4095 has an even block count (tail 31); K=100 has 4 blocks; K=4064+32 odd count -> GEMV per row
    for m, k, n in [(64, 4095, 5), (64, 100, 3), (48, 4128, 4)]:
        for fmt, qt in FMTS.items():
            run(hip, orc, qt, m, k, n)


def test_graph_replay_after_workspace_growth(hip, orc):
    """A graph recorded with a stream's batched-call workspace keeps working
    after a larger eager call on the same stream grows that workspace (the old
    buffer is retired, not freed): every replay equals the eager result bit
    for bit."""
    qt, m, k = oracle.Q4_0, 4096, 4096
    rng = np.random.default_rng(77)
    w = (rng.standard_normal((m, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    blocks = orc.quantize(qt, w, threads=THREADS)
    wt = hip.Weight.upload(qt, blocks, m, k)
    sp = hip.stream_create(0)  # a stream with no workspace yet
    x16 = hip.DeviceBuffer.from_array(rng.standard_normal((16, k), dtype=np.float32))
    y16 = hip.DeviceBuffer(16 * m * 4)
    x512 = hip.DeviceBuffer.from_array(rng.standard_normal((512, k), dtype=np.float32))
    y512 = hip.DeviceBuffer(512 * m * 4)
    print("gemm workspace growth: eager N=16, record, eager N=512, replays", flush=True)
    wt.linear_device(x16, y16, rows=16, stream=sp)  # creates the stream's workspace (N=16 size)
    hip.synchronize(sp)
    want = y16.download(np.float32)
    g = hip.Graph(hip.make_calls([(wt, x16, y16, 16)]), sp)
    wt.linear_device(x512, y512, rows=512, stream=sp)  # grows the workspace
    hip.synchronize(sp)
    for i in range(3):
        y16.fill(0)
        g.launch(sp)
        hip.synchronize(sp)
        got = y16.download(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {i} differs"
        wt.linear_device(x512, y512, rows=512, stream=sp)  # eager work between replays
        hip.synchronize(sp)
    g.destroy()
    hip.stream_destroy(sp)
    wt.free()


def _fused_rows(hip, orc, qt, ms, k, n, seed):
    """mlq_hip_quant_linear_fused with `n` token rows over weights of ms rows
    sharing x: every output against the oracle, and the per-call results of
    mlq_hip_quant_linear for comparison."""
    rng = np.random.default_rng(900 + seed)
    x = rng.standard_normal((n, k), dtype=np.float32)
    blocks = [orc.quantize(qt, (rng.standard_normal((m, k), dtype=np.float32) * np.float32(0.02)), threads=THREADS)
              for m in ms]
    ws = [hip.Weight.upload(qt, b, m, k) for b, m in zip(blocks, ms)]
    xb = hip.DeviceBuffer.from_array(x)
    ys = [hip.DeviceBuffer(4 * n * m) for m in ms]
    print(f"fused gemm qt={qt} Ms={ms} K={k} N={n}", flush=True)
    hip.linear_fused(hip.make_calls([(w, xb, y, n) for w, y in zip(ws, ys)]))
    hip.synchronize()
    got = [y.download(np.float32, n * m).reshape(n, m) for y, m in zip(ys, ms)]
    single = [w.linear_host(x) for w in ws]
    for g, b, m in zip(got, blocks, ms):
        check_close(g, orc.linear(qt, x, b, m, threads=THREADS), x, qt, b, f"fused qt={qt} M={m} N={n}")
    for w in ws:
        w.free()
    xb.free()
    for y in ys:
        y.free()
    return got, single


@pytest.mark.parametrize("ms,k,n", [((256, 128, 72), 896, 16), ((256, 128, 72), 896, 40), ((256, 128, 72), 896, 300),
                                    ((128, 256), 4096, 64), ((100, 128, 64), 896, 40), ((64, 64, 64, 64), 896, 20)],
                         ids=["g3_n16", "g3_n40", "g3_n300", "g2_n64", "ragged_first", "four_calls"])
def test_fused_batched_rows(hip, orc, ms, k, n):
    """Batched rows through the fused entry: the grouped GEMM (up to three
    weights, each but the last a whole number of row tiles) or, where the
    shapes do not allow it (a first weight of 100 rows, four calls), one
    launch per call -- every output within the tolerance of the oracle."""
    for fmt, qt in FMTS.items():
        _fused_rows(hip, orc, qt, ms, k, n, seed=len(ms) + n)


def test_fused_batched_qkv_512_rows_bit_identical(hip, orc):
    """q/k/v-shaped group at 512 rows: one K split at both the single-call and
    the group's total M, so the grouped launch must give every row the bits of
    mlq_hip_quant_linear."""
    for fmt in ("q4_0", "q8_0"):
        got, single = _fused_rows(hip, orc, FMTS[fmt], (4096, 4096, 4096), 4096, 512, seed=7)
        for i, (g, s) in enumerate(zip(got, single)):
            assert np.array_equal(g.view(np.uint32), s.view(np.uint32)), f"{fmt} call {i}"

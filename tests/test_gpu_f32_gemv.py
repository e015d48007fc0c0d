"""GPU parity of the f32 decode GEMV (mlq_hip_quant_linear_fused_f32: the
reference's arithmetic, src/quant.cpp:413-429 with the dequant functions of
src/quant.cpp:435-460 -- each weight dequantized to f32, f32 multiply-adds
with x) against the CPU oracle, through the C ABI.

Bound: tests/tolerance.py.  The worst error / bound is printed, not
bounded further: an f32 sum in another order differs from the CPU's
sequential f32 sum by about that sum's own rounding, which at K = 4096 is
already ~0.1 of the bound's floor for outputs near zero (the bench records
this path's margin beside the integer path's).  Shapes: BASELINE.json's
LLaMA-7B and Qwen2-0.5B linears, all three formats, a fused q/k/v group, a
one-pair row, a ragged tail block, and a row count that is not a multiple of
the grid's waves."""

import os

import numpy as np
import pytest

import oracle
from tolerance import check_close

pytestmark = pytest.mark.gpu

FMTS = {"q8_0": oracle.Q8_0, "q4_0": oracle.Q4_0, "q4_1": oracle.Q4_1}
THREADS = min(16, os.cpu_count() or 1)
MARGIN = 1.0  # the tolerance itself (check_close raises beyond it)


def run(hip, orc, qt, ms, k, seed):
    """One fused f32 launch over len(ms) weights sharing x; returns the worst
    error / bound over all outputs."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(k, dtype=np.float32)
    xd = hip.DeviceBuffer.from_array(x)
    ws, blocks, ys = [], [], []
    for i, m in enumerate(ms):
        w = (rng.standard_normal((m, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
        b = orc.quantize(qt, w, threads=THREADS)
        blocks.append(b)
        ws.append(hip.Weight.upload(qt, b, m, k))
        ys.append(hip.DeviceBuffer(4 * m))
    print(f"f32 gemv qt={qt} M={ms} K={k}", flush=True)
    hip.linear_fused_f32(hip.make_calls([(w, xd, y, 1) for w, y in zip(ws, ys)]))
    hip.synchronize()
    worst = 0.0
    for m, w, b, y in zip(ms, ws, blocks, ys):
        want = orc.linear(qt, x, b, m, threads=THREADS)
        got = y.download(np.float32)
        worst = max(worst, check_close(got, want, x, qt, b, f"f32 qt={qt} {m}x{k}"))
        w.free()
        y.free()
    xd.free()
    print(f"  worst error / bound {worst:.4f}", flush=True)
    return worst


@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("shape", [(4096, 4096), (11008, 4096), (4096, 11008), (32000, 4096), (896, 896),
                                   (4864, 896), (896, 4864), (128, 896)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_f32_gemv_shapes(hip, orc, fmt, shape):
    worst = run(hip, orc, FMTS[fmt], [shape[0]], shape[1], 11 + shape[0] + shape[1])
    assert worst < MARGIN, f"worst error {worst:.4f} of the bound"


@pytest.mark.parametrize("fmt", list(FMTS))
def test_f32_gemv_fused_group_and_edges(hip, orc, fmt):
    qt = FMTS[fmt]
    assert run(hip, orc, qt, [4096, 1024, 1024], 4096, 5) < MARGIN  # q/k/v (grouped-query sizes)
    assert run(hip, orc, qt, [37], 64, 6) < MARGIN                  # one pair per row, 37 rows
    assert run(hip, orc, qt, [300], 4030, 7) < MARGIN               # tail block of 30 elements

def test_f32_gemv_validation(hip, orc):
    w = hip.Weight.upload(oracle.Q4_0, orc.quantize(oracle.Q4_0, np.zeros((8, 64), np.float32)), 8, 64)
    x = hip.DeviceBuffer(4 * 2 * 64)
    y = hip.DeviceBuffer(4 * 2 * 8)
    with pytest.raises(hip.MlqError, match="one token row"):
        hip.linear_fused_f32(hip.make_calls([(w, x, y, 2)]))
    w.free()
    odd = hip.Weight.upload(oracle.Q4_0, orc.quantize(oracle.Q4_0, np.zeros((8, 96), np.float32)), 8, 96)
    with pytest.raises(hip.MlqError, match="even block count"):
        hip.linear_fused_f32(hip.make_calls([(odd, x, y, 1)]))
    odd.free()

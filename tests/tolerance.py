"""The parity criteria used by every GPU-vs-CPU comparison.

* BASELINE criterion (the north star's): per output
  |y_gpu - y_cpu| <= max(1e-3 * |y_cpu|, 1e-3 * ||x||_2 * max_b |d_b|),
  with ||x|| taken per x row and max |d| over all blocks of W.
* Reference criterion (tests/test_cuda_quant.cpp:23-36): abs err <= 1e-3, or
  abs err / max(1, |y_cpu|) <= 1e-3.
Both must hold, except where a caller passes reference_bound=False: inputs
whose products reach 1e6 and cancel to O(1), where fp32 rounding of any
summation order other than the CPU's exceeds an unscaled 1e-3 and the
BASELINE bound alone applies.
"""

import numpy as np

REL = 1e-3
ABS_REF = 1e-3


def block_scales(qtype: int, blocks: np.ndarray) -> np.ndarray:
    d = blocks[:, 0:2].copy().view(np.uint16).ravel()
    return d.view(np.float16).astype(np.float32)


def check_close(y_gpu, y_cpu, x, qtype, blocks, label="", reference_bound=True):
    y_gpu = np.asarray(y_gpu, np.float32)
    y_cpu = np.asarray(y_cpu, np.float32)
    assert y_gpu.shape == y_cpu.shape, f"{label}: shape {y_gpu.shape} vs {y_cpu.shape}"
    x = np.asarray(x, np.float32)
    k = x.shape[-1]
    xr = x.reshape(-1, k)
    xnorm = np.sqrt((xr.astype(np.float64) ** 2).sum(axis=1))  # per row
    dmax = float(np.abs(block_scales(qtype, blocks)).max()) if blocks.size else 0.0
    yg = y_gpu.reshape(xr.shape[0], -1).astype(np.float64)
    yc = y_cpu.reshape(xr.shape[0], -1).astype(np.float64)
    err = np.abs(yg - yc)
    floor = (REL * xnorm * dmax)[:, None]
    bound = np.maximum(REL * np.abs(yc), floor)
    bad = ~(err <= bound)
    ref_ok = (err <= ABS_REF) | (err / np.maximum(1.0, np.abs(yc)) <= REL)
    if not reference_bound:
        ref_ok = np.ones_like(bad)
    if bad.any() or (~ref_ok).any():
        i = np.unravel_index(np.argmax(err / np.maximum(bound, 1e-30)), err.shape)
        raise AssertionError(
            f"{label}: {int(bad.sum())} outputs outside the BASELINE bound, "
            f"{int((~ref_ok).sum())} outside the reference bound; worst at {i}: "
            f"gpu={yg[i]!r} cpu={yc[i]!r} err={err[i]:.3e} bound={bound[i]:.3e}")
    return float((err / np.maximum(bound, 1e-30)).max()) if err.size else 0.0

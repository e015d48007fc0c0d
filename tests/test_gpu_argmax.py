"""GPU parity of the fused greedy pick (lm_head GEMV + argmax).

mlq_hip_quant_linear_argmax / mlq_hip_sample_greedy replace downloading the
logits and picking on the host: MiniSampler::sample_greedy
(src/sampler.cpp:91-95) = validate_logits (src/sampler.cpp:15-24, throws
"sampler: logits must be finite") then argmax (src/ops.cpp:179-192, first
index of the maximum).  Checked here, through the C ABI:
* the y the picking launch writes is bit-identical to the plain GEMV's;
* the token is the oracle's argmax (mlq_oracle_argmax, first maximum) of that
  same y, and -1 / the reference's error message when a logit is not finite;
* against the CPU oracle's y: within the parity bound, and the oracle's own
  greedy token is the same unless its top two logits lie within that bound;
* ties planted across workgroups (duplicated weight rows), +0/-0 ties, and
  the per-stream state being reused across launches of every grid size.
"""

import os
import sys

import numpy as np
import pytest

import oracle
from tolerance import REL, block_scales, check_close

pytestmark = pytest.mark.gpu

FMTS = {"q8_0": oracle.Q8_0, "q4_0": oracle.Q4_0, "q4_1": oracle.Q4_1}
THREADS = min(16, os.cpu_count() or 1)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def make(orc, qt, m, k, seed=0):
    rng = np.random.default_rng(500 + 3 * m + 5 * k + seed)
    w = (rng.standard_normal((m, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = rng.standard_normal(k, dtype=np.float32)
    return orc.quantize(qt, w, threads=THREADS), x


def want_token(orc, y):
    """sample_greedy's answer on logits y: -1 where validate_logits throws."""
    if not np.isfinite(y).all():
        return -1
    return orc.argmax(y)


def pick(hip, orc, qt, blocks, m, k, x, label):
    """Runs the picking launch (with y, and without y through the synchronous
    entry) next to the plain GEMV; returns (y, token)."""
    say(f"pick {label} M={m} K={k} kernel={hip.kernel_name(qt, 1, m, k)}")
    wt = hip.Weight.upload(qt, blocks, m, k)
    xb = hip.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    y_plain = hip.DeviceBuffer(4 * m)
    y_pick = hip.DeviceBuffer(4 * m)
    tok = hip.DeviceBuffer(4)
    tok.upload(np.array([12345], np.int32))
    wt.linear_device(xb, y_plain)
    wt.linear_argmax(xb, y_pick, tok)
    hip.synchronize()
    yp = y_plain.download(np.float32, m)
    yk = y_pick.download(np.float32, m)
    t = int(tok.download(np.int32, 1)[0])
    assert np.array_equal(yp.view(np.uint32), yk.view(np.uint32)), f"{label}: picking launch changed y"
    assert t == want_token(orc, yk), f"{label}: token {t}, oracle argmax of the same y {want_token(orc, yk)}"
    if t >= 0:
        assert wt.sample_greedy(xb) == t, f"{label}: synchronous entry disagrees"
    else:
        with pytest.raises(hip.MlqError, match="sampler: logits must be finite"):
            wt.sample_greedy(xb)
    for b in (xb, y_plain, y_pick, tok):
        b.free()
    wt.free()
    return yk, t


def check_against_oracle(orc, qt, blocks, m, x, y, t, label):
    y_cpu = orc.linear(qt, x, blocks, m, threads=THREADS)
    check_close(y, y_cpu, x, qt, blocks, label)
    t_cpu = orc.argmax(y_cpu)
    if t_cpu != t:
        # Only a near tie may pick differently: both logits within the bound.
        floor = REL * float(np.sqrt((x.astype(np.float64) ** 2).sum())) * float(np.abs(block_scales(qt, blocks)).max())
        bound = 2 * max(REL * abs(float(y_cpu[t_cpu])), floor)
        gap = float(y_cpu[t_cpu]) - float(y_cpu[t])
        assert gap <= bound, f"{label}: GPU token {t}, oracle {t_cpu}, oracle gap {gap:.3e} > {bound:.3e}"
    return t_cpu == t


# lm_head shapes of BASELINE configs 2 and 3, and the other 7B shapes (the
# multi-chunk kernel at K = 11008).
@pytest.mark.parametrize("shape", [(151936, 896), (32000, 4096), (11008, 4096), (4096, 11008)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_pick_full_shapes(hip, orc, shape):
    m, k = shape
    for fmt, qt in FMTS.items():
        blocks, x = make(orc, qt, m, k)
        y, t = pick(hip, orc, qt, blocks, m, k, x, fmt)
        assert check_against_oracle(orc, qt, blocks, m, x, y, t, f"{fmt} {m}x{k}")


# Every kernel family: one 16-lane or 64-lane row group, several chunks,
# and the generic kernel (odd block counts, K beyond the LDS budget).
@pytest.mark.parametrize("shape", [(1, 32), (5, 13), (7, 33), (17, 65), (3, 4095), (300, 4096),
                                   (64, 4160), (40, 20000), (1001, 4095), (2500, 896)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_pick_small_and_ragged(hip, orc, shape):
    m, k = shape
    for fmt, qt in FMTS.items():
        blocks, x = make(orc, qt, m, k, seed=1)
        y, t = pick(hip, orc, qt, blocks, m, k, x, fmt)
        check_against_oracle(orc, qt, blocks, m, x, y, t, f"{fmt} {m}x{k}")


@pytest.mark.parametrize("shape", [(32000, 4096), (20000, 896), (3000, 11008), (1001, 4095)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_pick_ties_take_first_index(hip, orc, shape):
    """Copies of the maximal row placed before and after it (other workgroups
    and fold groups): the lowest copy wins, as the reference's strict '>'."""
    m, k = shape
    qt = oracle.Q4_0
    blocks, x = make(orc, qt, m, k, seed=2)
    nb = (k + 31) // 32
    _, a = pick(hip, orc, qt, blocks, m, k, x, "untied")
    rows = blocks.reshape(m, nb, -1)
    for lo in sorted({m // 3, 1, m - 2} - {a}):
        tied = rows.copy()
        tied[lo] = rows[a]
        tied[m - 1] = rows[a]
        y, t = pick(hip, orc, qt, tied.reshape(m * nb, -1), m, k, x, f"tie {lo}/{a}/{m - 1}")
        assert y[lo] == y[a] == y[m - 1]
        assert t == min(lo, a), f"tie at rows {lo}, {a}, {m - 1}: token {t}"


def test_pick_signed_zero_ties(hip, orc):
    """All scales +0 or -0: every logit is +0 or -0, which compare equal, so
    the pick is row 0 whatever the signs."""
    m, k = 4096, 4096
    for fmt, qt in FMTS.items():
        blocks, x = make(orc, qt, m, k, seed=3)
        z = blocks.copy()
        d = np.zeros(z.shape[0], np.uint16)
        d[1::3] = 0x8000
        z[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
        if qt == oracle.Q4_1:
            z[:, 2:4] = 0  # m = +0
        y, t = pick(hip, orc, qt, z, m, k, x, f"{fmt} zero scales")
        assert (y == 0).all()
        assert t == 0


def test_pick_nonfinite_logits(hip, orc):
    m, k = 32000, 4096
    qt = oracle.Q4_0
    nb = k // 32
    blocks, x = make(orc, qt, m, k, seed=4)
    # One infinite scale in the last row, then a NaN scale in row 0.
    for row, bits in ((m - 1, 0x7C00), (0, 0x7E00), (m // 2, 0xFC00)):
        bad = blocks.copy()
        bad[row * nb + 5, 0:2] = np.array([bits], np.uint16).view(np.uint8)
        _, t = pick(hip, orc, qt, bad, m, k, x, f"scale {bits:#06x} at row {row}")
        assert t == -1
    # An infinite input makes every logit infinite or NaN.
    xi = x.copy()
    xi[7] = np.inf
    _, t = pick(hip, orc, qt, blocks, m, k, xi, "infinite x")
    assert t == -1
    # The state is clean afterwards: a finite call picks normally.
    y, t = pick(hip, orc, qt, blocks, m, k, x, "finite again")
    assert t >= 0


def test_pick_state_reused_across_grids(hip, orc):
    """One stream's pick state serves launches of 1 to 512 workgroups (fewer
    and more than the 8 fold groups) back to back."""
    cases = [(5, 13), (32000, 4096), (1, 32), (151936, 896), (40, 20000), (9, 64), (4096, 11008), (5, 13)]
    for i, (m, k) in enumerate(cases):
        qt = list(FMTS.values())[i % 3]
        blocks, x = make(orc, qt, m, k, seed=10 + i)
        y, t = pick(hip, orc, qt, blocks, m, k, x, f"reuse {i}")
        check_against_oracle(orc, qt, blocks, m, x, y, t, f"reuse {i} {m}x{k}")


def test_pick_argument_errors(hip, orc):
    qt = oracle.Q8_0
    blocks, x = make(orc, qt, 64, 64)
    wt = hip.Weight.upload(qt, blocks, 64, 64)
    xb = hip.DeviceBuffer.from_array(x)
    tok = hip.DeviceBuffer(4)
    rc = hip.load().mlq_hip_quant_linear_argmax(wt.h, xb.ptr, None, None, None)
    assert rc != 0 and "token pointer is null" in hip.last_error()
    host_x = np.zeros(64, np.float32)
    rc = hip.load().mlq_hip_quant_linear_argmax(wt.h, host_x.ctypes.data, None, tok.ptr, None)
    assert rc != 0 and "input" in hip.last_error()
    rc = hip.load().mlq_hip_quant_linear_argmax(None, xb.ptr, None, tok.ptr, None)
    assert rc != 0 and "null weight handle" in hip.last_error()
    for b in (xb, tok):
        b.free()
    wt.free()


def test_pick_in_recorded_graph(hip, orc):
    """The picking launch recorded with mlq_hip_graph_begin/_end next to a plain
    GEMV, replayed with eager work between replays: every replay's y and token
    equal an eager launch's on the same input."""
    m, k = 32000, 4096
    qt = oracle.Q4_0
    blocks, x = make(orc, qt, m, k, seed=5)
    wt = hip.Weight.upload(qt, blocks, m, k)
    xb = hip.DeviceBuffer.from_array(x)
    y_graph = hip.DeviceBuffer(4 * m)
    y_plain = hip.DeviceBuffer(4 * m)
    y_eager = hip.DeviceBuffer(4 * m)
    tok = hip.DeviceBuffer(8)
    s = hip.stream(0)
    wt.linear_argmax(xb, y_eager, tok, s)  # first call outside capture creates the stream's state
    hip.synchronize(s)

    def issue():
        wt.linear_device(xb, y_plain, stream=s, sync=False)
        wt.linear_argmax(xb, y_graph, tok, s)

    g = hip.Graph.record(issue, s, keep=(xb, y_graph, y_plain, tok))
    rng = np.random.default_rng(123)
    for rep in range(4):
        xi = rng.standard_normal(k, dtype=np.float32)
        xb.upload(xi)
        say(f"graph replay {rep}")
        g.launch(s)
        hip.synchronize(s)
        tg = int(tok.download(np.int32, 1)[0])
        yg = y_graph.download(np.float32, m)
        yp = y_plain.download(np.float32, m)
        wt.linear_argmax(xb, y_eager, tok, s)
        hip.synchronize(s)
        te = int(tok.download(np.int32, 1)[0])
        ye = y_eager.download(np.float32, m)
        assert np.array_equal(yg.view(np.uint32), ye.view(np.uint32)), f"replay {rep}: y differs from eager"
        assert np.array_equal(yp.view(np.uint32), ye.view(np.uint32)), f"replay {rep}: plain GEMV differs"
        assert tg == te == orc.argmax(ye), f"replay {rep}: graph {tg}, eager {te}"
    g.destroy()
    for b in (xb, y_graph, y_plain, y_eager, tok):
        b.free()
    wt.free()

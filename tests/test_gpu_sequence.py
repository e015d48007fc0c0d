"""GPU tests of the persistent GEMV sequence (mlq_hip_sequence_*).

A sequence runs a chain of GEMVs in one launch with device-wide barriers
between stages.  Per call its outputs must equal one mlq_hip_quant_linear
launch per call bit for bit (same lane-group width, same summation order), in
every mode (persistent, per-stage, independent, pipelined, LDS ring), for
chained calls whose x is an earlier call's y (what the barriers are for), for
fused stages (q/k/v, gate/up) and across graph replays with eager work in
between.  One chain is also checked against the CPU oracle
to the parity bound, and the host-side validation and the bounded barrier wait
are exercised.
"""

import sys

import numpy as np
import pytest

import oracle
from tolerance import check_close

pytestmark = pytest.mark.gpu

FMTS = {"q8_0": oracle.Q8_0, "q4_0": oracle.Q4_0, "q4_1": oracle.Q4_1}


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class Lin:
    """A device weight N(0, 0.02) quantized on the device, plus its blocks."""

    def __init__(self, hip, qt, m, k, seed):
        self.qt, self.m, self.k = qt, m, k
        nb = (k + 31) // 32
        f = hip.DeviceBuffer(4 * m * k)
        hip.fill_normal(f, m * k, seed, 0.0, 0.02)
        self.buf = hip.DeviceBuffer(m * nb * hip.BLOCK_BYTES[qt])
        hip.quantize_device(qt, f, m, k, self.buf)
        f.free()
        self.w = hip.Weight.wrap(qt, self.buf, m * nb, m, k)

    def blocks(self):
        bb = {oracle.Q8_0: 34, oracle.Q4_0: 18, oracle.Q4_1: 20}[self.qt]
        return self.buf.download(np.uint8).reshape(-1, bb)


def vec(hip, n, seed):
    b = hip.DeviceBuffer(4 * n)
    hip.fill_normal(b, n, seed, 0.0, 1.0)
    return b


def per_call(hip, calls):
    """Reference: one launch per call, in order, on the library stream."""
    for w, x, y in calls:
        w.w.linear_device(x, y)


def snapshot(bufs):
    return [b.download(np.float32) for b in bufs]


def llama_layer(hip, qt, seed, hidden=4096, ffn=11008):
    """q,k,v | o | gate,up | down with the real data flow: o reads v's output
    (a stand-in for attention), down reads up's output (for silu(gate)*up)."""
    lq, lk, lv = (Lin(hip, qt, hidden, hidden, seed + i) for i in range(3))
    lo = Lin(hip, qt, hidden, hidden, seed + 3)
    lg, lu = Lin(hip, qt, ffn, hidden, seed + 4), Lin(hip, qt, ffn, hidden, seed + 5)
    ld = Lin(hip, qt, hidden, ffn, seed + 6)
    x = vec(hip, hidden, seed + 100)
    yq, yk, yv, yo = (hip.DeviceBuffer(4 * hidden) for _ in range(4))
    yg, yu = hip.DeviceBuffer(4 * ffn), hip.DeviceBuffer(4 * ffn)
    yd = hip.DeviceBuffer(4 * hidden)
    calls = [(lq, x, yq), (lk, x, yk), (lv, x, yv), (lo, yv, yo), (lg, yo, yg), (lu, yo, yu), (ld, yu, yd)]
    stages = [0, 0, 0, 1, 2, 2, 3]
    keep = [lq, lk, lv, lo, lg, lu, ld, x]
    return calls, stages, [yq, yk, yv, yo, yg, yu, yd], keep


def run_sequence(hip, calls, stages, mode):
    arr = hip.make_calls([(w.w, x, y, 1) for w, x, y in calls])
    seq = hip.Sequence(arr, stages, mode)
    seq.launch()
    hip.synchronize()
    assert seq.status() == 0, "a barrier wait timed out"
    return seq


@pytest.mark.parametrize("fmt", list(FMTS))
def test_chain_matches_per_call_launches(hip, fmt):
    qt = FMTS[fmt]
    calls, stages, outs, keep = llama_layer(hip, qt, seed=11)
    say(f"sequence chain {fmt}: per-call reference")
    per_call(hip, calls)
    want = snapshot(outs)
    for b in outs:
        b.fill(0)
    for mode in (hip.SEQ_PERSISTENT, hip.SEQ_PER_STAGE, hip.SEQ_PIPELINED, hip.SEQ_LDS_RING):
        say(f"sequence chain {fmt} mode={mode}")
        seq = run_sequence(hip, calls, stages, mode)
        got = snapshot(outs)
        for i, (g, w) in enumerate(zip(got, want)):
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), f"{fmt} mode {mode} call {i} differs"
        info = seq.info()
        assert info["stages"] == 4
        seq.destroy()
        for b in outs:
            b.fill(0)


@pytest.mark.parametrize("mode", ["persistent", "lds_ring"])
def test_chain_against_oracle(hip, orc, mode):
    """A dependent Q4_0 chain 4096 -> 11008 -> 4096 checked call by call against
    the CPU oracle on the inputs each call actually saw."""
    qt = oracle.Q4_0
    l1, l2, l3 = Lin(hip, qt, 11008, 4096, 5), Lin(hip, qt, 4096, 11008, 6), Lin(hip, qt, 4096, 4096, 7)
    x = vec(hip, 4096, 8)
    y1, y2, y3 = hip.DeviceBuffer(4 * 11008), hip.DeviceBuffer(4 * 4096), hip.DeviceBuffer(4 * 4096)
    calls = [(l1, x, y1), (l2, y1, y2), (l3, y2, y3)]
    say(f"sequence chain vs oracle ({mode})")
    run_sequence(hip, calls, None, hip.SEQ_PERSISTENT if mode == "persistent" else hip.SEQ_LDS_RING)
    ins = [x.download(np.float32), y1.download(np.float32), y2.download(np.float32)]
    for (lin, _, yb), xin in zip(calls, ins):
        blocks = lin.blocks()
        want = orc.linear(qt, xin, blocks, lin.m, threads=16)
        check_close(yb.download(np.float32), want, xin, qt, blocks, f"chain {lin.m}x{lin.k}")


@pytest.mark.parametrize("shape", [(896, 896), (128, 896), (4864, 896), (896, 4864), (300, 2048),
                                   (37, 64), (1000, 3072), (77, 15360), (600, 4090)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_independent_shapes_all_modes(hip, shape):
    """Every lane-group width (16 / 32 / 64), ragged row counts, a 4-call stage,
    the largest supported K and a partial last block, in every mode (the
    LDS-ring mode where the rows are summed in 64-lane groups), against
    per-call launches."""
    m, k = shape
    for fmt, qt in FMTS.items():
        lins = [Lin(hip, qt, m + 3 * i, k, 40 + i) for i in range(4)]
        x = vec(hip, k, 99)
        outs = [hip.DeviceBuffer(4 * (m + 3 * i)) for i in range(4)]
        calls = [(lins[i], x, outs[i]) for i in range(4)]
        per_call(hip, calls)
        want = snapshot(outs)
        modes = [hip.SEQ_PERSISTENT, hip.SEQ_PER_STAGE, hip.SEQ_INDEPENDENT]
        if k % 32 == 0:  # the pipelined chain copies x in whole blocks
            modes.append(hip.SEQ_PIPELINED)
        if k in (2048, 3072, 4090, 15360):  # rows summed in 64-lane groups (4090: a partial last block)
            modes.append(hip.SEQ_LDS_RING)
        for mode in modes:
            for stages in ([0, 0, 0, 0], [0, 1, 1, 2], None):
                for b in outs:
                    b.fill(0)
                say(f"sequence {fmt} {m}x{k} mode={mode} stages={stages}")
                run_sequence(hip, calls, stages, mode)
                for i, (g, w) in enumerate(zip(snapshot(outs), want)):
                    assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), \
                        f"{fmt} {m}x{k} mode {mode} stages {stages} call {i}"


def test_mixed_formats_split_launches(hip):
    """Formats and widths change along the chain: one launch per run, same bits."""
    a = Lin(hip, oracle.Q8_0, 896, 4096, 1)
    b = Lin(hip, oracle.Q4_0, 4096, 896, 2)
    c = Lin(hip, oracle.Q4_1, 4096, 4096, 3)
    d = Lin(hip, oracle.Q4_0, 4096, 4096, 4)
    x = vec(hip, 4096, 5)
    ya, yb, yc, yd = (hip.DeviceBuffer(4 * n) for n in (896, 4096, 4096, 4096))
    calls = [(a, x, ya), (b, ya, yb), (c, yb, yc), (d, yc, yd)]
    per_call(hip, calls)
    want = snapshot([ya, yb, yc, yd])
    for buf in (ya, yb, yc, yd):
        buf.fill(0)
    seq = run_sequence(hip, calls, None, hip.SEQ_PERSISTENT)
    assert seq.info()["launches"] == 4
    for i, (g, w) in enumerate(zip(snapshot([ya, yb, yc, yd]), want)):
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), f"call {i}"


SEQ_MODES = {"persistent": "SEQ_PERSISTENT", "pipelined": "SEQ_PIPELINED", "lds_ring": "SEQ_LDS_RING"}


@pytest.mark.parametrize("mode", list(SEQ_MODES))
def test_graph_replays(hip, mode):
    """A captured sequence replayed with new x contents and eager work between
    replays: every replay equals per-call launches on the same x."""
    calls, stages, outs, keep = llama_layer(hip, oracle.Q4_0, seed=21)
    x = keep[-1]
    arr = hip.make_calls([(w.w, xx, y, 1) for w, xx, y in calls])
    seq = hip.Sequence(arr, stages, getattr(hip, SEQ_MODES[mode]))
    g = hip.Graph(sequence=seq)
    scratch = hip.DeviceBuffer(4 * 4096)
    for rep in range(4):
        hip.fill_normal(x, 4096, 500 + rep, 0.0, 1.0)
        hip.synchronize()
        say(f"sequence graph replay {rep}")
        g.launch()
        hip.synchronize()
        assert seq.status() == 0
        got = snapshot(outs)
        hip.fill_normal(scratch, 4096, 9, 0.0, 1.0)  # eager work between replays
        per_call(hip, calls)
        want = snapshot(outs)
        for i, (a, b) in enumerate(zip(got, want)):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"replay {rep} call {i}"
    g.destroy()
    seq.destroy()


def test_ring_stamps_need_the_measurement_build(hip):
    """mlq_hip_ring_stamps answers only from the measurement build (make
    stamps); the product library refuses with MLQ_ERR_NOT_BUILT and says how
    to build it, and checks its size argument first."""
    buf = np.zeros(hip.RING_STAMP_SHAPE, np.uint64)
    with pytest.raises(hip.MlqError, match="expected 18432"):
        hip._check(hip.load().mlq_hip_ring_stamps(buf.ctypes.data, 5))
    with pytest.raises(hip.MlqError, match="make stamps"):
        hip.ring_stamps()


def test_ring_stamps_bench_leg(hip):
    """The measurement build's boundary timestamps through `bench.py
    --ring-stamps` (a child process loads libmlq_hip_stamps.so): two layers of
    the sweep, every interval table printed for the three stamped workgroups."""
    import os
    import subprocess
    if not os.path.exists(hip.STAMPS_LIB_PATH):
        pytest.skip("the measurement build is not built (make -C mini-llama-cpp-release_amd stamps)")
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    say("bench.py --ring-stamps, 2 layers")
    r = subprocess.run([sys.executable, "bench.py", "--ring-stamps", "--layers", "2", "--steps", "2", "--warmup", "1"],
                       cwd=repo, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert r.stdout.count("| grid barrier |") == 3, r.stdout[-2000:]
    assert r.stdout.count("| loader: last unit in LDS |") == 3


def test_validation_messages(hip):
    l1 = Lin(hip, oracle.Q4_0, 64, 128, 1)
    l2 = Lin(hip, oracle.Q4_0, 64, 256, 2)
    odd = Lin(hip, oracle.Q4_0, 64, 96, 3)  # 3 blocks per row
    l64 = Lin(hip, oracle.Q4_0, 64, 64, 5)
    x = vec(hip, 256, 4)
    y = hip.DeviceBuffer(4 * 64)
    y2 = hip.DeviceBuffer(4 * 64)

    def create(calls, stages=None, mode=hip.SEQ_PERSISTENT):
        return hip.Sequence(hip.make_calls(calls), stages, mode)

    with pytest.raises(hip.MlqError, match="a sequence runs GEMV calls"):
        create([(l1.w, x, y, 2)])
    with pytest.raises(hip.MlqError, match="even block count"):
        create([(odd.w, x, y, 1)])
    with pytest.raises(hip.MlqError, match="differs from call 0 of its stage"):
        create([(l1.w, x, y, 1), (l2.w, x, y2, 1)], [0, 0])
    with pytest.raises(hip.MlqError, match="of one stage overlap"):
        create([(l1.w, x, y, 1), (l1.w, x, y, 1)], [0, 0])
    with pytest.raises(hip.MlqError, match="overlaps its stage's input"):
        create([(l1.w, x, x, 1)])
    with pytest.raises(hip.MlqError, match="overlaps the weight of call"):
        create([(l1.w, x, l1.buf.ptr, 1)])
    with pytest.raises(hip.MlqError, match="MLQ_SEQ_INDEPENDENT needs independent calls"):
        create([(l1.w, x, y, 1), (l64.w, y, y2, 1)], None, hip.SEQ_INDEPENDENT)
    with pytest.raises(hip.MlqError, match="at most 4"):
        ys = [hip.DeviceBuffer(4 * 64) for _ in range(5)]
        create([(l1.w, x, ys[i], 1) for i in range(5)], [0] * 5)
    with pytest.raises(hip.MlqError, match="unknown mode"):
        create([(l1.w, x, y, 1)], None, 7)
    k40 = Lin(hip, oracle.Q4_0, 64, 40, 6)  # two blocks per row, the second partial
    with pytest.raises(hip.MlqError, match="MLQ_SEQ_PIPELINED needs in_features % 32 == 0"):
        create([(k40.w, x, y, 1)], None, hip.SEQ_PIPELINED)
    create([(k40.w, x, y, 1)], None, hip.SEQ_PERSISTENT).destroy()
    with pytest.raises(hip.MlqError, match="MLQ_SEQ_LDS_RING needs rows summed in 64-lane groups"):
        create([(l2.w, x, y, 1)], None, hip.SEQ_LDS_RING)
    # a dependent chain is fine in the barrier modes
    create([(l1.w, x, y, 1), (l64.w, y, y2, 1)]).destroy()


@pytest.mark.parametrize("mode", list(SEQ_MODES))
def test_barrier_wait_bound_recovers(hip, mode):
    """With a one-poll bound the barrier waits give up instead of spinning; the
    launch still ends, the status reports it, and the next launch with the
    default bound is correct again (the barrier words reset themselves)."""
    calls, stages, outs, keep = llama_layer(hip, oracle.Q4_0, seed=31)
    per_call(hip, calls)
    want = snapshot(outs)
    arr = hip.make_calls([(w.w, x, y, 1) for w, x, y in calls])
    seq = hip.Sequence(arr, stages, getattr(hip, SEQ_MODES[mode]))
    seq.set_spin_limit(1)
    say("sequence with a one-poll barrier bound")
    seq.launch()
    hip.synchronize()
    timeouts = seq.status()
    say(f"  timeouts reported: {timeouts}")
    assert timeouts in (0, 1)
    assert seq.status() == 0, "status must clear"
    seq.set_spin_limit(1 << 20)
    seq.launch()
    hip.synchronize()
    assert seq.status() == 0
    for i, (g, w) in enumerate(zip(snapshot(outs), want)):
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), f"call {i} after recovery"


@pytest.mark.parametrize("shape", [(4096, 4096), (11008, 4096), (896, 896), (128, 896), (33, 4864),
                                   (64, 96), (40, 20000), (7, 33)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_fused_launch_matches_per_call(hip, shape):
    """mlq_hip_quant_linear_fused: 1-4 calls sharing x in one launch (pair
    kernels, odd block counts and K past the pair-kernel limit, which take the
    byte-load kernel), bit-identical to one launch per call."""
    m, k = shape
    for fmt, qt in FMTS.items():
        lins = [Lin(hip, qt, m + 5 * i, k, 60 + i) for i in range(4)]
        x = vec(hip, k, 61)
        outs = [hip.DeviceBuffer(4 * (m + 5 * i)) for i in range(4)]
        calls = [(lins[i], x, outs[i]) for i in range(4)]
        per_call(hip, calls)
        want = snapshot(outs)
        for n in (1, 2, 3, 4):
            for b in outs:
                b.fill(0)
            say(f"fused {fmt} {m}x{k} n={n}")
            hip.linear_fused(hip.make_calls([(c[0].w, c[1], c[2], 1) for c in calls[:n]]))
            hip.synchronize()
            for i, (g, w) in enumerate(zip(snapshot(outs[:n]), want[:n])):
                assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), f"fused {fmt} {m}x{k} n={n} call {i}"


def test_fused_validation(hip):
    l1 = Lin(hip, oracle.Q4_0, 64, 128, 1)
    l2 = Lin(hip, oracle.Q8_0, 64, 128, 2)
    x = vec(hip, 256, 3)
    y = [hip.DeviceBuffer(4 * 64) for _ in range(5)]

    def fused(calls):
        hip.linear_fused(hip.make_calls(calls))

    with pytest.raises(hip.MlqError, match="differs from call 0"):
        fused([(l1.w, x, y[0], 1), (l2.w, x, y[1], 1)])
    with pytest.raises(hip.MlqError, match="at most 4"):
        fused([(l1.w, x, y[i], 1) for i in range(5)])
    with pytest.raises(hip.MlqError, match="overlaps the output of call 0"):
        fused([(l1.w, x, y[0], 1), (l1.w, x, y[0], 1)])
    with pytest.raises(hip.MlqError, match="overlaps the input"):
        fused([(l1.w, x, x, 1)])
    with pytest.raises(hip.MlqError, match="differs from call 0"):
        fused([(l1.w, x, y[0], 1), (l1.w, x, y[1], 2)])


def test_stream_floor_runs_and_validates(hip):
    """mlq_hip_stream_floor (the weight stream of a fused launch without the
    arithmetic, a measurement) accepts the fused group shapes and refuses a
    sink that is too small or mixed in_features."""
    qkv = [Lin(hip, oracle.Q4_0, 4096, 4096, 60 + i) for i in range(3)]
    down = Lin(hip, oracle.Q4_0, 4096, 11008, 63)
    x = vec(hip, 4096, 64)
    y = hip.DeviceBuffer(4 * 4096)
    sink = hip.DeviceBuffer(4 * 65536)
    for calls in ([(l.w, x, y, 1) for l in qkv], [(down.w, x, y, 1)]):
        hip.stream_floor(hip.make_calls(calls), sink)
    hip.synchronize()
    small = hip.DeviceBuffer(1024)
    with pytest.raises(hip.MlqError, match="sink"):
        hip.stream_floor(hip.make_calls([(qkv[0].w, x, y, 1)]), small)
    with pytest.raises(hip.MlqError, match="differs from call 0"):
        hip.stream_floor(hip.make_calls([(qkv[0].w, x, y, 1), (down.w, x, y, 1)]), sink)


def test_stream_probe_runs_and_validates(hip):
    """mlq_hip_stream_probe (the floor's launch alone, and its bytes read with
    plain coalesced loads; measurements) runs on the fused group shapes and
    refuses an unknown mode and a small sink."""
    qkv = [Lin(hip, oracle.Q4_0, 4096, 4096, 70 + i) for i in range(3)]
    down = Lin(hip, oracle.Q4_0, 4096, 11008, 73)
    x = vec(hip, 4096, 74)
    y = hip.DeviceBuffer(4 * 4096)
    sink = hip.DeviceBuffer(4 * 65536)
    for mode in (hip.PROBE_EMPTY, hip.PROBE_LOAD):
        for calls in ([(l.w, x, y, 1) for l in qkv], [(down.w, x, y, 1)]):
            hip.stream_probe(hip.make_calls(calls), mode, sink)
    hip.synchronize()
    with pytest.raises(hip.MlqError, match="unknown mode"):
        hip.stream_probe(hip.make_calls([(qkv[0].w, x, y, 1)]), 3, sink)
    with pytest.raises(hip.MlqError, match="sink"):
        hip.stream_probe(hip.make_calls([(qkv[0].w, x, y, 1)]), hip.PROBE_LOAD, hip.DeviceBuffer(1024))

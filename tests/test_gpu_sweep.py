"""BASELINE config 5 at full size: the 225-call LLaMA-7B Q4_0 decode linear
sweep (3.727 GB) in the launch structure the bench times as its headline --
one fused launch per decode stage (q/k/v | o | gate/up | down, then lm_head),
129 dependent launches recorded as one graph -- and in the persistent
sequence kernels with grid barriers between the same stages (plain and
pipelined).

Every one of the 225 outputs is checked against the CPU linear of the oracle
(the reference's linear_quantized_impl, src/quant.cpp:367-433) on the same
blocks and x, within the BASELINE tolerance, and the greedy token of the
lm_head output (argmax, src/ops.cpp:179-192) must be the CPU's exactly."""

import os
import sys

import numpy as np
import pytest

import oracle
from tolerance import check_close

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def sweep(hip):
    from sweep_workload import Sweep

    say("config 5 sweep: generating 225 Q4_0 weights (3.727 GB) on the device")
    sw = Sweep(layers=32)
    yield sw
    sw.free()


@pytest.fixture(scope="module")
def cpu_outputs(sweep, orc):
    """The oracle's y for every call, with the blocks and x read back from the device."""
    out = []
    for name, w, x, _ in sweep.calls_desc:
        nblk = w.m * w.nb
        blocks = w._keep.download(np.uint8, nblk * 18).reshape(nblk, 18)
        xv = x.download(np.float32)
        out.append((name, w, blocks, xv, orc.linear(oracle.Q4_0, xv, blocks, w.m, threads=THREADS)))
    return out


@pytest.mark.parametrize("launch", ["per_stage", "sequence", "pipelined"])
def test_config5_sweep_matches_cpu(hip, sweep, cpu_outputs, orc, launch):
    say(f"config 5 sweep, launch {launch}: 225 calls, every output against the CPU linear")
    stream = hip.stream(0)
    mode = {"per_stage": hip.SEQ_PER_STAGE, "sequence": hip.SEQ_PERSISTENT, "pipelined": hip.SEQ_PIPELINED}[launch]
    seq = hip.Sequence(sweep.calls, sweep.stage_ids(), mode)
    graph = hip.Graph(sequence=seq) if launch == "per_stage" else None
    for y in sweep.ys:
        y.fill(0)
    hip.synchronize(stream)
    runs = []
    for _ in range(2):  # run twice: the second run must give the same bits
        if graph is not None:
            graph.launch(stream)
        else:
            seq.launch(stream)
        hip.synchronize(stream)
        runs.append([y.download(np.float32, w.m) for (_, w, _, _), y in zip(sweep.calls_desc, sweep.ys)])
    assert seq.status() == 0, "a barrier wait of the sequence timed out"
    worst = 0.0
    for (name, w, blocks, xv, want), got, again in zip(cpu_outputs, runs[0], runs[1]):
        assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), f"{launch} {name}: runs differ"
        worst = max(worst, check_close(got, want, xv, oracle.Q4_0, blocks, f"{launch} {name}"))
    name, w, blocks, xv, want = cpu_outputs[-1]
    assert name == "lm_head"
    got = sweep.ys[-1].download(np.float32, w.m)
    assert int(np.argmax(got)) == orc.argmax(want), "greedy token of the sweep differs from the CPU's"
    say(f"  {launch}: worst err/bound {worst:.3g}, token {orc.argmax(want)}")
    if graph is not None:
        graph.destroy()
    seq.destroy()

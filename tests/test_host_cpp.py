"""The C++ host layer (hip_q*_linear, backend selection) through its own test
binary, laid out like the reference's tests/test_cuda_quant.cpp."""

import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "host", "test_hip_quant")


def run(mode):
    assert os.path.exists(BIN), "build with __graft_entry__.build() (make -C tests/host)"
    r = subprocess.run([BIN, mode], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


def test_host_layer_cpu_side():
    assert "PASS hip_quant_cpu_side" in run("cpu")


@pytest.mark.gpu
def test_host_layer_parity_on_device():
    out = run("all")
    for tag in ("PASS hip_quant_q8_0", "PASS hip_quant_q4", "PASS hip_quant_forms"):
        assert tag in out, out

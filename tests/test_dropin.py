"""The reference's own CUDA quant test (tests/test_cuda_quant.cpp, compiled
unchanged with its device cases enabled) run on the HIP library through
tests/dropin/hip_backend.cpp, the reference's device-backend interface
(include/mini_llama/cuda_runtime.h, cuda_quant.h) implemented over the C ABI.

Modes q8_0 and q4 are the reference's linear cases (tests/test_cuda_quant.cpp:
293-420): host-weight, device-weight and device-input forms, 1-D and batched x,
bias, K = 13 / 64 / 65 (partial and odd blocks), against the reference's own
CPU linear_q*() with its own tolerance (abs or rel 1e-3).  Its forward modes
need the reference's device attention / norm / KV-cache interfaces, which are
outside the quantized-linear drop-in.

The binary is built by `make -C oracle dropin` (from __graft_entry__.build()
where the reference sources exist) and travels prebuilt."""

import os
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(REPO, "oracle", "_ref", "test_cuda_quant_hip")


def test_dropin_binary_links_the_hip_library():
    """CPU: the binary exists and resolves its device interface through libmlq_hip.so."""
    assert os.path.exists(BIN), "build it with `make -C oracle dropin` (needs the reference sources)"
    out = subprocess.run(["ldd", BIN], capture_output=True, text=True).stdout
    assert "libmlq_hip.so" in out and "not found" not in out, out


@pytest.mark.gpu
@pytest.mark.parametrize("mode,expect", [("q8_0", "PASS cuda_quant_q8_0"), ("q4", "PASS cuda_quant_q4")])
def test_reference_cuda_quant_cases_on_hip(mode, expect):
    assert os.path.exists(BIN), "build it with `make -C oracle dropin` (needs the reference sources)"
    print(f"reference test_cuda_quant {mode} through the HIP drop-in", flush=True)
    r = subprocess.run([BIN, mode], capture_output=True, text=True, timeout=120, cwd=REPO)
    print(r.stdout + r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert expect in r.stdout

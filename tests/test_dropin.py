"""The reference built for its device backend, with that backend served by the
HIP library through the package's drop-in (mini-llama-cpp-release_amd/dropin/:
the reference's cuda_runtime.h, cuda_quant.h, cuda_ops.h, cuda_attention.h,
cuda_matmul.h and backend.h interfaces on the C ABI; the reference's own
src/cuda_tensor.cpp and src/cuda_kv_cache.cpp compiled unchanged over it).

The reference's nine device test programs (tests/test_cuda_*.cpp, compiled
unchanged with its CUDA-build define) run every case the reference's CMake
registers for them (CMakeLists.txt:103-214, the 16 add_test entries) on the
MI355X, with the reference's own tolerances and counters -- e.g. the tiny
quantized model's one-token forward: 21 uploaded weights, 15 device linear
calls, 2 device attention calls, 0 host-to-device and 1 device-to-host copy
(tests/test_cuda_quant.cpp:422-471).  The reference's CLI (src/main.cpp,
unchanged) generates the same greedy tokens with --backend hip as with
--backend cpu.

Everything runs from tests/golden, where models/tiny holds the reference's
tiny model fixture (models/tiny/model.json, model.bin, vocab.json).  The
binaries are built by `make -C oracle dropin` (from __graft_entry__.build()
where the reference sources exist) and travel prebuilt."""

import os
import re
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OUT = os.path.join(REPO, "oracle", "_ref", "dropin")
CWD = os.path.join(REPO, "tests", "golden")

# (program, argument, line printed on success): the reference's add_test list.
CASES = [
    ("test_cuda_runtime", None, "PASS cuda_runtime"),
    ("test_cuda_matmul", "matmul", "PASS cuda_matmul"),
    ("test_cuda_matmul", "linear", "PASS cuda_linear"),
    ("test_cuda_quant", "q8_0", "PASS cuda_quant_q8_0"),
    ("test_cuda_quant", "q4", "PASS cuda_quant_q4"),
    ("test_cuda_quant", "forward", "PASS cuda_forward_quant"),
    ("test_cuda_quant", "forward_q4", "PASS cuda_forward_q4"),
    ("test_cuda_forward_buffer", "f32", "PASS cuda_forward_buffer"),
    ("test_cuda_forward_buffer", "q8_0", "PASS cuda_forward_device_resident"),
    ("test_cuda_attention", "direct", "PASS cuda_attention"),
    ("test_cuda_attention", "kv", "PASS cuda_kv_attention"),
    ("test_cuda_attention", "forward", "PASS cuda_forward_attention"),
    ("test_cuda_forward_linear", None, "PASS cuda_forward_linear"),
    ("test_cuda_ops", None, "PASS cuda_ops"),
    ("test_cuda_kv_cache", None, "PASS cuda_kv_cache"),
    ("test_cuda_forward", None, "PASS cuda_forward"),
]
PROGRAMS = sorted({c[0] for c in CASES}) + ["mini-llama"]


def _bin(name):
    path = os.path.join(OUT, name)
    assert os.path.exists(path), "build it with `make -C oracle dropin` (needs the reference sources)"
    return path


@pytest.mark.parametrize("name", PROGRAMS)
def test_dropin_program_links_the_hip_library(name):
    """CPU: each program exists and resolves its device interfaces through libmlq_hip.so."""
    out = subprocess.run(["ldd", _bin(name)], capture_output=True, text=True).stdout
    assert "libmlq_hip.so" in out and "not found" not in out, out


def test_tiny_model_fixture_present():
    for f in ("model.json", "model.bin", "vocab.json"):
        assert os.path.exists(os.path.join(CWD, "models", "tiny", f)), f


@pytest.mark.gpu
@pytest.mark.parametrize("prog,mode,expect", CASES, ids=[f"{p}-{m or 'all'}" for p, m, _ in CASES])
def test_reference_device_tests_on_hip(prog, mode, expect):
    print(f"reference {prog} {mode or ''} through the HIP drop-in", flush=True)
    cmd = [_bin(prog)] + ([mode] if mode else [])
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120, cwd=CWD)
    print(r.stdout + r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert expect in r.stdout


def _generate(backend, quant):
    cmd = [_bin("mini-llama"), "generate", "--prompt", "hello", "--n-predict", "12", "--backend", backend,
           "--quant", quant, "--threads", "4"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120, cwd=CWD)
    assert r.returncode == 0, r.stdout + r.stderr
    m = re.search(r"generated tokens: \[([^\]]*)\]", r.stdout)
    assert m, r.stdout
    return m.group(1), r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("quant", ["q8_0", "q4_0"])
def test_reference_cli_backend_hip_generates_cpu_tokens(quant):
    """src/main.cpp's generate with --backend hip: weights uploaded, the decode
    on the device (the reference's device forward over the drop-in), the same
    greedy tokens as --backend cpu."""
    print(f"reference CLI generate --backend hip --quant {quant}", flush=True)
    cpu, _ = _generate("cpu", quant)
    dev, out = _generate("hip", quant)
    print(out, flush=True)
    assert "backend: cuda" in out and "compute: cuda linear" in out
    assert "HIP library" in out
    assert dev == cpu, f"hip {dev} vs cpu {cpu}"

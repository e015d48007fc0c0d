"""The library's Makefile must fail when a kernel source does not compile, and
must not link an object left over from an earlier build (CPU only: hipcc
cross-compiles without a GPU)."""

import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MAKEFILE = os.path.join(REPO, "mini-llama-cpp-release_amd", "Makefile")

pytestmark = pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc"), reason="hipcc not installed")


def _tree(tmp_path, source):
    pkg = tmp_path / "pkg"
    (pkg / "csrc").mkdir(parents=True)
    (tmp_path / "include").mkdir()
    (tmp_path / "include" / "mlq_hip.h").write_text("#pragma once\n")
    shutil.copy(MAKEFILE, pkg / "Makefile")
    (pkg / "csrc" / "k.hip").write_text(source)
    return pkg


GOOD = "#include <hip/hip_runtime.h>\n__global__ void k(float* y) { y[threadIdx.x] = 1.0f; }\n"
BAD = "#include <hip/hip_runtime.h>\n__global__ void k(float* y) { y[threadIdx.x] = undeclared_name; }\n"


def test_broken_kernel_fails_the_build(tmp_path):
    pkg = _tree(tmp_path, GOOD)
    r = subprocess.run(["make", "-s", "-C", str(pkg), "-B"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert (pkg / "libmlq_hip.so").exists()
    # The object of the good source stays in place; a broken edit must not
    # reuse it.
    (pkg / "csrc" / "k.hip").write_text(BAD)
    r = subprocess.run(["make", "-s", "-C", str(pkg), "-B"], capture_output=True, text=True)
    assert r.returncode != 0, "make succeeded on a source that does not compile"
    assert "undeclared_name" in r.stdout + r.stderr
    assert not (pkg / "_build" / "k.o").exists(), "a stale object survived a failed compile"

"""CPU-side checks of the C-ABI library: it loads without a GPU, exports every
entry point include/mlq_hip.h declares, and its ctypes binding covers them.
No compute call is made here (no device in this container)."""

import ctypes
import os
import re

import pytest

import mlq_hip

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "mlq_hip.h")


def declared_entry_points():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mlq_hip_[a-z0-9_]+)\s*\(", text)))


def test_library_is_built_and_loads():
    assert os.path.exists(mlq_hip.LIB_PATH), "run __graft_entry__.build() first"
    lib = mlq_hip.load()
    assert lib.mlq_hip_built() == 1


def test_exports_every_declared_symbol():
    lib = ctypes.CDLL(mlq_hip.LIB_PATH)
    names = declared_entry_points()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_header():
    assert sorted(mlq_hip.EXPORTED) == declared_entry_points()


def test_constants_match_header():
    text = open(HEADER).read()
    consts = dict(re.findall(r"#define (MLQ_[A-Z0-9_]+) (0x[0-9a-f]+|\d+)", text))
    val = {k: int(v, 0) for k, v in consts.items()}
    assert (val["MLQ_F32"], val["MLQ_Q8_0"], val["MLQ_Q4_0"], val["MLQ_Q4_1"]) == (0, 1, 2, 3)
    assert (val["MLQ_Q8_0_BLOCK_BYTES"], val["MLQ_Q4_0_BLOCK_BYTES"], val["MLQ_Q4_1_BLOCK_BYTES"]) == (34, 18, 20)
    assert (val["MLQ_X_ON_DEVICE"], val["MLQ_Y_ON_DEVICE"], val["MLQ_ASYNC"]) == (
        mlq_hip.X_ON_DEVICE, mlq_hip.Y_ON_DEVICE, mlq_hip.ASYNC)


def test_host_side_validation_without_gpu():
    """Argument checks run before any device work, so they answer here too."""
    lib = mlq_hip.load()
    h = ctypes.c_void_p()
    rc = lib.mlq_hip_upload_weight(0, 7, None, 0, 4, 32, ctypes.byref(h))
    assert rc == 1 and "unsupported quant type 7" in mlq_hip.last_error()
    blocks = (ctypes.c_uint8 * (34 * 3))()
    rc = lib.mlq_hip_upload_weight(0, 1, blocks, 3, 4, 32, ctypes.byref(h))
    assert rc == 2 and mlq_hip.last_error() == "HIP weight upload: Q8_0 block count mismatch, expected 4, got 3"
    rc = lib.mlq_hip_quant_linear(None, None, 1, None, 0, None)
    assert rc == 1 and "null weight handle" in mlq_hip.last_error()


def test_kernel_selection_names():
    # decode shapes of the benchmark take the pair kernel; odd block counts the generic one
    assert mlq_hip.kernel_name(mlq_hip.Q4_0, 1, 4096, 4096) == "gemv_single_q4_0_lpr64"
    assert mlq_hip.kernel_name(mlq_hip.Q4_0, 1, 32000, 4096) == "gemv_single_q4_0_lpr64"
    assert mlq_hip.kernel_name(mlq_hip.Q8_0, 1, 4096, 11008) == "gemv_multi_q8_0_lpr64"
    assert mlq_hip.kernel_name(mlq_hip.Q4_0, 1, 896, 4864) == "gemv_multi_q4_0_lpr16"
    assert mlq_hip.kernel_name(mlq_hip.Q4_1, 1, 151936, 896) == "gemv_single_q4_1_lpr16"
    assert mlq_hip.kernel_name(mlq_hip.Q4_0, 1, 5, 13) == "gemv_generic_q4_0"
    assert mlq_hip.kernel_name(mlq_hip.Q4_0, 64, 4096, 4096).startswith("gemm_mfma_q4_0")

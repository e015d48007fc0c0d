"""bench.py --profile-summary: the per-stage tables committed under profiles/
come from it, so its selection of timed dispatches and its stage assignment
are checked on a synthetic rocprofv3 CSV (CPU only)."""

import csv
import os
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "mini-llama-cpp-release_amd"))

import bench  # noqa: E402

GEMV = "void mlq::(anonymous namespace)::gemv_single_kernel<2, 64, 8, 3, 0, 2>(mlq::GemvGroup, float const*)"
MULTI = "void mlq::(anonymous namespace)::gemv_multi_kernel<2, 64, 16, 2, 0, 1>(mlq::GemvGroup, float const*)"
FLOOR = "void mlq::(anonymous namespace)::stream_floor_kernel<2, 64, 3>(mlq::GemvGroup, int)"


def _trace(path, warm, timed):
    """warm + timed steps of 129 GEMV launches, then of 129 floor launches.
    Durations encode (timed?, stage): warm-up launches take 1000 us, timed
    ones 10 + stage index (0..3) or 20 for lm_head."""
    rows, t = [], 0
    for fam in ("gemv", "floor"):
        for step in range(warm + timed):
            for i in range(129):
                kind = 4 if i == 128 else i % 4
                name = FLOOR if fam == "floor" else (MULTI if kind == 3 else GEMV)
                dur_us = 1000 if step < warm else (20 if kind == 4 else 10 + kind)
                rows.append({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + dur_us * 1000})
                t += dur_us * 1000 + 500
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        w.writerows(rows)


def test_timed_dispatches_and_stages(tmp_path):
    _trace(tmp_path / "kt_kernel_trace.csv", warm=3, timed=2)
    out = bench.profile_summary(str(tmp_path), steps=2)
    lines = [l for l in out.splitlines() if l.startswith("| mlq::")]
    assert len(lines) == 10  # 5 stages x (gemv, floor)
    by = {}
    for l in lines:
        cells = [c.strip() for c in l.strip("|").split("|")]
        by.setdefault(cells[1], []).append((cells[0], int(cells[2]), float(cells[3]), float(cells[6])))
    expect = {"q/k/v fused 12288x4096": 10.0, "o 4096x4096": 11.0, "gate/up fused 22016x4096": 12.0,
              "down 4096x11008": 13.0, "lm_head 32000x4096": 20.0}
    for stage, avg in expect.items():
        for kernel, n, a, mx in by[stage]:
            assert n == (2 if stage.startswith("lm_head") else 64), (stage, n)
            assert a == avg and mx == avg, (stage, kernel, a, mx)  # no warm-up launch (1000 us) kept
    assert "down 4096x11008" in out and "gemv_multi_kernel" in out
    assert out.count("kernel time per step") == 2


def test_too_few_dispatches_prints_nothing(tmp_path):
    _trace(tmp_path / "kt_kernel_trace.csv", warm=0, timed=1)
    assert "| mlq::" not in bench.profile_summary(str(tmp_path), steps=2)


GEMM = "void mlq::(anonymous namespace)::gemm_chunk_kernel<2, 2, 2, 2, true>(mlq::(anonymous namespace)::ChunkArgs)"
XSPLIT = "void mlq::(anonymous namespace)::xsplit_kernel<2>(float const*, int, int, int, int, _Float16*, float*, float*)"
COPY = "__amd_rocclr_copyBuffer"


def test_kernel_summary_groups_gemm_kernels(tmp_path):
    """bench.py --kernel-summary: every dispatch of the GEMM and x-split kernels
    grouped by name (other kernels left out), mean counters per dispatch, and
    the largest copy reported for calibrating byte counters."""
    rows, t = [], 0
    for name, dur in [(XSPLIT, 7), (GEMM, 60), (GEMV, 5), (XSPLIT, 9), (GEMM, 62)]:
        rows.append({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + dur * 1000})
        t += dur * 1000 + 100
    with open(tmp_path / "kt_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        w.writerows(rows)
    crow = [(1, COPY, 1048576.0), (2, COPY, 10.0), (3, GEMM, 100.0), (4, GEMM, 300.0), (5, XSPLIT, 50.0),
            (6, GEMV, 7.0)]
    with open(tmp_path / "c_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for i, name, v in crow:
            w.writerow({"Dispatch_Id": i, "Kernel_Name": name, "Counter_Name": "FETCH_SIZE", "Counter_Value": v})
    out = bench.kernel_summary(str(tmp_path))
    lines = [l for l in out.splitlines() if l.startswith("| mlq::")]
    assert len(lines) == 4 and "gemv" not in out  # 2 kernels x (trace, counters)
    dur = {l.split("|")[1].strip(): float(l.split("|")[3]) for l in lines if l.count("|") == 7}
    assert dur["mlq::gemm_chunk_kernel<2, 2, 2, 2, true>"] == 61.0
    assert dur["mlq::xsplit_kernel<2>"] == 8.0
    cnt = {l.split("|")[1].strip(): float(l.split("|")[3]) for l in lines if l.count("|") == 4}
    assert cnt["mlq::gemm_chunk_kernel<2, 2, 2, 2, true>"] == 200.0 and cnt["mlq::xsplit_kernel<2>"] == 50.0
    assert "calibration copy): FETCH_SIZE 1048576.0" in out

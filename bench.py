#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-linear path (one GPU).

Step = one LLaMA-7B-shaped Q4_0 decode linear sweep:
32 layers x (q, k, v, o 4096x4096; gate, up 11008x4096; down 4096x11008) plus
lm_head 32000x4096 = 225 GEMV calls over 3.727 GB of resident weights, with a
fresh x ~ N(0, 1) per layer (x for q..up, h for down), all generated on the
device before timing.  `value` is algorithmic bytes (weight blocks + 4K + 4M
per call) per second over the timed steps.

Headline launch mode (`--launch per_stage`): the decode step's data flow, in
stream order -- per layer the q/k/v calls (same x) as one fused launch, then
o, then gate/up (same x) fused, then down; 129 launches per step captured as
one graph.  Every launch may depend on the previous one, as in a real decode
step.  The other modes are timed too and reported in config.sweep_us_by_launch:
one launch per call (graph / plain), the persistent sequence kernel with grid
barriers between the same 129 stages (sequence), and the persistent kernel
without barriers (independent: valid only because this sweep's inputs are all
fresh; not a decode step).

Also reported (not the headline value):
  * gemv[]: per-shape GEMV time / GB/s for BASELINE configs 1-3, each cycling
    max(32, ceil(1 GB / W bytes)) distinct weight copies so the 256 MB MALL
    cannot hold the working set, one dependent call after another; for the
    config 3 (LLaMA) shapes also `independent_streams`: the same calls as four
    independent chains on four streams, whose overlap hides the dependent-
    launch gap (the kernel's sustained rate, not a decode step);
  * gemm[]: prefill GEMM (config 4) time, TFLOP/s and MFMA share of peak;
  * parity: every sweep output against the reference's CPU linear on the same
    blocks, and greedy argmax of the lm_head output;
  * cpu_baseline: the reference's own threaded CPU quant linear (oracle/_ref,
    compiled from the reference sources; the restated oracle if absent) over
    the whole sweep on all host cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
                       [--launch per_stage|graph|plain|sequence|independent]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "mini-llama-cpp-release_amd"))
sys.path.insert(0, REPO)

import mlq_hip as hip  # noqa: E402

sys.path.insert(0, os.path.join(REPO, "tests"))
from sweep_workload import LAYER, Sweep, gemv_bytes, make_weight  # noqa: E402,F401

METRIC = "quant matvec HBM GB/s (% of 8 TB/s peak) + µs per 7B-shape decode linear sweep"
HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
BB = {hip.Q8_0: 34, hip.Q4_0: 18, hip.Q4_1: 20}
FMT_NAME = {hip.Q8_0: "q8_0", hip.Q4_0: "q4_0", hip.Q4_1: "q4_1"}


TRAFFIC_PROFILE = os.path.join(REPO, "profiles", "gemv_q4_0_llama7b_sweep_hbm_traffic.md")

KERNEL_BY_LAUNCH = {
    "graph": "Q4_0 GEMV family (gemv_single / gemv_multi), one launch per call",
    "plain": "Q4_0 GEMV family (gemv_single / gemv_multi), one launch per call",
    "per_stage": "Q4_0 GEMV family (gemv_single / gemv_multi), one fused launch per stage (q,k,v | o | gate,up | down)",
    "sequence": "gemv_sequence (persistent, grid barriers between stages)",
    "independent": "gemv_sequence (persistent, no barriers)",
    "pipelined": "gemv_chain (persistent, grid barriers between stages; weight ring across barriers, control wave "
                 "per workgroup for stores, arrival and x)",
    "lds_ring": "gemv_ring (persistent, grid barriers between stages; loader waves stream every stage's weights "
                "into an LDS ring per CU, compute waves stage x and take the weights from the ring)",
}


def measured_traffic(launch):
    """HBM bytes per launch of the sweep in this launch mode from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (calibrated against a copy of
    known size), or None when that mode has not been profiled."""
    try:
        for line in open(TRAFFIC_PROFILE):
            if line.startswith(f"traffic_bytes_per_launch[{launch}]:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_region(fn, steps, stream):
    start, stop = hip.Event(), hip.Event()
    hip.synchronize(stream)
    start.record(stream)
    for _ in range(steps):
        fn()
    stop.record(stream)
    hip.synchronize(stream)
    return start.elapsed_ms(stop)


def cpu_model():
    """The host CPU (from /proc/cpuinfo: model name, family / model / stepping
    numbers, logical CPUs), for the baseline line; some hosts report only a
    generic model name, which the numbers then identify."""
    fields, cpus = {}, 0
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key = key.strip()
                if key == "processor":
                    cpus += 1
                elif key in ("model name", "cpu family", "model", "stepping") and key not in fields:
                    fields[key] = val.strip()
    except OSError:
        return "unknown"
    name = fields.get("model name", "unknown")
    ids = ", ".join(f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields)
    return f"{name} ({ids}; {cpus} logical CPUs)" if ids else name


def cpu_sweep_check(sw: Sweep, threads: int, runs: int = 3, alt=None):
    """Run the reference CPU linear over the whole sweep on the same blocks and
    compare every output with the GPU's.  Timing follows the reference's own
    benchmark pattern (src/main.cpp:1226-1238): one untimed warm-up sweep, then
    `runs` timed sweeps, median reported; each sweep calls the threaded
    linear() once per weight (parallel_for over all host cores,
    src/thread_pool.cpp:23-73).  alt: a callable that recomputes the sweep's
    outputs with another GPU path; its outputs are checked against the same
    CPU results (worst_err_over_bound_alt)."""
    import oracle

    sys.path.insert(0, os.path.join(REPO, "tests"))
    from tolerance import check_close

    ref = oracle.reference()
    kind = "reference" if ref is not None else "port"
    orc = oracle.get()
    prepared = []
    cpu_bytes = 0
    for name, w, x, y in sw.calls_desc:
        nblk = w.m * w.nb
        blocks = w._keep.download(np.uint8, nblk * BB[w.qtype]).reshape(nblk, BB[w.qtype])
        rw = ref.weight(w.qtype, blocks, w.m, w.k) if ref is not None else None
        prepared.append((name, w, blocks, rw, x.download(np.float32), y.download(np.float32),
                         np.empty(w.m, np.float32)))
        cpu_bytes += gemv_bytes(w.qtype, w.m, w.k)

    def sweep_once():
        t0 = time.perf_counter()
        for _, w, blocks, rw, xv, _, yc in prepared:
            if rw is not None:
                rw.linear(xv, yc, threads)
            else:
                yc[:] = orc.linear(w.qtype, xv, blocks, w.m, threads=threads)
        return time.perf_counter() - t0

    warm = sweep_once()
    times = [sweep_once() for _ in range(runs)]
    worst = 0.0
    for name, w, blocks, _, xv, yg, yc in prepared:
        worst = max(worst, check_close(yg, yc, xv, w.qtype, blocks, name))
        if name == "lm_head":
            arg_gpu, arg_cpu = int(np.argmax(yg)), orc.argmax(yc)
            top2 = np.sort(yc)[-2:]
    worst_alt = None
    if alt is not None:
        alt()
        worst_alt = 0.0
        for (name, w, blocks, _, xv, _, yc), (_, _, _, y) in zip(prepared, sw.calls_desc):
            worst_alt = max(worst_alt, check_close(y.download(np.float32), yc, xv, w.qtype, blocks, name))
    del prepared
    return {
        "worst_err_over_bound_alt": worst_alt,
        "kind": kind, "cpu_s": float(np.median(times)), "cpu_s_runs": [round(t, 4) for t in times],
        "cpu_s_warmup": round(warm, 4), "cpu_bytes": cpu_bytes, "worst_err_over_bound": worst,
        "argmax_gpu": arg_gpu, "argmax_cpu": arg_cpu, "argmax_top2_gap": float(top2[1] - top2[0]),
    }


def floor_bench(sw: Sweep, stream, steps: int, warmup: int, probe=None):
    """The sweep's 129 stages as weight-stream-only launches (mlq_hip_stream_floor:
    the GEMV kernels' grid, work units and request ring, no arithmetic),
    recorded as one graph like the headline: the floor that one launch per
    stage pays for launching and streaming the weights.  probe: the floor's
    parts instead (mlq_hip_stream_probe): PROBE_EMPTY, the same grid launched
    with no work (the dependent-launch cost), or PROBE_LOAD, the same bytes
    read with plain coalesced 16-byte loads (launch plus stream, without the
    GEMV's work units)."""
    ids = sw.stage_ids()
    groups, i = [], 0
    while i < len(ids):
        j = i + 1
        while j < len(ids) and ids[j] == ids[i]:
            j += 1
        groups.append(hip.make_calls([(w, x, y, 1) for (_, w, x, y) in sw.calls_desc[i:j]]))
        i = j
    sink = hip.DeviceBuffer(4 * 65536)
    if probe is None:
        graph = hip.Graph.record(lambda: [hip.stream_floor(g, sink, stream) for g in groups], stream,
                                 keep=(groups, sink))
    else:
        graph = hip.Graph.record(lambda: [hip.stream_probe(g, probe, sink, stream) for g in groups], stream,
                                 keep=(groups, sink))
    for _ in range(warmup):
        graph.launch(stream)
    ms = time_region(lambda: graph.launch(stream), steps, stream) / steps
    graph.destroy()
    sink.free()
    note = {None: "mlq_hip_stream_floor per stage (weights streamed with the GEMV grid and ring, no "
                  "arithmetic), one graph of the same 129 dependent launches as per_stage",
            hip.PROBE_EMPTY: "mlq_hip_stream_probe(MLQ_PROBE_EMPTY) per stage: the floor's grid launched with "
                             "no work, one graph of 129 dependent launches (the launch cost alone)",
            hip.PROBE_LOAD: "mlq_hip_stream_probe(MLQ_PROBE_LOAD) per stage: the stage's weight bytes read with "
                            "plain coalesced 16-byte loads on the floor's grid, one graph of 129 dependent "
                            "launches (launch plus stream, no GEMV work units)"}[probe]
    res = {"launches": len(groups), "us_per_step": round(ms * 1e3, 1),
           "us_per_launch": round(ms * 1e3 / len(groups), 3), "note": note}
    if probe != hip.PROBE_EMPTY:
        res["gbs"] = round(sw.bytes / (ms * 1e-3) / 1e9, 1)
    return res


def f32_sweep_bench(sw: Sweep, stream, steps: int, warmup: int):
    """The sweep's 129 stages on the f32 GEMV (mlq_hip_quant_linear_fused_f32:
    each weight dequantized to f32 and multiplied into an f32 sum of x, the
    reference's arithmetic, src/quant.cpp:413-429), recorded as one graph like
    the headline: what the integer path's speed is bought against.  Returns
    the timing and a function that reruns the sweep once (for the margin
    check against the CPU results)."""
    ids = sw.stage_ids()
    groups, i = [], 0
    while i < len(ids):
        j = i + 1
        while j < len(ids) and ids[j] == ids[i]:
            j += 1
        groups.append(hip.make_calls([(w, x, y, 1) for (_, w, x, y) in sw.calls_desc[i:j]]))
        i = j
    graph = hip.Graph.record(lambda: [hip.linear_fused_f32(g, stream) for g in groups], stream, keep=groups)
    for _ in range(warmup):
        graph.launch(stream)
    ms = time_region(lambda: graph.launch(stream), steps, stream) / steps

    def rerun():
        graph.launch(stream)
        hip.synchronize(stream)

    res = {"launches": len(groups), "us_per_step": round(ms * 1e3, 1),
           "gbs": round(sw.bytes / (ms * 1e-3) / 1e9, 1),
           "frac_of_peak": round(sw.bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "note": "mlq_hip_quant_linear_fused_f32 per stage (weights dequantized to f32, f32 multiply-adds "
                   "with f32 x, as src/quant.cpp:413-429), one graph of the same 129 dependent launches as "
                   "per_stage"}
    return res, rerun, graph


# ------------------------------------------------------------------ per-shape GEMV
GEMV_CONFIGS = (
    [("c1_qwen_ffn_up", hip.Q8_0, 4864, 896)] +
    [(f"c2_qwen_{n}", qt, m, k) for qt in (hip.Q4_0, hip.Q4_1)
     for (n, m, k) in (("q_o", 896, 896), ("k_v", 128, 896), ("gate_up", 4864, 896),
                       ("down", 896, 4864), ("lm_head", 151936, 896))] +
    [(f"c3_llama_{n}", qt, m, k) for qt in (hip.Q8_0, hip.Q4_0, hip.Q4_1)
     for (n, m, k) in (("qkvo", 4096, 4096), ("gate_up", 11008, 4096), ("down", 4096, 11008),
                       ("lm_head", 32000, 4096))]
)


def weight_copies(qt, m, k, seed):
    """One seeded weight and enough device copies of it that cycling through
    them streams at least 1 GB (no copy is still in the 256 MB MALL when it is
    read again)."""
    wbytes = m * ((k + 31) // 32) * BB[qt]
    copies = max(32, math.ceil(1e9 / wbytes))
    tmp = hip.DeviceBuffer(4 * m * k)
    base = make_weight(qt, m, k, seed, tmp)
    tmp.free()
    bufs = [base._keep]
    for _ in range(copies - 1):
        b = hip.DeviceBuffer(wbytes)
        hip.load().mlq_hip_memcpy_dtod(b.ptr, base._keep.ptr, wbytes, None)
        bufs.append(b)
    ws = [hip.Weight.wrap(qt, b, m * ((k + 31) // 32), m, k) for b in bufs]
    return wbytes, copies, bufs, ws


def gemv_shape_bench(name, qt, m, k, stream, reps_target=400, streams=None):
    wbytes, copies, bufs, ws = weight_copies(qt, m, k, 4242 + m + k + qt)
    x = hip.DeviceBuffer(4 * k)
    hip.fill_normal(x, k, 99, 0.0, 1.0)
    y = hip.DeviceBuffer(4 * m)
    calls = hip.make_calls([(w, x, y, 1) for w in ws])
    graph = hip.Graph(calls, stream)  # arguments validated once, at capture
    hip.synchronize(stream)
    loops = max(1, reps_target // copies)
    graph.launch(stream)  # warm-up
    ms = time_region(lambda: graph.launch(stream), loops, stream)
    graph.destroy()
    n = loops * copies
    us = ms * 1e3 / n
    gbs = gemv_bytes(qt, m, k) / (us * 1e-6) / 1e9
    res = {"name": name, "fmt": FMT_NAME[qt], "M": m, "K": k, "copies": copies,
           "working_set_gb": round(copies * wbytes / 1e9, 3), "us_per_call": round(us, 3),
           "gbs": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
           "kernel": hip.kernel_name(qt, 1, m, k)}
    if streams:
        # The same calls as `len(streams)` independent chains (each its own y,
        # its own stream, one graph each): consecutive calls of a chain still
        # wait for each other, calls of different chains may overlap, so the
        # dependent-launch gap and each launch's ramp and tail are hidden.
        # Host-timed around all chains (a few ms per run).
        nst = len(streams)
        ys = [hip.DeviceBuffer(4 * m) for _ in range(nst)]
        graphs = [hip.Graph(hip.make_calls([(w, x, ys[i], 1) for w in ws[i::nst]]), streams[i]) for i in range(nst)]
        for i in range(nst):
            graphs[i].launch(streams[i])
        for st in streams:
            hip.synchronize(st)
        t0 = time.perf_counter()
        for _ in range(loops):
            for i in range(nst):
                graphs[i].launch(streams[i])
        for st in streams:
            hip.synchronize(st)
        us_ov = (time.perf_counter() - t0) * 1e6 / (loops * copies)
        for g in graphs:
            g.destroy()
        for b in ys:
            b.free()
        gbs_ov = gemv_bytes(qt, m, k) / (us_ov * 1e-6) / 1e9
        res["independent_streams"] = {"streams": nst, "us_per_call": round(us_ov, 3), "gbs": round(gbs_ov, 1),
                                      "frac_of_peak": round(gbs_ov / HBM_PEAK_GBS, 4)}
    for w in ws:
        w.free()
    for b in bufs:
        b.free()
    return res


def ingest_bench(layers=4):
    """GGUF ingest of LLaMA-7B-shaped Q4_0 linears (`layers` layers of q, k, v,
    o, gate, up, down and the lm_head) from a page-cache-warm file: the
    mapping straight to HBM (mlq_hip_gguf_upload_weight) against the
    reference's sequence, each tensor read into host memory and then uploaded
    (read_gguf_tensor_raw + upload, src/gguf.cpp:586-622, src/model.cpp:145-272)."""
    import tempfile

    sys.path.insert(0, os.path.join(REPO, "tests"))
    import gguf_writer as gw

    rng = np.random.default_rng(1)
    shapes = []
    for layer in range(layers):
        for op, (m, k) in (("attn_q", (4096, 4096)), ("attn_k", (4096, 4096)), ("attn_v", (4096, 4096)),
                           ("attn_output", (4096, 4096)), ("ffn_gate", (11008, 4096)), ("ffn_up", (11008, 4096)),
                           ("ffn_down", (4096, 11008))):
            shapes.append((f"blk.{layer}.{op}.weight", m, k))
    shapes.append(("output.weight", 32000, 4096))
    tensors = [(n, [k, m], gw.GGML_Q4_0, rng.integers(0, 256, m * (k // 32) * 18, dtype=np.uint8).tobytes())
               for n, m, k in shapes]
    fd, path = tempfile.mkstemp(suffix=".gguf")
    os.close(fd)
    try:
        gw.write(path, [("general.architecture", gw.STRING, "llama")], tensors, alignment=32)
        total = sum(len(t[3]) for t in tensors)
        del tensors
        g = hip.GgufFile(path)
        infos = {t["name"]: t for t in g.tensors()}
        data_offset = g.header()["data_offset"]
        for n, _, _ in shapes[:2]:  # warm the pinned stage and the runtime
            g.upload_weight(n).free()
        t0 = time.perf_counter()
        ws = [g.upload_weight(n) for n, _, _ in shapes]
        t_map = time.perf_counter() - t0
        for w in ws:
            w.free()
        g.close()
        t0 = time.perf_counter()
        ws = []
        with open(path, "rb") as f:
            for n, m, k in shapes:
                f.seek(data_offset + infos[n]["offset"])
                raw = np.frombuffer(f.read(infos[n]["nbytes"]), np.uint8)
                ws.append(hip.Weight.upload(hip.Q4_0, raw.reshape(-1, 18), m, k))
        t_read = time.perf_counter() - t0
        for w in ws:
            w.free()
    finally:
        os.unlink(path)
    return {"tensors": len(shapes), "bytes": total, "s_mapping_to_hbm": round(t_map, 4),
            "gbs_mapping_to_hbm": round(total / t_map / 1e9, 2), "s_read_then_upload": round(t_read, 4),
            "gbs_read_then_upload": round(total / t_read / 1e9, 2),
            "note": "file in the page cache; host-to-device over PCIe; synthetic Q4_0 blocks"}


def write_llama7b_q4_0(path, layers=32):
    """A LLaMA-7B-shaped Q4_0 model file (dim 4096, hidden 11008, 32 heads,
    vocab 32000; F32 embedding and norms, Q4_0 linears and lm_head) with
    synthetic weights: random nibbles, block scale 2^-10.  Returns its bytes."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import gguf_writer as gw

    dim, hidden, heads, vocab = 4096, 11008, 32, 32000
    rng = np.random.default_rng(5)
    meta = [("general.architecture", gw.STRING, "llama"), ("llama.block_count", gw.U32, layers),
            ("llama.embedding_length", gw.U32, dim), ("llama.feed_forward_length", gw.U32, hidden),
            ("llama.attention.head_count", gw.U32, heads), ("llama.attention.head_count_kv", gw.U32, heads),
            ("llama.context_length", gw.U32, 4096), ("llama.rope.freq_base", gw.F32, 10000.0),
            ("llama.attention.layer_norm_rms_epsilon", gw.F32, 1e-5),
            ("tokenizer.ggml.tokens", gw.ARRAY, (gw.STRING, [f"t{i}" for i in range(vocab)]))]
    specs, kinds = [], []

    def q40(name, m, k):
        specs.append((name, [k, m], gw.GGML_Q4_0, m * (k // 32) * 18))
        kinds.append(("q", m, k))

    def f32(name, shape):
        n = int(np.prod(shape))
        specs.append((name, list(reversed(shape)), gw.GGML_F32, 4 * n))
        kinds.append(("f", n, 0))

    f32("token_embd.weight", (vocab, dim))
    for l in range(layers):
        p = f"blk.{l}."
        f32(p + "attn_norm.weight", (dim,))
        for n in ("attn_q", "attn_k", "attn_v", "attn_output"):
            q40(p + n + ".weight", dim, dim)
        f32(p + "ffn_norm.weight", (dim,))
        q40(p + "ffn_gate.weight", hidden, dim)
        q40(p + "ffn_up.weight", hidden, dim)
        q40(p + "ffn_down.weight", dim, hidden)
    f32("output_norm.weight", (dim,))
    q40("output.weight", vocab, dim)

    def produce(i):
        kind, a, b = kinds[i]
        if kind == "f":
            sd, mean = (0.01, 1.0) if a <= 65536 else (0.02, 0.0)
            return (mean + sd * rng.standard_normal(a)).astype(np.float32).tobytes()
        blocks = rng.integers(0, 256, (a * (b // 32), 18), dtype=np.uint8)
        blocks[:, 0:2] = np.array([0x1400], np.uint16).view(np.uint8)  # d = 2^-10
        return blocks.tobytes()

    gw.write_stream(path, meta, specs, produce)
    return sum(x[3] for x in specs)


def decode_bench(n_new=128, layers=32, cpu=False):
    """Greedy decode on the LLaMA-7B-shaped Q4_0 model of write_llama7b_q4_0
    through mlq_hip_decoder_generate: every op on the device, the picked token
    fed back on the device, one recorded step replayed per token."""
    import tempfile

    fd, path = tempfile.mkstemp(suffix=".gguf")
    os.close(fd)
    cpu_leg = None
    try:
        t0 = time.perf_counter()
        nbytes = write_llama7b_q4_0(path, layers)
        t_write = time.perf_counter() - t0
        t0 = time.perf_counter()
        dec = hip.Decoder(path, max_seq_len=2048)
        t_load = time.perf_counter() - t0
        if cpu:
            cpu_leg = decode_cpu_baseline(path, dec)
    finally:
        os.unlink(path)
    prompt = [1, 2, 3, 4]
    dec.generate(prompt, 8)  # records the step
    t0 = time.perf_counter()
    toks = dec.generate(prompt, n_new)
    dt = time.perf_counter() - t0
    # Batched prefill of a 512-token prompt (one pass of 512 rows: MFMA
    # GEMMs for the linears and the causal attention); one warm-up, then the
    # median of three.
    long_prompt = (np.arange(512) * 7 % 32000).tolist()
    dec.prefill(long_prompt)  # warm-up (GEMM workspace, kernels)
    pre_runs = []
    for _ in range(3):
        t0 = time.perf_counter()
        dec.prefill(long_prompt)
        pre_runs.append(time.perf_counter() - t0)
    dt_pre = sorted(pre_runs)[1]  # median of three
    # Decode at ~1k context: two generations after the same 960-token prompt,
    # 8 and 72 new tokens; their difference is 64 steps at positions 967..1030.
    ctx_prompt = (np.arange(960) * 13 % 32000).tolist()
    times = []
    for n in (8, 72):
        t0 = time.perf_counter()
        dec.generate(ctx_prompt, n)
        times.append(time.perf_counter() - t0)
    dt_ctx = (times[1] - times[0]) / 64
    dec.close()
    # Roofline of both legs: a decode step streams every quantized linear once
    # (Q4_0: 18 bytes per 32 weights); a prefill pass does 2 flops per linear
    # weight and token (attention, norms and RoPE left out).
    lin_params = layers * (4 * 4096 * 4096 + 3 * 11008 * 4096) + 32000 * 4096
    step_bytes = lin_params * 18 // 32
    dec_gbs = step_bytes / (dt / n_new) / 1e9
    pre_tflops = 2.0 * lin_params * len(long_prompt) / dt_pre / 1e12
    return {"model": "llama7b-shaped q4_0 (synthetic weights)", "layers": layers, "prompt_tokens": len(prompt),
            "new_tokens": n_new, "s": round(dt, 4), "tokens_per_s": round(n_new / dt, 1),
            "ms_per_token": round(dt * 1e3 / n_new, 3), "distinct_tokens": len(set(toks)),
            "prefill_tokens": len(long_prompt), "prefill_s": round(dt_pre, 4),
            "prefill_tokens_per_s": round(len(long_prompt) / dt_pre, 1),
            "weight_bytes_per_token": step_bytes, "weight_gbs": round(dec_gbs, 1),
            "weight_frac_of_hbm_peak": round(dec_gbs / HBM_PEAK_GBS, 4),
            "prefill_linear_tflops": round(pre_tflops, 1),
            "tokens_per_s_at_1k_context": round(1.0 / dt_ctx, 1), "ms_per_token_at_1k_context": round(dt_ctx * 1e3, 3),
            "prefill_frac_of_fp16_dense_peak": round(pre_tflops / FP16_PEAK_TFLOPS, 4),
            "file_gb": round(nbytes / 1e9, 3), "s_write_file": round(t_write, 2), "s_load": round(t_load, 2),
            "cpu_baseline": cpu_leg,
            "note": "wall time of one mlq_hip_decoder_generate call (prompt steps, recorded step replayed per "
                    "token, one upload, one download); attention over positions 0..131; the 1k-context rate is the "
                    "difference of two generations after the same 960-token prompt (64 steps at positions 967..1030)"}


def decode_cpu_baseline(path, dec, tokens=(11, 22, 33, 44)):
    """The reference's own load_gguf_model + forward_token (oracle/_ref, the
    threaded CPU path) on the same model file, a bounded sample of tokens;
    its logits also check the device decoder's at full size."""
    import oracle

    ref = oracle.reference()
    if ref is None:
        return None
    threads = os.cpu_count() or 1
    t0 = time.perf_counter()
    rd = ref.decoder(path, threads)
    t_load = time.perf_counter() - t0
    times, worst = [], 0.0
    for pos, t in enumerate(tokens):
        t0 = time.perf_counter()
        want = rd.forward(t, pos)
        times.append(time.perf_counter() - t0)
        got = dec.forward(t, pos)
        worst = max(worst, float(np.abs(got.astype(np.float64) - want).max()) / max(1.0, float(np.abs(want).max())))
    del rd
    per_token = float(np.median(times[1:]))  # the first token is the warm-up
    if worst > 1e-3:
        raise SystemExit(f"decoder logits differ from the reference's by {worst:.2e} of max |logit|")
    return {"kind": "reference", "cores": threads, "cpu_model": cpu_model(), "tokens_per_s": round(1.0 / per_token, 3),
            "ms_per_token": round(per_token * 1e3, 1), "s_load": round(t_load, 2),
            "sample": f"forward_token at positions 0..{len(tokens) - 1}: position 0 is the warm-up, the rate is "
                      f"the median of the other {len(tokens) - 1} ({', '.join(f'{t * 1e3:.0f}' for t in times[1:])} ms)",
            "gpu_vs_reference_max_rel_logit_diff": worst}


def decode_steps_bench(steps):
    """forward() steps (forward_token: logits to the host each step) on the
    model of decode_bench, positions 0..steps-1."""
    import tempfile

    fd, path = tempfile.mkstemp(suffix=".gguf")
    os.close(fd)
    try:
        write_llama7b_q4_0(path)
        dec = hip.Decoder(path, max_seq_len=max(256, steps))
    finally:
        os.unlink(path)
    dec.forward(1, 0)
    t0 = time.perf_counter()
    for pos in range(steps):
        dec.forward(pos % 100 + 1, pos)
    dt = time.perf_counter() - t0
    dec.close()
    return {"forward_steps": steps, "s": round(dt, 4), "ms_per_step": round(dt * 1e3 / steps, 3),
            "note": "each step synchronizes and downloads the logits (forward_token)"}


def prefill_steps_bench(runs=3, tokens=512):
    """Batched prefill only (mlq_hip_decoder_prefill, no generation) of a
    `tokens`-token prompt on the model of decode_bench: one warm-up, then
    `runs` timed prefills (for kernel profiles of the prefill path)."""
    import tempfile

    fd, path = tempfile.mkstemp(suffix=".gguf")
    os.close(fd)
    try:
        write_llama7b_q4_0(path)
        dec = hip.Decoder(path, max_seq_len=max(2048, tokens))
    finally:
        os.unlink(path)
    prompt = (np.arange(tokens) * 7 % 32000).tolist()
    dec.prefill(prompt)
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        dec.prefill(prompt)
        times.append(time.perf_counter() - t0)
    dec.close()
    med = sorted(times)[len(times) // 2]
    return {"prefill_tokens": tokens, "runs": runs, "ms": [round(t * 1e3, 3) for t in times],
            "tokens_per_s_median": round(tokens / med, 1),
            "note": "one warm-up prefill, then the timed ones; each returns the last row's logits to the host"}


PICK_CONFIGS = ([("c2_qwen_lm_head", qt, 151936, 896) for qt in (hip.Q8_0, hip.Q4_0, hip.Q4_1)] +
                [("c3_llama_lm_head", qt, 32000, 4096) for qt in (hip.Q8_0, hip.Q4_0, hip.Q4_1)])


def pick_shape_bench(name, qt, m, k, stream, reps_target=400):
    """Greedy decode's last step: the lm_head GEMV with the argmax fused in
    (mlq_hip_quant_linear_argmax, logits not written) against the plain GEMV
    that writes the logits for a host argmax.  Both as graphs over the same
    cycled weight copies; every copy must pick the plain GEMV's argmax."""
    wbytes, copies, bufs, ws = weight_copies(qt, m, k, 4242 + m + k + qt)
    x = hip.DeviceBuffer(4 * k)
    hip.fill_normal(x, k, 99, 0.0, 1.0)
    y = hip.DeviceBuffer(4 * m)
    tok = hip.DeviceBuffer(4 * copies)
    calls = hip.make_calls([(w, x, y, 1) for w in ws])
    plain = hip.Graph(calls, stream)
    ws[0].linear_argmax(x, None, tok, stream)  # creates the stream's pick state outside capture
    hip.synchronize(stream)

    def issue():
        for i, w in enumerate(ws):
            hip._check(hip.load().mlq_hip_quant_linear_argmax(w.h, x.ptr, None, tok.ptr + 4 * i, stream))

    picked = hip.Graph.record(issue, stream, keep=(x, tok))
    loops = max(1, reps_target // copies)
    plain.launch(stream)
    picked.launch(stream)
    ms_plain = time_region(lambda: plain.launch(stream), loops, stream)
    ms_pick = time_region(lambda: picked.launch(stream), loops, stream)
    hip.synchronize(stream)
    want = int(np.argmax(y.download(np.float32)))
    got = tok.download(np.int32)
    if not (got == want).all():
        raise SystemExit(f"{name}: fused pick {sorted(set(got.tolist()))} != argmax of the GEMV's logits {want}")
    plain.destroy()
    picked.destroy()
    n = loops * copies
    us_plain, us_pick = ms_plain * 1e3 / n, ms_pick * 1e3 / n
    pick_bytes = wbytes + 4.0 * k  # the pick writes no logits
    res = {"name": name, "fmt": FMT_NAME[qt], "M": m, "K": k, "copies": copies,
           "us_gemv_logits": round(us_plain, 3), "us_gemv_argmax": round(us_pick, 3),
           "gbs_argmax": round(pick_bytes / (us_pick * 1e-6) / 1e9, 1),
           "frac_of_peak_argmax": round(pick_bytes / (us_pick * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
           "d2h_bytes_per_token": {"logits": 4 * m, "argmax": 4}, "token": want}
    for w in ws:
        w.free()
    for b in bufs + [x, y, tok]:
        b.free()
    return res


GEMM_CONFIGS = [(qt, m, 4096, n) for qt in (hip.Q8_0, hip.Q4_0) for m in (4096, 11008) for n in (16, 64, 512)]


def gemm_shape_bench(qt, m, k, n, stream, reps_target=100):
    """Y[N, M] = X[N, K] . W^T through the MFMA path, with
    weight copies cycled so the working set exceeds the MALL."""
    wbytes = m * ((k + 31) // 32) * BB[qt]
    copies = max(8, math.ceil(1e9 / wbytes))
    tmp = hip.DeviceBuffer(4 * m * k)
    base = make_weight(qt, m, k, 777 + m + n + qt, tmp)
    tmp.free()
    bufs = [base._keep]
    for _ in range(copies - 1):
        b = hip.DeviceBuffer(wbytes)
        hip.load().mlq_hip_memcpy_dtod(b.ptr, base._keep.ptr, wbytes, None)
        bufs.append(b)
    ws = [hip.Weight.wrap(qt, b, m * ((k + 31) // 32), m, k) for b in bufs]
    x = hip.DeviceBuffer(4 * n * k)
    hip.fill_normal(x, n * k, 31 + n, 0.0, 1.0)
    y = hip.DeviceBuffer(4 * n * m)
    calls = hip.make_calls([(w, x, y, n) for w in ws])
    graph = hip.Graph(calls, stream)
    hip.synchronize(stream)
    loops = max(1, reps_target // copies)
    graph.launch(stream)
    ms = time_region(lambda: graph.launch(stream), loops, stream)
    graph.destroy()
    us = ms * 1e3 / (loops * copies)
    flops = 2.0 * m * k * n
    tflops = flops / (us * 1e-6) / 1e12
    bytes_ = wbytes + 4.0 * n * k + 4.0 * n * m
    res = {"fmt": FMT_NAME[qt], "M": m, "K": k, "N": n, "us_per_call": round(us, 2),
           "tflops": round(tflops, 2), "frac_of_fp16_dense_peak": round(tflops / FP16_PEAK_TFLOPS, 4),
           "gbs": round(bytes_ / (us * 1e-6) / 1e9, 1), "kernel": hip.kernel_name(qt, n, m, k),
           "note": "useful flops 2*M*K*N; the kernel issues 2x that on MFMA (x split hi+lo fp16)"}
    for w in ws:
        w.free()
    for b in bufs:
        b.free()
    return res


_JSON_FD = None


STAGE_NAMES = ("q/k/v fused 12288x4096", "o 4096x4096", "gate/up fused 22016x4096", "down 4096x11008")


def profile_summary(path: str, steps: int, stages: int = 129) -> None:
    """Per-stage table of a rocprofv3 CSV output directory (`-f csv`) of a
    `--no-shapes --no-cpu --no-variants --launch per_stage` run: the last
    `steps` x `stages` dispatches of the GEMV kernels, of the f32 GEMV, of the
    stream floor kernel and of the two probes (empty launch, load only), i.e.
    the timed steps of each leg (each leg runs its warm-up steps before its
    timed ones).  A kernel trace gives durations (per step from the per-stage
    medians, which the tracer's occasional stretched dispatch does not move,
    and from the means); a counter collection gives each counter's mean per
    dispatch.  Returns the text."""
    import csv
    import glob
    import statistics

    lines = []
    out = lines.append

    def family(name):
        if "gemv_single" in name or "gemv_multi" in name:
            return "gemv"
        for key, fam in (("gemv_f32", "f32"), ("stream_floor", "floor"), ("probe_empty", "empty"),
                         ("probe_load", "load")):
            if key in name:
                return fam
        return None

    families = ("gemv", "f32", "floor", "load", "empty")

    def short(name):
        return name.replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0]

    def stage(i):
        return "lm_head 32000x4096" if i % stages == stages - 1 else STAGE_NAMES[(i % stages) % 4]

    last = steps * stages
    trace = glob.glob(os.path.join(path, "**", "*kernel_trace.csv"), recursive=True)
    counters = glob.glob(os.path.join(path, "**", "*counter_collection.csv"), recursive=True)
    if trace:
        rows = sorted(csv.DictReader(open(trace[0])), key=lambda r: int(r["Start_Timestamp"]))
        for fam in families:
            sel = [r for r in rows if family(r["Kernel_Name"]) == fam][-last:]
            if len(sel) < last:
                continue
            out(f"\n{fam}: last {len(sel)} dispatches ({steps} steps)\n")
            out("| kernel | stage | dispatches | avg us | median us | min us | max us |")
            out("|---|---|---|---|---|---|---|")
            by = {}
            for i, r in enumerate(sel):
                key = (short(r["Kernel_Name"]), stage(i))
                by.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
            total = 0.0
            total_med = 0.0
            for (k, st), v in by.items():
                total += sum(v)
                total_med += statistics.median(v) * len(v) / steps
                out(f"| {k} | {st} | {len(v)} | {statistics.mean(v):.3f} | {statistics.median(v):.3f} | "
                      f"{min(v):.3f} | {max(v):.3f} |")
            out(f"\nkernel time per step {total_med:.1f} us from the per-stage medians "
                f"({total_med * steps / len(sel):.3f} us per launch); {total / steps:.1f} us from the means")
    if counters:
        per = {}
        for r in csv.DictReader(open(counters[0])):
            per.setdefault(int(r["Dispatch_Id"]), [r["Kernel_Name"], {}])[1][r["Counter_Name"]] = float(r["Counter_Value"])
        ids = sorted(per)
        for fam in families:
            sel = [i for i in ids if family(per[i][0]) == fam][-last:]
            if len(sel) < last:
                continue
            names = sorted(per[sel[0]][1])
            out(f"\n{fam}: last {len(sel)} dispatches ({steps} steps), mean per dispatch\n")
            out("| kernel | stage | dispatches | " + " | ".join(names) + " |")
            out("|---|---|---|" + "---|" * len(names))
            by = {}
            for j, i in enumerate(sel):
                by.setdefault((short(per[i][0]), stage(j)), []).append(per[i][1])
            for (k, st), v in by.items():
                out(f"| {k} | {st} | {len(v)} | " +
                      " | ".join(f"{statistics.mean(d[n] for d in v):.1f}" for n in names) + " |")
        copies = [per[i][1] for i in ids if "copyBuffer" in per[i][0]]
        if copies:
            big = max(copies, key=lambda d: sum(d.values()))
            out("\nlargest __amd_rocclr_copyBuffer dispatch (the calibration copy): " +
                  ", ".join(f"{n} {v:.1f}" for n, v in sorted(big.items())))
    return "\n".join(lines) + "\n"


def kernel_summary(path: str, match=("gemm_", "xsplit_kernel")) -> str:
    """Per-kernel table of a rocprofv3 CSV output directory (`-f csv`) of a
    `--gemm-only` run: every dispatch of each kernel whose name contains one
    of `match`, grouped by full kernel name (template arguments included);
    durations from a kernel trace, each counter's mean per dispatch from a
    counter collection, and the largest copyBuffer dispatch (the
    `--calibration-copy-mb` copy) for scaling byte counters.  Returns the text."""
    import csv
    import glob
    import statistics

    lines = []
    out = lines.append

    def short(name):
        return name.replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0]

    trace = glob.glob(os.path.join(path, "**", "*kernel_trace.csv"), recursive=True)
    counters = glob.glob(os.path.join(path, "**", "*counter_collection.csv"), recursive=True)
    if trace:
        by = {}
        for r in csv.DictReader(open(trace[0])):
            if any(m in r["Kernel_Name"] for m in match):
                by.setdefault(short(r["Kernel_Name"]), []).append(
                    (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        out("| kernel | dispatches | avg us | median us | min us | max us |")
        out("|---|---|---|---|---|---|")
        for k, v in by.items():
            out(f"| {k} | {len(v)} | {statistics.mean(v):.3f} | {statistics.median(v):.3f} | "
                f"{min(v):.3f} | {max(v):.3f} |")
    if counters:
        per = {}
        for r in csv.DictReader(open(counters[0])):
            per.setdefault(int(r["Dispatch_Id"]), [r["Kernel_Name"], {}])[1][r["Counter_Name"]] = float(r["Counter_Value"])
        by = {}
        for i in sorted(per):
            if any(m in per[i][0] for m in match):
                by.setdefault(short(per[i][0]), []).append(per[i][1])
        if by:
            names = sorted(next(iter(by.values()))[0])
            out("\n| kernel | dispatches | " + " | ".join(names) + " |")
            out("|---|---|" + "---|" * len(names))
            for k, v in by.items():
                out(f"| {k} | {len(v)} | " + " | ".join(f"{statistics.mean(d.get(n, 0.0) for d in v):.1f}"
                                                        for n in names) + " |")
        copies = [d for name, d in per.values() if "copyBuffer" in name]
        if copies:
            big = max(copies, key=lambda d: sum(d.values()))
            out("\nlargest __amd_rocclr_copyBuffer dispatch (the calibration copy): " +
                ", ".join(f"{n} {v:.1f}" for n, v in sorted(big.items())))
    return "\n".join(lines) + "\n"


def calibration_copy(mb: int, stream) -> None:
    """One device-to-device copy of `mb` MiB: a dispatch of known traffic
    against which a profiler's byte counters are scaled."""
    nbytes = mb << 20
    src, dst = hip.DeviceBuffer(nbytes), hip.DeviceBuffer(nbytes)
    hip.load().mlq_hip_memcpy_dtod(dst.ptr, src.ptr, nbytes, stream)
    hip.synchronize(stream)
    log(f"calibration copy: {nbytes} bytes read and written")
    src.free()
    dst.free()


def ring_stamps_report(layers: int, steps: int, warmup: int, stream) -> str:
    """Per-stage boundary timestamps of the LDS-ring persistent chain on the
    sweep (the measurement build's s_memrealtime stamps, 100 MHz), as markdown:
    per stage kind, the median over the timed launches and layers 1 .. L-1 of
    each interval, for the three stamped workgroups."""
    sw = Sweep(layers=layers)
    seq = hip.Sequence(sw.calls, sw.stage_ids(), hip.SEQ_LDS_RING)
    for _ in range(warmup):
        seq.launch(stream)
    hip.synchronize(stream)
    runs, walls = [], []
    for _ in range(steps):
        seq.launch(stream)
        hip.synchronize(stream)
        runs.append(hip.ring_stamps().astype(np.int64))
    if seq.status() != 0:
        raise SystemExit("ring stamps: a barrier or ring wait timed out")
    nst = len(set(sw.stage_ids()))
    kinds = ["q/k/v", "o", "gate/up", "down"]
    cols = [("y stores complete", 0, 1), ("all compute waves done", 1, 2), ("grid barrier", 2, 3),
            ("x staged", 3, 4), ("all x staged", 4, 5), ("to first unit", 5, 6), ("first unit's wait", 6, 7)]
    out = [f"LDS-ring persistent chain on the sweep ({layers} layers, {nst} stages): {steps} timed launches after "
           f"{warmup} warm-up; µs, medians over launches and layers 1..{layers - 1}; loader times relative to "
           "the stage's entry (negative: before it)\n"]
    for wi, wname in enumerate(["0", "G/2 + 1", "G - 1"]):
        per = {k: {} for k in kinds}
        for st in runs:
            a = st[wi]
            walls.append((a[nst - 1, 8:20].max() - a[0, 0]) / 100.0)
            for s in range(4, min(nst - 1, 4 * layers)):
                d = per[kinds[s % 4]]
                e = a[s]
                for name, i0, i1 in cols:
                    d.setdefault(name, []).append((e[i1] - e[i0]) / 100.0)
                d.setdefault("rows (first unit to last wave done)", []).append((e[8:20].max() - e[7]) / 100.0)
                d.setdefault("stage (entry to next entry)", []).append((a[s + 1, 0] - e[0]) / 100.0)
                d.setdefault("loader: first unit requested", []).append((e[22] - e[0]) / 100.0)
                d.setdefault("loader: first unit in LDS", []).append((e[20] - e[0]) / 100.0)
                d.setdefault("loader: last unit in LDS", []).append((e[21] - e[0]) / 100.0)
        names = list(per[kinds[0]].keys())
        out.append(f"\nworkgroup {wname}: stage 0 entry to the last stage's end "
                   f"{np.median(walls[-len(runs):]):.1f} µs (median over launches)\n")
        out.append("| interval | " + " | ".join(kinds) + " |")
        out.append("|---|" + "---|" * len(kinds))
        for n in names:
            out.append(f"| {n} | " + " | ".join(f"{np.median(per[k][n]):.2f}" for k in kinds) + " |")
    seq.destroy()
    sw.free()
    return "\n".join(out) + "\n"


def emit(obj):
    """Writes the one JSON line to the process's original stdout.  main()
    points fd 1 at stderr first: C code loaded here (the reference's GGUF
    loader behind the CPU baseline among it) prints progress on stdout."""
    line = (json.dumps(obj) + "\n").encode()
    os.write(_JSON_FD if _JSON_FD is not None else 1, line)


def main():
    global _JSON_FD
    sys.stdout.flush()
    _JSON_FD = os.dup(1)
    os.dup2(2, 1)
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--launch", choices=["graph", "plain", "sequence", "per_stage", "independent", "pipelined", "lds_ring"],
                    default="per_stage")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline / parity leg")
    ap.add_argument("--no-shapes", action="store_true", help="skip the per-shape GEMV / GEMM tables")
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-probes", action="store_true",
                    help="skip the f32 GEMV, empty-launch and load-only legs (profiled runs: one of those "
                         "graph launches ended in a host SIGSEGV under rocprofv3's kernel trace)")
    ap.add_argument("--no-variants", action="store_true",
                    help="time only the --launch mode (for profiling one mode's kernels)")
    ap.add_argument("--calibration-copy-mb", type=int, default=0,
                    help="before timing, run one device-to-device copy of this many MiB: a kernel of "
                         "known traffic that scales the rocprofv3 FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the device-resident decode leg and print its JSON")
    ap.add_argument("--decode-steps", type=int, default=0,
                    help="with --decode-only: instead run this many single forward() steps (one launch "
                         "sequence per token, no recorded graph) on the same model, for kernel profiles")
    ap.add_argument("--prefill-runs", type=int, default=0,
                    help="with --decode-only: instead run only batched prefills of a 512-token prompt "
                         "(one warm-up, then this many timed), for kernel profiles of the prefill path")
    ap.add_argument("--gemm-only", action="store_true",
                    help="run only the prefill GEMM table (config 4) and print it as one JSON line")
    ap.add_argument("--gemm-filter", default="",
                    help="with --gemm-only: keep the configs named fmt:M:N (comma-separated, e.g. q4_0:4096:64); "
                         "fmt:M:N:K adds a shape with K other than 4096")
    ap.add_argument("--profile-summary", default="",
                    help="print per-stage tables of this rocprofv3 CSV output directory (of a --launch "
                         "per_stage --no-variants run with the same --steps) and exit; no GPU use")
    ap.add_argument("--ring-stamps", action="store_true",
                    help="load the measurement build (libmlq_hip_stamps.so: make -C mini-llama-cpp-release_amd "
                         "stamps), run the sweep in the lds_ring mode --steps times after --warmup and print "
                         "its per-stage boundary timestamps as tables")
    ap.add_argument("--kernel-summary", default="",
                    help="print per-kernel tables (GEMM and x split) of this rocprofv3 CSV output "
                         "directory (of a --gemm-only run) and exit; no GPU use")
    args = ap.parse_args()
    if args.profile_summary:
        os.write(_JSON_FD, profile_summary(args.profile_summary, args.steps).encode())
        return
    if args.kernel_summary:
        os.write(_JSON_FD, kernel_summary(args.kernel_summary).encode())
        return
    if args.ring_stamps:
        hip.load(hip.STAMPS_LIB_PATH)
        hip.init(0)
        os.write(_JSON_FD, ring_stamps_report(args.layers, args.steps, args.warmup, hip.stream(0)).encode())
        return
    if args.gemm_only:
        hip.load()
        hip.init(0)
        stream = hip.stream(0)
        keep = {f for f in args.gemm_filter.split(",") if f}
        if args.calibration_copy_mb > 0:
            calibration_copy(args.calibration_copy_mb, stream)
        rows = []
        configs = list(GEMM_CONFIGS)
        by_name = {v: k for k, v in FMT_NAME.items()}
        for f in sorted(keep):
            parts = f.split(":")
            if len(parts) == 4:  # fmt:M:N:K, a shape outside the config-4 list
                configs.append((by_name[parts[0]], int(parts[1]), int(parts[3]), int(parts[2])))
        for cfg in configs:
            qt, m, k, n = cfg
            name = f"{FMT_NAME[qt]}:{m}:{n}" + ("" if k == 4096 else f":{k}")
            if keep and name not in keep:
                continue
            r = gemm_shape_bench(*cfg, stream)
            log(f"  gemm {r['fmt']} {r['M']:>6}x{r['K']:<5} N={r['N']:<4} {r['us_per_call']:9.2f} us "
                f"{r['tflops']:8.1f} TFLOP/s ({100 * r['frac_of_fp16_dense_peak']:.1f}% of fp16 peak) "
                f"{r['gbs']:8.1f} GB/s {r['kernel']}")
            rows.append(r)
        emit({"gemm": rows})
        return
    if args.decode_only:
        hip.load()
        hip.init(0)
        if args.decode_steps > 0:
            emit(decode_steps_bench(args.decode_steps))
        elif args.prefill_runs > 0:
            emit(prefill_steps_bench(args.prefill_runs))
        else:
            emit(decode_bench())
        return

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(the sweep shards by output rows across GPUs by design, but no multi-GPU path is "
              "built or measured)", file=sys.stderr)
        sys.exit(2)

    hip.load()
    hip.init(0)
    stream = hip.stream(0)
    log(hip.device_info(0))
    t0 = time.time()
    sw = Sweep(layers=args.layers)
    log(f"sweep ready: {sw.n()} calls, {sw.bytes / 1e9:.3f} GB, setup {time.time() - t0:.1f}s")

    if args.calibration_copy_mb > 0:
        calibration_copy(args.calibration_copy_mb, stream)

    # Every way of running the sweep; `--launch` picks the headline.
    #   graph / plain: one launch per call (225), captured as a graph or issued from C;
    #   sequence:  one persistent launch, barriers between the 129 dependent stages;
    #   per_stage: one grouped launch per stage (129), captured as a graph;
    #   independent: one persistent launch without barriers (the sweep's inputs are
    #              all fresh, so nothing depends on anything; reported, not headline).
    seqs = {m: hip.Sequence(sw.calls, sw.stage_ids(), mode)
            for m, mode in (("sequence", hip.SEQ_PERSISTENT), ("per_stage", hip.SEQ_PER_STAGE),
                            ("independent", hip.SEQ_INDEPENDENT), ("pipelined", hip.SEQ_PIPELINED),
                            ("lds_ring", hip.SEQ_LDS_RING))}
    graph = hip.Graph(sw.calls, stream)
    stage_graph = hip.Graph(sequence=seqs["per_stage"])
    steps_by_mode = {
        "graph": lambda: graph.launch(stream),
        "plain": lambda: hip.linear_many(sw.calls, stream),
        "sequence": lambda: seqs["sequence"].launch(stream),
        "per_stage": lambda: stage_graph.launch(stream),
        "independent": lambda: seqs["independent"].launch(stream),
        "pipelined": lambda: seqs["pipelined"].launch(stream),
        "lds_ring": lambda: seqs["lds_ring"].launch(stream),
    }
    variants = {}
    for name, fn in steps_by_mode.items():
        if args.no_variants and name != args.launch:
            continue
        for _ in range(args.warmup):
            fn()
        hip.synchronize(stream)
        variants[name] = time_region(fn, args.steps, stream) / args.steps
        for sq in seqs.values():
            if sq.status() != 0:
                raise SystemExit(f"sweep {name}: a sequence barrier wait timed out")
        log(f"sweep {name:12s}: {variants[name] * 1e3:8.1f} us/step, "
            f"{sw.bytes / (variants[name] * 1e-3) / 1e9:8.1f} GB/s")
    # The headline mode runs last before the parity check, so the outputs the
    # CPU compares are the headline's.
    step = steps_by_mode[args.launch]
    for _ in range(args.warmup):
        step()
    hip.synchronize(stream)
    for y in sw.ys:
        y.fill(0)
    ms = time_region(step, args.steps, stream)
    ms_step = ms / args.steps
    gbs = sw.bytes / (ms_step * 1e-3) / 1e9
    floor = floor_bench(sw, stream, args.steps, args.warmup)
    log(f"sweep floor (weights only, one launch per stage): {floor['us_per_step']:8.1f} us/step, "
        f"{floor['gbs']:8.1f} GB/s")
    f32_line = f32_rerun = f32_graph = empty = load_only = None
    if not args.no_probes:
        f32_line, f32_rerun, f32_graph = f32_sweep_bench(sw, stream, args.steps, args.warmup)
        log(f"sweep f32 GEMV (the reference's arithmetic, one launch per stage): {f32_line['us_per_step']:8.1f} "
            f"us/step, {f32_line['gbs']:8.1f} GB/s")
        # The headline's outputs again for the CPU check below (the f32 sweep wrote them).
        step()
        hip.synchronize(stream)
        empty = floor_bench(sw, stream, args.steps, args.warmup, hip.PROBE_EMPTY)
        load_only = floor_bench(sw, stream, args.steps, args.warmup, hip.PROBE_LOAD)
        log(f"sweep launch cost (129 empty dependent launches): {empty['us_per_step']:8.1f} us/step, "
            f"{empty['us_per_launch']:.3f} us/launch; load-only chain: {load_only['us_per_step']:8.1f} us/step, "
            f"{load_only['gbs']:8.1f} GB/s")
    seq_info = seqs["sequence"].info()
    launches = {"graph": sw.n(), "plain": sw.n(), "per_stage": seqs["per_stage"].info()["launches"],
                "sequence": seq_info["launches"], "independent": seqs["independent"].info()["launches"],
                "pipelined": seqs["pipelined"].info()["launches"],
                "lds_ring": seqs["lds_ring"].info()["launches"]}[args.launch]
    log(f"sweep: {ms_step * 1e3:.1f} us/step, {gbs:.1f} GB/s ({args.launch}); sequence {seq_info}")

    shapes = []
    if not args.no_shapes:
        side = [hip.stream_create(0) for _ in range(4)]
        for cfg in GEMV_CONFIGS:
            r = gemv_shape_bench(*cfg, stream, streams=side if cfg[0].startswith("c3_") else None)
            ov = r.get("independent_streams")
            log(f"  {r['name']:22s} {r['fmt']} {r['M']:>6}x{r['K']:<6} {r['us_per_call']:8.2f} us "
                f"{r['gbs']:8.1f} GB/s ({100 * r['frac_of_peak']:.1f}%) {r['kernel']}" +
                (f"; 4 independent streams {ov['us_per_call']:.2f} us ({100 * ov['frac_of_peak']:.1f}%)" if ov else ""))
            shapes.append(r)
        for st in side:
            hip.stream_destroy(st)

    picks = []
    if not args.no_shapes:
        for cfg in PICK_CONFIGS:
            r = pick_shape_bench(*cfg, stream)
            log(f"  pick {r['name']:18s} {r['fmt']} {r['M']:>6}x{r['K']:<5} GEMV+logits {r['us_gemv_logits']:7.2f} us, "
                f"GEMV+argmax {r['us_gemv_argmax']:7.2f} us ({100 * r['frac_of_peak_argmax']:.1f}% of peak), "
                f"token {r['token']}")
            picks.append(r)

    decode = None
    if not args.no_shapes:
        decode = decode_bench(cpu=not args.no_cpu)
        log(f"  decode {decode['model']}: {decode['tokens_per_s']} tokens/s ({decode['ms_per_token']} ms/token, "
            f"weights at {decode['weight_gbs']} GB/s = {100 * decode['weight_frac_of_hbm_peak']:.1f}% of HBM peak), "
            f"batched prefill {decode['prefill_tokens_per_s']} tokens/s ({decode['prefill_linear_tflops']} TFLOP/s "
            f"in the linears), load {decode['s_load']} s")

    ingest = None
    if not args.no_shapes:
        ingest = ingest_bench()
        log(f"  gguf ingest {ingest['bytes'] / 1e6:.0f} MB in {ingest['tensors']} tensors: mapping -> HBM "
            f"{ingest['gbs_mapping_to_hbm']} GB/s, read then upload {ingest['gbs_read_then_upload']} GB/s")

    gemm = []
    if not args.no_shapes:
        for cfg in GEMM_CONFIGS:
            r = gemm_shape_bench(*cfg, stream)
            log(f"  gemm {r['fmt']} {r['M']:>6}x{r['K']:<5} N={r['N']:<4} {r['us_per_call']:9.2f} us "
                f"{r['tflops']:8.1f} TFLOP/s ({100 * r['frac_of_fp16_dense_peak']:.1f}% of fp16 peak) "
                f"{r['gbs']:8.1f} GB/s {r['kernel']}")
            gemm.append(r)

    cpu = None
    parity = None
    if not args.no_cpu:
        import oracle

        threads = os.cpu_count() or 1
        chk = cpu_sweep_check(sw, threads, alt=f32_rerun)
        if f32_line is not None:
            f32_line["worst_err_over_bound"] = round(chk["worst_err_over_bound_alt"], 6)
        cpu = {"value": round(chk["cpu_bytes"] / chk["cpu_s"] / 1e9, 3), "unit": "GB/s",
               "cores": threads, "cpu_model": cpu_model(), "kind": chk["kind"],
               "sample": f"whole sweep ({sw.n()} calls, {chk['cpu_bytes'] / 1e9:.3f} GB): one warm-up sweep "
                         f"({chk['cpu_s_warmup'] * 1e3:.0f} ms), then the median of {len(chk['cpu_s_runs'])} "
                         f"timed sweeps ({', '.join(f'{t * 1e3:.0f}' for t in chk['cpu_s_runs'])} ms); "
                         f"the reference's threaded linear() with {threads} threads",
               "ms_per_sweep": round(chk["cpu_s"] * 1e3, 1)}
        parity = {"outputs_within_tolerance": True,
                  "worst_err_over_bound": round(chk["worst_err_over_bound"], 4),
                  "argmax_gpu": chk["argmax_gpu"], "argmax_cpu": chk["argmax_cpu"],
                  "argmax_match": chk["argmax_gpu"] == chk["argmax_cpu"],
                  "argmax_top2_gap": chk["argmax_top2_gap"]}
        log(f"cpu baseline: {cpu}; parity: {parity}")
        if not parity["argmax_match"]:
            raise SystemExit("argmax mismatch between GPU and CPU sweep")

    if f32_graph is not None:
        f32_graph.destroy()
    out = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8 dot4 -> i32, f32 accumulate",
        "dtype_detail": ("x as a block-scaled integer per 32 elements (Q4_0/Q4_1: 16-bit, two int8 limbs; "
                         "Q8_0: 23-bit, three limbs), weights as stored (u4 nibbles / i8), exact int32 "
                         "block sums from v_dot4, then f32 scaling and f32 row accumulation"),
        "data": "synthetic (device-generated N(0,0.02) weights quantized by the reference's Q4_0 rule, x~N(0,1))",
        "config": {"workload": "llama7b_q4_0_decode_linear_sweep", "layers": args.layers,
                   "calls_per_step": sw.n(), "stages_per_step": seq_info["stages"],
                   "bytes_per_step": sw.bytes, "launch": args.launch,
                   "sweep_us": round(ms_step * 1e3, 1),
                   "sweep_us_by_launch": {k: round(v * 1e3, 1) for k, v in variants.items()},
                   "per_stage_f32_gemv": f32_line,
                   "per_stage_floor": floor, "per_stage_empty_launches": empty,
                   "per_stage_load_only": load_only},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(args.launch),
                     "algorithmic_bytes_per_launch": round(sw.bytes / launches),
                     "launches_per_step": launches,
                     "avg_launch_us": round(ms_step * 1e3 / launches, 3),
                     "kernel": KERNEL_BY_LAUNCH[args.launch]},
        "cpu_baseline": cpu,
        "parity": parity,
        "gemv": shapes,
        "lm_head_argmax": picks,
        "gguf_ingest": ingest,
        "decode": decode,
        "gemm": gemm,
    }
    emit(out)


if __name__ == "__main__":
    main()

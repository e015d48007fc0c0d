"""The BASELINE config 5 workload (test and bench infrastructure): a
LLaMA-7B-shaped Q4_0 decode linear sweep, 32 layers x (q, k, v, o 4096x4096;
gate, up 11008x4096; down 4096x11008) plus lm_head 32000x4096 = 225 GEMV calls
over 3.727 GB of device-resident weights generated and quantized on the device
(the reference's Q4_0 rule, src/quant.cpp:207-270), with a fresh x ~ N(0, 1)
per layer (x for q..up, h for down).  Shared by bench.py (the headline) and
tests/test_gpu_sweep.py (its parity against the CPU linear)."""

from __future__ import annotations

import mlq_hip as hip

BB = {hip.Q8_0: 34, hip.Q4_0: 18, hip.Q4_1: 20}


def gemv_bytes(qt, m, k):
    return m * ((k + 31) // 32) * BB[qt] + 4 * k + 4 * m


def make_weight(qt, m, k, seed, tmp):
    """Generate W ~ N(0, 0.02) on the device and quantize it in place (device
    quantizer, bit-identical to the reference quantizers)."""
    nbytes = m * ((k + 31) // 32) * BB[qt]
    blocks = hip.DeviceBuffer(nbytes)
    hip.fill_normal(tmp, m * k, seed, 0.0, 0.02)
    hip.quantize_device(qt, tmp, m, k, blocks)
    return hip.Weight.wrap(qt, blocks, m * ((k + 31) // 32), m, k)


# ------------------------------------------------------------------ sweep
LAYER = [("q", 4096, 4096, "x"), ("k", 4096, 4096, "x"), ("v", 4096, 4096, "x"),
         ("o", 4096, 4096, "x"), ("gate", 11008, 4096, "x"), ("up", 11008, 4096, "x"),
         ("down", 4096, 11008, "h")]


class Sweep:
    def __init__(self, layers=32, qt=hip.Q4_0, seed=7):
        self.qt = qt
        tmp = hip.DeviceBuffer(4 * 32000 * 4096)  # f32 scratch for the largest weight (lm_head)
        self.weights, self.calls_desc, self.ys, self.xs = [], [], [], []
        for l in range(layers):
            x = hip.DeviceBuffer(4 * 4096)
            h = hip.DeviceBuffer(4 * 11008)
            hip.fill_normal(x, 4096, seed * 1000003 + 2 * l, 0.0, 1.0)
            hip.fill_normal(h, 11008, seed * 1000003 + 2 * l + 1, 0.0, 1.0)
            self.xs.append((x, h))
            for j, (name, m, k, src) in enumerate(LAYER):
                w = make_weight(qt, m, k, seed * 7919 + 16 * l + j, tmp)
                y = hip.DeviceBuffer(4 * m)
                self.weights.append(w)
                self.ys.append(y)
                self.calls_desc.append((f"layers.{l}.{name}", w, x if src == "x" else h, y))
        xf = hip.DeviceBuffer(4 * 4096)
        hip.fill_normal(xf, 4096, seed * 1000003 + 999_999, 0.0, 1.0)
        self.x_final = xf
        lm = make_weight(qt, 32000, 4096, seed * 7919 + 999_999, tmp)
        ylm = hip.DeviceBuffer(4 * 32000)
        self.weights.append(lm)
        self.ys.append(ylm)
        self.calls_desc.append(("lm_head", lm, xf, ylm))
        hip.synchronize(hip.stream(0))
        tmp.free()
        self.calls = hip.make_calls([(w, x, y, 1) for (_, w, x, y) in self.calls_desc])
        self.bytes = sum(gemv_bytes(qt, w.m, w.k) for (_, w, _, _) in self.calls_desc)

    def n(self):
        return len(self.calls_desc)

    def stage_ids(self):
        """Decode data flow per layer: q,k,v share x | o | gate,up share x | down;
        lm_head last.  Every change of id is a dependency barrier."""
        ids = []
        for l in range(len(self.calls_desc) // len(LAYER)):
            ids += [4 * l, 4 * l, 4 * l, 4 * l + 1, 4 * l + 2, 4 * l + 2, 4 * l + 3]
        ids.append(ids[-1] + 1 if ids else 0)
        return ids

    def free(self):
        """Releases the sweep's device memory (3.7 GB at 32 layers)."""
        for w in self.weights:
            w.free()
            if w._keep is not None:
                w._keep.free()
        for b in self.ys:
            b.free()
        for x, h in self.xs:
            x.free()
            h.free()
        self.x_final.free()

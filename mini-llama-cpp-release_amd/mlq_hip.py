"""ctypes binding of libmlq_hip.so (include/mlq_hip.h) for tests, bench and smoke.

This is plumbing, not a second implementation: every entry calls the C ABI,
and there is no CPU fallback -- ``load()`` raises if the HIP library was not
built, and every call raises ``MlqError`` with the library's message when the
C ABI returns a nonzero code.

The module deliberately does not import torch: the library owns its device
memory, streams and events, so a process never carries two HIP runtimes.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmlq_hip.so")

F32, Q8_0, Q4_0, Q4_1 = 0, 1, 2, 3
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18, Q4_1: 20}
QK = 32
X_ON_DEVICE, Y_ON_DEVICE, ASYNC = 1, 2, 4
SEQ_PERSISTENT, SEQ_PER_STAGE, SEQ_INDEPENDENT, SEQ_PIPELINED, SEQ_LDS_RING = 0, 1, 2, 3, 4

_vp = ctypes.c_void_p


class MlqError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[mlq {code}] {msg}")
        self.code = code
        self.msg = msg


class LinearCall(ctypes.Structure):
    _fields_ = [("w", _vp), ("x", _vp), ("y", _vp), ("rows", ctypes.c_int)]


class DecoderConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("n_layers", "dim", "hidden_dim", "n_heads", "n_kv_heads", "head_dim",
                                              "vocab_size", "max_seq_len")] + \
               [("rope_theta", ctypes.c_float), ("rms_norm_eps", ctypes.c_float), ("rope_neox", ctypes.c_int)]


class DeviceProps(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64), ("major", ctypes.c_int),
                ("minor", ctypes.c_int), ("total_memory_bytes", ctypes.c_size_t), ("compute_units", ctypes.c_int),
                ("driver_version", ctypes.c_int), ("runtime_version", ctypes.c_int)]


_LIB = None

_SIGS = {
    "mlq_hip_last_error": (ctypes.c_char_p, []),
    "mlq_hip_built": (ctypes.c_int, []),
    "mlq_hip_device_count": (ctypes.c_int, [ctypes.POINTER(ctypes.c_int)]),
    "mlq_hip_device_info": (ctypes.c_int, [ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t]),
    "mlq_hip_device_props": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(DeviceProps)]),
    "mlq_hip_init": (ctypes.c_int, [ctypes.c_int]),
    "mlq_hip_upload_weight": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _vp, ctypes.c_size_t,
                                              ctypes.c_int, ctypes.c_int, ctypes.POINTER(_vp)]),
    "mlq_hip_wrap_weight": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _vp, ctypes.c_size_t,
                                            ctypes.c_int, ctypes.c_int, ctypes.POINTER(_vp)]),
    "mlq_hip_free_weight": (ctypes.c_int, [_vp]),
    "mlq_hip_weight_info": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int),
                                            ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_size_t),
                                            ctypes.POINTER(_vp), ctypes.POINTER(ctypes.c_int)]),
    "mlq_hip_quant_linear": (ctypes.c_int, [_vp, _vp, ctypes.c_int, _vp, ctypes.c_int, _vp]),
    "mlq_hip_quant_linear_noalloc": (ctypes.c_int, [_vp, _vp, ctypes.c_int, _vp, _vp]),
    "mlq_hip_stream_floor": (ctypes.c_int, [ctypes.POINTER(LinearCall), ctypes.c_int, _vp, _vp]),
    "mlq_hip_quant_linear_fused_f32": (ctypes.c_int, [ctypes.POINTER(LinearCall), ctypes.c_int, _vp]),
    "mlq_hip_stream_probe": (ctypes.c_int, [ctypes.POINTER(LinearCall), ctypes.c_int, ctypes.c_int, _vp, _vp]),
    "mlq_hip_ring_stamps": (ctypes.c_int, [_vp, ctypes.c_size_t]),
    "mlq_hip_quant_linear_device": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _vp, ctypes.c_size_t,
                                                    ctypes.c_int, ctypes.c_int, _vp, ctypes.c_int, _vp, _vp]),
    "mlq_hip_quant_linear_many": (ctypes.c_int, [ctypes.POINTER(LinearCall), ctypes.c_int, _vp]),
    "mlq_hip_quant_linear_fused": (ctypes.c_int, [ctypes.POINTER(LinearCall), ctypes.c_int, _vp]),
    "mlq_hip_quant_linear_argmax": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp]),
    "mlq_hip_sample_greedy": (ctypes.c_int, [_vp, _vp, _vp, ctypes.POINTER(ctypes.c_int), _vp]),
    "mlq_hip_quantize": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _vp, ctypes.c_int, ctypes.c_int, _vp, _vp]),
    "mlq_hip_malloc": (ctypes.c_int, [ctypes.c_int, ctypes.c_size_t, ctypes.POINTER(_vp)]),
    "mlq_hip_free": (ctypes.c_int, [_vp]),
    "mlq_hip_memcpy_htod": (ctypes.c_int, [_vp, _vp, ctypes.c_size_t]),
    "mlq_hip_memcpy_dtoh": (ctypes.c_int, [_vp, _vp, ctypes.c_size_t]),
    "mlq_hip_memcpy_dtod": (ctypes.c_int, [_vp, _vp, ctypes.c_size_t, _vp]),
    "mlq_hip_memset": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_size_t]),
    "mlq_hip_stream": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(_vp)]),
    "mlq_hip_stream_create": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(_vp)]),
    "mlq_hip_stream_destroy": (ctypes.c_int, [_vp]),
    "mlq_hip_synchronize": (ctypes.c_int, [_vp]),
    "mlq_hip_event_create": (ctypes.c_int, [ctypes.POINTER(_vp)]),
    "mlq_hip_event_destroy": (ctypes.c_int, [_vp]),
    "mlq_hip_event_record": (ctypes.c_int, [_vp, _vp]),
    "mlq_hip_event_elapsed_ms": (ctypes.c_int, [_vp, _vp, ctypes.POINTER(ctypes.c_float)]),
    "mlq_hip_graph_capture_many": (ctypes.c_int, [ctypes.POINTER(LinearCall), ctypes.c_int, _vp,
                                                   ctypes.POINTER(_vp)]),
    "mlq_hip_graph_launch": (ctypes.c_int, [_vp, _vp]),
    "mlq_hip_graph_destroy": (ctypes.c_int, [_vp]),
    "mlq_hip_gguf_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "mlq_hip_gguf_close": (ctypes.c_int, [_vp]),
    "mlq_hip_gguf_header": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint64),
                                            ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "mlq_hip_gguf_metadata": (ctypes.c_int, [_vp, ctypes.c_uint64, ctypes.c_char_p, ctypes.c_size_t,
                                              ctypes.POINTER(ctypes.c_uint32), ctypes.c_char_p, ctypes.c_size_t]),
    "mlq_hip_gguf_tensor": (ctypes.c_int, [_vp, ctypes.c_uint64, ctypes.c_char_p, ctypes.c_size_t,
                                            ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint64),
                                            ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint64),
                                            ctypes.POINTER(ctypes.c_uint64)]),
    "mlq_hip_gguf_find": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]),
    "mlq_hip_gguf_tensor_data": (ctypes.c_int, [_vp, ctypes.c_uint64, ctypes.POINTER(_vp),
                                                 ctypes.POINTER(ctypes.c_uint64)]),
    "mlq_hip_gguf_upload_weight": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(_vp)]),
    "mlq_hip_decoder_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_vp)]),
    "mlq_hip_decoder_config": (ctypes.c_int, [_vp, ctypes.POINTER(DecoderConfig)]),
    "mlq_hip_decoder_forward": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, _vp]),
    "mlq_hip_decoder_generate": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.c_int, _vp]),
    "mlq_hip_decoder_prefill": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.c_int, _vp]),
    "mlq_hip_decoder_close": (ctypes.c_int, [_vp]),
    "mlq_hip_graph_begin": (ctypes.c_int, [ctypes.c_int, _vp]),
    "mlq_hip_graph_end": (ctypes.c_int, [ctypes.c_int, _vp, ctypes.POINTER(_vp)]),
    "mlq_hip_sequence_create": (ctypes.c_int, [ctypes.POINTER(LinearCall), ctypes.c_int,
                                                ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.POINTER(_vp)]),
    "mlq_hip_sequence_launch": (ctypes.c_int, [_vp, _vp]),
    "mlq_hip_sequence_status": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_int)]),
    "mlq_hip_sequence_set_spin_limit": (ctypes.c_int, [_vp, ctypes.c_uint]),
    "mlq_hip_sequence_info": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int),
                                              ctypes.POINTER(ctypes.c_int)]),
    "mlq_hip_sequence_destroy": (ctypes.c_int, [_vp]),
    "mlq_hip_graph_capture_sequence": (ctypes.c_int, [_vp, _vp, ctypes.POINTER(_vp)]),
    "mlq_hip_fill_normal": (ctypes.c_int, [_vp, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_float,
                                            ctypes.c_float, _vp]),
    "mlq_hip_rmsnorm": (ctypes.c_int, [ctypes.c_int, _vp, _vp, ctypes.c_int, ctypes.c_float, _vp, _vp]),
    "mlq_hip_silu": (ctypes.c_int, [ctypes.c_int, _vp, ctypes.c_size_t, _vp, _vp]),
    "mlq_hip_mul": (ctypes.c_int, [ctypes.c_int, _vp, _vp, ctypes.c_size_t, _vp, _vp]),
    "mlq_hip_add": (ctypes.c_int, [ctypes.c_int, _vp, _vp, ctypes.c_size_t, _vp, _vp]),
    "mlq_hip_softmax": (ctypes.c_int, [ctypes.c_int, _vp, ctypes.c_int, _vp, _vp]),
    "mlq_hip_embedding": (ctypes.c_int, [ctypes.c_int, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, _vp]),
    "mlq_hip_rope": (ctypes.c_int, [ctypes.c_int, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                     ctypes.c_int, _vp]),
    "mlq_hip_attention_decode": (ctypes.c_int, [ctypes.c_int, _vp, _vp, _vp] + [ctypes.c_int] * 7 + [_vp, _vp]),
    "mlq_hip_matmul_f32": (ctypes.c_int, [ctypes.c_int, _vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, _vp, _vp]),
    "mlq_hip_kernel_name": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_char_p, ctypes.c_size_t]),
}

EXPORTED = tuple(_SIGS)


def load(path: str = LIB_PATH):
    """Load the HIP library (raises if it is not built: there is no fallback)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is missing: build it with `make -C mini-llama-cpp-release_amd` "
            "(there is no CPU fallback for the HIP path)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGS.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    _LIB = lib
    return lib


def _check(rc: int) -> None:
    if rc != 0:
        raise MlqError(rc, _LIB.mlq_hip_last_error().decode(errors="surrogateescape"))


def last_error() -> str:
    return load().mlq_hip_last_error().decode(errors="surrogateescape")


def device_count() -> int:
    n = ctypes.c_int(0)
    _check(load().mlq_hip_device_count(ctypes.byref(n)))
    return n.value


def device_info(device: int = 0) -> str:
    buf = ctypes.create_string_buffer(256)
    _check(load().mlq_hip_device_info(device, buf, 256))
    return buf.value.decode()


def device_props(device: int = 0) -> dict:
    p = DeviceProps()
    _check(load().mlq_hip_device_props(device, ctypes.byref(p)))
    return {"name": p.name.decode(), "arch": p.arch.decode(), "major": p.major, "minor": p.minor,
            "total_memory_bytes": p.total_memory_bytes, "compute_units": p.compute_units,
            "driver_version": p.driver_version, "runtime_version": p.runtime_version}


def init(device: int = 0) -> None:
    _check(load().mlq_hip_init(device))


def kernel_name(qtype: int, rows: int, m: int, k: int) -> str:
    buf = ctypes.create_string_buffer(128)
    _check(load().mlq_hip_kernel_name(qtype, rows, m, k, buf, 128))
    return buf.value.decode()


class DeviceBuffer:
    """Owned device allocation (hipMalloc through the C ABI)."""

    def __init__(self, nbytes: int, device: int = 0):
        lib = load()
        p = _vp()
        _check(lib.mlq_hip_malloc(device, max(int(nbytes), 1), ctypes.byref(p)))
        self.ptr = p.value
        self.nbytes = int(nbytes)
        self.device = device

    @classmethod
    def from_array(cls, a: np.ndarray, device: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes, device)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        _check(_LIB.mlq_hip_memcpy_htod(self.ptr + offset, a.ctypes.data, a.nbytes))

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        _check(_LIB.mlq_hip_memcpy_dtoh(out.ctypes.data, self.ptr + offset, out.nbytes))
        return out

    def fill(self, value: int = 0) -> None:
        _check(_LIB.mlq_hip_memset(self.ptr, value, self.nbytes))

    def free(self) -> None:
        if getattr(self, "ptr", None):
            _LIB.mlq_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Weight:
    """A quantized [M, K] weight resident on the device (mlq_weight_t)."""

    def __init__(self, handle: int, qtype: int, m: int, k: int, keep=None):
        self.h = handle
        self.qtype, self.m, self.k = qtype, m, k
        self.nb = (k + QK - 1) // QK
        self._keep = keep  # a wrapped DeviceBuffer must outlive the handle

    @classmethod
    def upload(cls, qtype: int, blocks: np.ndarray, m: int, k: int, device: int = 0) -> "Weight":
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        h = _vp()
        _check(load().mlq_hip_upload_weight(device, qtype, blocks.ctypes.data, blocks.shape[0], m, k,
                                            ctypes.byref(h)))
        return cls(h.value, qtype, m, k)

    @classmethod
    def wrap(cls, qtype: int, buf: DeviceBuffer, n_blocks: int, m: int, k: int, device: int = 0) -> "Weight":
        h = _vp()
        _check(load().mlq_hip_wrap_weight(device, qtype, buf.ptr, n_blocks, m, k, ctypes.byref(h)))
        return cls(h.value, qtype, m, k, keep=buf)

    def linear_host(self, x: np.ndarray) -> np.ndarray:
        """y = x W^T with host x / y (the *_device_weight form)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows = x.size // self.k
        y = np.empty(x.shape[:-1] + (self.m,), dtype=np.float32)
        _check(_LIB.mlq_hip_quant_linear(self.h, x.ctypes.data, rows, y.ctypes.data, 0, None))
        return y

    def linear_device(self, x: DeviceBuffer, y: DeviceBuffer, rows: int = 1, stream=None,
                      sync: bool = True) -> None:
        flags = X_ON_DEVICE | Y_ON_DEVICE | (0 if sync else ASYNC)
        _check(_LIB.mlq_hip_quant_linear(self.h, x.ptr, rows, y.ptr, flags, stream))

    def linear_noalloc(self, x: DeviceBuffer, y: DeviceBuffer, rows: int = 1, stream=None) -> None:
        """mlq_hip_quant_linear_noalloc: device x / y, asynchronous on `stream`,
        the library's fixed scratch instead of an allocated workspace."""
        _check(_LIB.mlq_hip_quant_linear_noalloc(self.h, x.ptr, rows, y.ptr, stream))

    def linear_argmax(self, x: DeviceBuffer, y: "DeviceBuffer | None", token: DeviceBuffer,
                      stream=None) -> None:
        """y = W x (skipped when y is None) and token[0] = first argmax of y, or -1
        when a logit is not finite; asynchronous (mlq_hip_quant_linear_argmax)."""
        _check(_LIB.mlq_hip_quant_linear_argmax(self.h, x.ptr, None if y is None else y.ptr, token.ptr, stream))

    def sample_greedy(self, x: DeviceBuffer, y: "DeviceBuffer | None" = None, stream=None) -> int:
        """Greedy token of the logits W x, returned to the host (mlq_hip_sample_greedy);
        raises MlqError("sampler: logits must be finite") like the reference sampler."""
        t = ctypes.c_int(-1)
        _check(_LIB.mlq_hip_sample_greedy(self.h, x.ptr, None if y is None else y.ptr, ctypes.byref(t), stream))
        return t.value

    def free(self) -> None:
        if getattr(self, "h", None):
            _LIB.mlq_hip_free_weight(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def quantize_device(qtype: int, src: DeviceBuffer, rows: int, row_len: int, dst: DeviceBuffer,
                    device: int = 0, stream=None) -> None:
    assert src.nbytes >= 4 * rows * row_len, "source buffer too small"
    assert dst.nbytes >= rows * ((row_len + QK - 1) // QK) * BLOCK_BYTES[qtype], "block buffer too small"
    _check(load().mlq_hip_quantize(device, qtype, src.ptr, rows, row_len, dst.ptr, stream))


def fill_normal(buf: DeviceBuffer, n: int, seed: int, mean: float = 0.0, std: float = 1.0,
                stream=None) -> None:
    assert buf.nbytes >= 4 * n, "destination buffer too small"
    _check(load().mlq_hip_fill_normal(buf.ptr, n, seed & (2 ** 64 - 1), mean, std, stream))


def linear_device_raw(qtype: int, w: DeviceBuffer, n_blocks: int, m: int, k: int, x: DeviceBuffer,
                      rows: int, y: DeviceBuffer, device: int = 0, stream=None) -> None:
    _check(load().mlq_hip_quant_linear_device(device, qtype, w.ptr, n_blocks, m, k, x.ptr, rows, y.ptr,
                                              stream))


def make_calls(calls) -> ctypes.Array:
    """calls: iterable of (Weight, x DeviceBuffer/ptr, y DeviceBuffer/ptr, rows)."""
    calls = list(calls)
    arr = (LinearCall * len(calls))()
    for i, (w, x, y, rows) in enumerate(calls):
        arr[i].w = w.h
        arr[i].x = x if isinstance(x, int) else x.ptr
        arr[i].y = y if isinstance(y, int) else y.ptr
        arr[i].rows = rows
    return arr


def linear_many(arr: ctypes.Array, stream=None) -> None:
    _check(load().mlq_hip_quant_linear_many(arr, len(arr), stream))


def stream_floor(arr: ctypes.Array, sink: "DeviceBuffer", stream=None) -> None:
    """mlq_hip_stream_floor: the weight stream of a fused launch of `arr`,
    without the arithmetic (a measurement of the per-launch floor)."""
    _check(load().mlq_hip_stream_floor(arr, len(arr), sink.ptr, stream))


PROBE_EMPTY, PROBE_LOAD = 1, 2


def stream_probe(arr: ctypes.Array, mode: int, sink: "DeviceBuffer", stream=None) -> None:
    """mlq_hip_stream_probe: the floor's grid with no work (PROBE_EMPTY) or
    the same weight bytes read with plain coalesced loads (PROBE_LOAD)."""
    _check(load().mlq_hip_stream_probe(arr, len(arr), mode, sink.ptr, stream))


STAMPS_LIB_PATH = os.path.join(HERE, "libmlq_hip_stamps.so")
RING_STAMP_SHAPE = (3, 256, 24)  # workgroups, stages, slots (include/mlq_hip.h)


def ring_stamps():
    """mlq_hip_ring_stamps: the last LDS-ring launch's boundary timestamps
    (s_memrealtime, 100 MHz) as a uint64 array of RING_STAMP_SHAPE; needs the
    measurement build (STAMPS_LIB_PATH, `make stamps`) loaded."""
    import numpy as np
    out = np.zeros(RING_STAMP_SHAPE, np.uint64)
    _check(load().mlq_hip_ring_stamps(out.ctypes.data, out.size))
    return out


def linear_fused_f32(arr: ctypes.Array, stream=None) -> None:
    """mlq_hip_quant_linear_fused_f32: the fused decode launch with the
    reference's f32 arithmetic (dequantized weights, f32 multiply-adds)."""
    _check(load().mlq_hip_quant_linear_fused_f32(arr, len(arr), stream))


def linear_fused(arr: ctypes.Array, stream=None) -> None:
    """One launch for up to 4 linears that share x: GEMVs (rows 1) or a grouped
    GEMM (rows > 1); asynchronous on `stream`."""
    _check(load().mlq_hip_quant_linear_fused(arr, len(arr), stream))


class Sequence:
    """A chain of GEMV calls run as persistent launches (mlq_hip_sequence_*).

    ``stages`` gives one stage id per call (consecutive equal ids form a stage of
    calls that share x); None puts every call in a stage of its own."""

    def __init__(self, arr: ctypes.Array, stages=None, mode: int = SEQ_PERSISTENT):
        h = _vp()
        ids = None
        if stages is not None:
            assert len(stages) == len(arr), "one stage id per call"
            ids = (ctypes.c_int * len(stages))(*stages)
        _check(load().mlq_hip_sequence_create(arr, len(arr), ids, mode, ctypes.byref(h)))
        self.h = h.value
        self._keep = (arr, ids)

    def launch(self, stream=None) -> None:
        _check(_LIB.mlq_hip_sequence_launch(self.h, stream))

    def status(self) -> int:
        n = ctypes.c_int(0)
        _check(_LIB.mlq_hip_sequence_status(self.h, ctypes.byref(n)))
        return n.value

    def set_spin_limit(self, polls: int) -> None:
        _check(_LIB.mlq_hip_sequence_set_spin_limit(self.h, polls))

    def info(self) -> dict:
        st, ln, gr = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(0)
        _check(_LIB.mlq_hip_sequence_info(self.h, ctypes.byref(st), ctypes.byref(ln), ctypes.byref(gr)))
        return {"stages": st.value, "launches": ln.value, "grid": gr.value}

    def destroy(self) -> None:
        if getattr(self, "h", None):
            _LIB.mlq_hip_sequence_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Graph:
    """A captured and instantiated graph of ``linear_many(arr)`` or of one
    sequence launch (``Graph(sequence=seq)``; the sequence must outlive it)."""

    def __init__(self, arr: ctypes.Array | None = None, stream=None, sequence: "Sequence | None" = None):
        h = _vp()
        if sequence is not None:
            _check(load().mlq_hip_graph_capture_sequence(sequence.h, stream, ctypes.byref(h)))
        else:
            _check(load().mlq_hip_graph_capture_many(arr, len(arr), stream, ctypes.byref(h)))
        self.h = h.value
        self._arr = arr
        self._seq = sequence

    @classmethod
    def record(cls, fn, stream=None, device: int = 0, keep=None) -> "Graph":
        """Capture whatever ``fn()`` launches asynchronously on ``stream``
        (mlq_hip_graph_begin / mlq_hip_graph_end); ``keep`` holds objects the
        graph's launches use."""
        lib = load()
        _check(lib.mlq_hip_graph_begin(device, stream))
        h = _vp()
        try:
            fn()
        except BaseException:
            if lib.mlq_hip_graph_end(device, stream, ctypes.byref(h)) == 0 and h.value:
                lib.mlq_hip_graph_destroy(h.value)
            raise
        _check(lib.mlq_hip_graph_end(device, stream, ctypes.byref(h)))
        g = cls.__new__(cls)
        g.h, g._arr, g._seq = h.value, keep, None
        return g

    def launch(self, stream=None) -> None:
        _check(_LIB.mlq_hip_graph_launch(self.h, stream))

    def destroy(self) -> None:
        if getattr(self, "h", None):
            _LIB.mlq_hip_graph_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


GGML_QTYPE = {8: Q8_0, 2: Q4_0, 3: Q4_1}  # GGML tensor type -> quant type


class GgufFile:
    """A GGUF model file mapped read-only and indexed (mlq_hip_gguf_*).  Needs
    no GPU except for upload_weight."""

    def __init__(self, path: str):
        h = _vp()
        _check(load().mlq_hip_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self.h = h.value

    def header(self) -> dict:
        v, nt, nm, off = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        _check(_LIB.mlq_hip_gguf_header(self.h, ctypes.byref(v), ctypes.byref(nt), ctypes.byref(nm),
                                        ctypes.byref(off)))
        return {"version": v.value, "n_tensors": nt.value, "n_metadata": nm.value, "data_offset": off.value}

    def metadata(self) -> list:
        """[(key, value type, value as the reference renders it)]"""
        out = []
        for i in range(self.header()["n_metadata"]):
            for cap in (1 << 16, (16 << 20) + 64):
                key, val, t = ctypes.create_string_buffer(cap), ctypes.create_string_buffer(cap), ctypes.c_uint32()
                rc = _LIB.mlq_hip_gguf_metadata(self.h, i, key, cap, ctypes.byref(t), val, cap)
                if rc != 6:  # MLQ_ERR_LIMIT: retry with the largest size a value can have
                    break
            _check(rc)
            out.append((key.value.decode(errors="surrogateescape"), t.value,
                        val.value.decode(errors="surrogateescape")))
        return out

    def tensors(self) -> list:
        out = []
        for i in range(self.header()["n_tensors"]):
            nd, t, off, nb = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64()
            dims = (ctypes.c_uint64 * 8)()
            for cap in (1 << 12, (16 << 20) + 64):
                name = ctypes.create_string_buffer(cap)
                rc = _LIB.mlq_hip_gguf_tensor(self.h, i, name, cap, ctypes.byref(nd), dims, ctypes.byref(t),
                                              ctypes.byref(off), ctypes.byref(nb))
                if rc != 6:  # MLQ_ERR_LIMIT: retry with the largest size a name can have
                    break
            _check(rc)
            out.append({"name": name.value.decode(errors="surrogateescape"),
                        "dims": [dims[d] for d in range(nd.value)],
                        "type": t.value, "offset": off.value, "nbytes": nb.value})
        return out

    def find(self, name: str) -> int:
        i = ctypes.c_uint64()
        _check(_LIB.mlq_hip_gguf_find(self.h, name.encode(), ctypes.byref(i)))
        return i.value

    def tensor_bytes(self, name: str) -> np.ndarray:
        """A copy of the tensor's bytes read from the mapping."""
        p, n = _vp(), ctypes.c_uint64()
        _check(_LIB.mlq_hip_gguf_tensor_data(self.h, self.find(name), ctypes.byref(p), ctypes.byref(n)))
        if not n.value:
            return np.zeros(0, np.uint8)
        return np.frombuffer(ctypes.string_at(p.value, n.value), dtype=np.uint8).copy()

    def upload_weight(self, name: str, device: int = 0) -> "Weight":
        info = self.tensors()[self.find(name)]
        h = _vp()
        _check(_LIB.mlq_hip_gguf_upload_weight(self.h, name.encode(), device, ctypes.byref(h)))
        return Weight(h.value, GGML_QTYPE[info["type"]], int(info["dims"][1]), int(info["dims"][0]))

    def close(self) -> None:
        if getattr(self, "h", None):
            _LIB.mlq_hip_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Decoder:
    """A GGUF model decoding on the device (mlq_hip_decoder_*)."""

    def __init__(self, path: str, device: int = 0, max_seq_len: int = 0):
        h = _vp()
        _check(load().mlq_hip_decoder_open(os.fsencode(path), device, max_seq_len, ctypes.byref(h)))
        self.h = h.value
        c = DecoderConfig()
        _check(_LIB.mlq_hip_decoder_config(self.h, ctypes.byref(c)))
        self.config = {n: getattr(c, n) for n, _ in DecoderConfig._fields_}

    def forward(self, token: int, pos: int) -> np.ndarray:
        logits = np.empty(self.config["vocab_size"], np.float32)
        _check(_LIB.mlq_hip_decoder_forward(self.h, token, pos, logits.ctypes.data))
        return logits

    def prefill(self, tokens, start: int = 0) -> np.ndarray:
        """Batched forward_batch; logits of the last token."""
        t = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty(self.config["vocab_size"], np.float32)
        _check(_LIB.mlq_hip_decoder_prefill(self.h, t.ctypes.data, t.size, start, logits.ctypes.data))
        return logits

    def generate(self, prompt, n_new: int) -> list:
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(n_new, 1), np.int32)
        _check(_LIB.mlq_hip_decoder_generate(self.h, p.ctypes.data, p.size, n_new, out.ctypes.data))
        return out[:n_new].tolist()

    def close(self) -> None:
        if getattr(self, "h", None):
            _LIB.mlq_hip_decoder_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def stream(device: int = 0) -> int:
    s = _vp()
    _check(load().mlq_hip_stream(device, ctypes.byref(s)))
    return s.value


def stream_create(device: int = 0) -> int:
    """A new stream on ``device`` (release it with stream_destroy)."""
    s = _vp()
    _check(load().mlq_hip_stream_create(device, ctypes.byref(s)))
    return s.value


def stream_destroy(stream: int) -> None:
    _check(load().mlq_hip_stream_destroy(stream))


def synchronize(stream=None) -> None:
    _check(load().mlq_hip_synchronize(stream))


class Event:
    def __init__(self):
        e = _vp()
        _check(load().mlq_hip_event_create(ctypes.byref(e)))
        self.h = e.value

    def record(self, stream=None) -> None:
        _check(_LIB.mlq_hip_event_record(self.h, stream))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0)
        _check(_LIB.mlq_hip_event_elapsed_ms(self.h, end.h, ctypes.byref(ms)))
        return float(ms.value)

    def __del__(self):
        try:
            if getattr(self, "h", None):
                _LIB.mlq_hip_event_destroy(self.h)
                self.h = None
        except Exception:
            pass

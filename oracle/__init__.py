"""mlq CPU oracle -- TEST INFRASTRUCTURE ONLY.

ctypes bindings for the C++ restatement of mini-llama.cpp's CPU quant path
(``oracle/oracle.cpp`` -> ``_build/libmlq_oracle.so``) and, where it was built,
for the reference's own CPU sources (``ref_shim.cpp`` -> ``_ref/libmlq_ref.so``).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
import this package, and only as the checker or the timed CPU baseline.  The
product library (``mini-llama-cpp-release_amd``) never imports or links it.

Blocks are handled as raw ``uint8`` arrays of shape ``(n_blocks, block_bytes)``
in the ggml byte layout (34 / 18 / 20 bytes per 32 elements).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "libmlq_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libmlq_ref.so")

F32, Q8_0, Q4_0, Q4_1 = 0, 1, 2, 3
QTYPES = {"q8_0": Q8_0, "q4_0": Q4_0, "q4_1": Q4_1}
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18, Q4_1: 20}
QK = 32

_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)


def build(reference: str | None = None) -> None:
    """Compile the oracle (and the reference shim when ``reference`` exists)."""
    subprocess.run(["make", "-s", "-C", HERE, "oracle"], check=True)
    if reference and os.path.isdir(os.path.join(reference, "src")):
        subprocess.run(["make", "-s", "-C", HERE, "-j8", "ref", f"REF={reference}"], check=True)


def _ptr(a: np.ndarray, ctype=ctypes.c_void_p):
    return a.ctypes.data_as(ctype) if ctype is not ctypes.c_void_p else ctypes.c_void_p(a.ctypes.data)


def n_blocks(rows: int, k: int) -> int:
    return rows * ((k + QK - 1) // QK)


class _Lib:
    """Common numpy-facing wrapper over either shared library."""

    prefix = ""

    def __init__(self, path: str):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (run oracle.build())")
        self.path = path
        self.lib = ctypes.CDLL(path)

    def _fn(self, name, restype, argtypes):
        f = getattr(self.lib, self.prefix + name)
        f.restype = restype
        f.argtypes = argtypes
        return f


class Oracle(_Lib):
    """The restated CPU path (``oracle.cpp``)."""

    prefix = "mlq_oracle_"

    def __init__(self, path: str = ORACLE_SO):
        super().__init__(path)
        self._enc = self._fn("fp16_from_f32_n", None, [_f32p, ctypes.c_size_t, _u16p])
        self._dec = self._fn("f32_from_fp16_n", None, [_u16p, ctypes.c_size_t, _f32p])
        self._quant = self._fn("quantize", ctypes.c_longlong,
                               [ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int])
        self._deq = self._fn("dequantize", ctypes.c_int,
                             [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _f32p])
        self._lin = self._fn("linear", ctypes.c_int,
                             [ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                              ctypes.c_size_t, ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_char_p,
                              ctypes.c_size_t])
        self._argmax = self._fn("argmax", ctypes.c_int, [_f32p, ctypes.c_size_t])
        self._hw = self._fn("hardware_threads", ctypes.c_int, [])

    def hardware_threads(self) -> int:
        return int(self._hw())

    def fp16_encode(self, v) -> np.ndarray:
        v = np.ascontiguousarray(v, dtype=np.float32).ravel()
        out = np.empty(v.size, dtype=np.uint16)
        self._enc(_ptr(v, _f32p), v.size, _ptr(out, _u16p))
        return out

    def fp16_decode(self, h) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
        out = np.empty(h.size, dtype=np.float32)
        self._dec(_ptr(h, _u16p), h.size, _ptr(out, _f32p))
        return out

    def quantize(self, qtype: int, w: np.ndarray, threads: int = 1) -> np.ndarray:
        """Quantize a [rows, K] (or [K]) f32 array; rows are the output features."""
        w = np.ascontiguousarray(w, dtype=np.float32)
        k = w.shape[-1]
        rows = w.size // k
        out = np.empty((n_blocks(rows, k), BLOCK_BYTES[qtype]), dtype=np.uint8)
        n = self._quant(qtype, _ptr(w, _f32p), rows, k, _ptr(out), threads)
        if n != out.shape[0]:
            raise ValueError(f"quantize failed ({n})")
        return out

    def dequantize(self, qtype: int, blocks: np.ndarray, rows: int, k: int) -> np.ndarray:
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        out = np.empty((rows, k), dtype=np.float32)
        if self._deq(qtype, _ptr(blocks), rows, k, _ptr(out, _f32p)) != 0:
            raise ValueError("dequantize failed")
        return out

    def linear(self, qtype: int, x: np.ndarray, blocks: np.ndarray, m: int, threads: int = 1) -> np.ndarray:
        """y = x @ W^T with W given as blocks of an [m, K] matrix; x is [K] or [rows, K]."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        k = x.shape[-1]
        rows = x.size // k
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        y = np.empty(x.shape[:-1] + (m,), dtype=np.float32)
        err = ctypes.create_string_buffer(512)
        rc = self._lin(qtype, _ptr(x, _f32p), rows, k, _ptr(blocks), blocks.shape[0], m,
                       _ptr(y, _f32p), threads, err, 512)
        if rc != 0:
            raise RuntimeError(err.value.decode())
        return y

    def argmax(self, v: np.ndarray) -> int:
        v = np.ascontiguousarray(v, dtype=np.float32).ravel()
        return int(self._argmax(_ptr(v, _f32p), v.size))


class Reference(_Lib):
    """The reference's own CPU sources behind ``ref_shim.cpp`` (built only where
    /root/reference exists; the .so travels with the tree)."""

    prefix = "mlq_ref_"

    def __init__(self, path: str = REF_SO):
        super().__init__(path)
        self._p41 = self._fn("fp16_probe_q4_1", ctypes.c_uint16, [ctypes.c_float])
        self._p8 = self._fn("fp16_probe_q8_0", ctypes.c_uint16, [ctypes.c_float])
        self._quant = self._fn("quantize", ctypes.c_longlong,
                               [ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p])
        self._deq = self._fn("dequantize", ctypes.c_int,
                             [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _f32p])
        self._lin = self._fn("linear", ctypes.c_int,
                             [ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                              ctypes.c_size_t, ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_char_p,
                              ctypes.c_size_t])
        self._wnew = self._fn("weight_new", ctypes.c_void_p,
                              [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int])
        self._wfree = self._fn("weight_free", None, [ctypes.c_void_p])
        self._wlin = self._fn("weight_linear", ctypes.c_int,
                              [ctypes.c_void_p, _f32p, ctypes.c_int, _f32p, ctypes.c_int])
        self._argmax = self._fn("argmax", ctypes.c_int, [_f32p, ctypes.c_int])
        self._hw = self._fn("hardware_threads", ctypes.c_int, [])

    def hardware_threads(self) -> int:
        return int(self._hw())

    # ---- GGUF (src/gguf.cpp, src/gguf_loader.cpp)
    def gguf(self, path: str) -> dict:
        """GGUFReader::load on ``path``: ok, load_error, the header fields and,
        as far as they were read, the metadata and tensor infos."""
        cp, vp, u32, u64 = ctypes.c_char_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64
        load = self._fn("gguf_load", vp, [cp, ctypes.POINTER(ctypes.c_int)])
        free = self._fn("gguf_free", None, [vp])
        err = self._fn("gguf_error", cp, [vp])
        hdr = self._fn("gguf_header", None, [vp] + [ctypes.POINTER(u32)] + [ctypes.POINTER(u64)] * 5)
        meta = self._fn("gguf_metadata", None, [vp, u64, ctypes.POINTER(cp), ctypes.POINTER(u32),
                                                 ctypes.POINTER(vp), ctypes.POINTER(u64)])
        ten = self._fn("gguf_tensor", None, [vp, u64, ctypes.POINTER(cp), ctypes.POINTER(u32),
                                              ctypes.POINTER(u64), ctypes.POINTER(u32), ctypes.POINTER(u64),
                                              ctypes.POINTER(u64)])
        ok = ctypes.c_int(0)
        h = load(os.fsencode(path), ctypes.byref(ok))
        try:
            v, nt, nm, off, nmr, ntr = u32(), u64(), u64(), u64(), u64(), u64()
            hdr(h, ctypes.byref(v), ctypes.byref(nt), ctypes.byref(nm), ctypes.byref(off), ctypes.byref(nmr),
                ctypes.byref(ntr))
            out = {"ok": bool(ok.value), "error": err(h).decode(errors="surrogateescape"), "version": v.value,
                   "n_tensors": nt.value,
                   "n_metadata": nm.value, "data_offset": off.value, "metadata": [], "tensors": []}
            for i in range(nmr.value):
                k, t, val, n = cp(), u32(), vp(), u64()
                meta(h, i, ctypes.byref(k), ctypes.byref(t), ctypes.byref(val), ctypes.byref(n))
                # Up to the first NUL, as a C string carries it.
                raw = ctypes.string_at(val.value, n.value).split(b"\0")[0] if n.value else b""
                out["metadata"].append((k.value.decode(errors="surrogateescape"), t.value,
                                        raw.decode(errors="surrogateescape")))
            for i in range(ntr.value):
                nme, nd, t, o, nb = cp(), u32(), u32(), u64(), u64()
                dims = (u64 * 8)()
                ten(h, i, ctypes.byref(nme), ctypes.byref(nd), dims, ctypes.byref(t), ctypes.byref(o),
                    ctypes.byref(nb))
                out["tensors"].append({"name": nme.value.decode(errors="surrogateescape"),
                                       "dims": [dims[d] for d in range(nd.value)],
                                       "type": t.value, "offset": o.value, "nbytes": nb.value})
            return out
        finally:
            free(h)

    def gguf_tensor_raw(self, path: str, index: int) -> np.ndarray:
        """read_gguf_tensor_raw for tensor ``index`` (empty where it fails)."""
        vp, u64 = ctypes.c_void_p, ctypes.c_uint64
        load = self._fn("gguf_load", vp, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_int)])
        free = self._fn("gguf_free", None, [vp])
        read = self._fn("gguf_read", ctypes.c_longlong, [ctypes.c_char_p, vp, u64, vp, u64])
        ok = ctypes.c_int(0)
        h = load(os.fsencode(path), ctypes.byref(ok))
        try:
            cap = os.path.getsize(path)
            buf = np.empty(max(cap, 1), np.uint8)
            n = read(os.fsencode(path), h, index, _ptr(buf), cap)
            return buf[:max(n, 0)].copy()
        finally:
            free(h)

    def type_names(self, t: int) -> tuple:
        ggml = self._fn("ggml_type_name", ctypes.c_char_p, [ctypes.c_uint32])
        val = self._fn("gguf_value_type_name", ctypes.c_char_p, [ctypes.c_uint32])
        return ggml(t).decode(), val(t).decode()

    def gguf_model_linears(self, path: str, names) -> dict:
        """load_gguf_model, then {name: (quant type, rows, cols, block bytes)}
        for the reference-named linears ``names``; raises with load_error."""
        vp = ctypes.c_void_p
        load = self._fn("gguf_model", vp, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_int)])
        free = self._fn("model_free", None, [vp])
        err = self._fn("model_error", ctypes.c_char_p, [vp])
        lin = self._fn("model_linear", ctypes.c_int,
                       [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int),
                        ctypes.POINTER(ctypes.c_int), ctypes.POINTER(vp), ctypes.POINTER(ctypes.c_uint64)])
        ok = ctypes.c_int(0)
        h = load(os.fsencode(path), ctypes.byref(ok))
        try:
            if not ok.value:
                raise RuntimeError(err(h).decode())
            out = {}
            for n in names:
                q, r, c, d, nb = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), vp(), ctypes.c_uint64()
                if lin(h, n.encode(), ctypes.byref(q), ctypes.byref(r), ctypes.byref(c), ctypes.byref(d),
                       ctypes.byref(nb)) != 0:
                    raise KeyError(n)
                out[n] = (q.value, r.value, c.value,
                          np.frombuffer(ctypes.string_at(d.value, nb.value), np.uint8).copy())
            return out
        finally:
            free(h)

    def decoder(self, path: str, threads: int = 0) -> "RefDecoder":
        return RefDecoder(self, path, threads)

    def fp16_probe_q4_1(self, v: float) -> int:
        return int(self._p41(float(v)))

    def fp16_probe_q8_0(self, v: float) -> int:
        return int(self._p8(float(v)))

    def quantize(self, qtype: int, w: np.ndarray) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.float32)
        k = w.shape[-1]
        rows = w.size // k
        out = np.empty((n_blocks(rows, k), BLOCK_BYTES[qtype]), dtype=np.uint8)
        n = self._quant(qtype, _ptr(w, _f32p), rows, k, _ptr(out))
        if n != out.shape[0]:
            raise ValueError(f"reference quantize failed ({n})")
        return out

    def dequantize(self, qtype: int, blocks: np.ndarray, rows: int, k: int) -> np.ndarray:
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        out = np.empty((rows, k), dtype=np.float32)
        if self._deq(qtype, _ptr(blocks), rows, k, _ptr(out, _f32p)) != 0:
            raise ValueError("reference dequantize failed")
        return out

    def linear(self, qtype: int, x: np.ndarray, blocks: np.ndarray, m: int, threads: int = 1) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        k = x.shape[-1]
        rows = x.size // k
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        y = np.empty(x.shape[:-1] + (m,), dtype=np.float32)
        err = ctypes.create_string_buffer(512)
        rc = self._lin(qtype, _ptr(x, _f32p), rows, k, _ptr(blocks), blocks.shape[0], m,
                       _ptr(y, _f32p), threads, err, 512)
        if rc != 0:
            raise RuntimeError(err.value.decode())
        return y

    def weight(self, qtype: int, blocks: np.ndarray, m: int, k: int) -> "RefWeight":
        return RefWeight(self, qtype, blocks, m, k)

    def argmax(self, v: np.ndarray) -> int:
        v = np.ascontiguousarray(v, dtype=np.float32).ravel()
        return int(self._argmax(_ptr(v, _f32p), v.size))


class RefWeight:
    """A reference QuantizedTensor built once, for timing repeated linear() calls."""

    def __init__(self, ref: Reference, qtype: int, blocks: np.ndarray, m: int, k: int):
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        self.ref, self.m, self.k = ref, m, k
        self.h = ref._wnew(qtype, _ptr(blocks), blocks.shape[0], m, k)
        if not self.h:
            raise ValueError("reference weight_new failed")

    def linear(self, x: np.ndarray, out: np.ndarray, threads: int) -> None:
        rows = x.size // self.k
        if self.ref._wlin(self.h, _ptr(x, _f32p), rows, _ptr(out, _f32p), threads) != 0:
            raise RuntimeError("reference linear failed")

    def __del__(self):
        if getattr(self, "h", None):
            self.ref._wfree(self.h)
            self.h = None


class RefDecoder:
    """load_gguf_model + forward_token of the reference (CPU, f32)."""

    def __init__(self, ref: Reference, path: str, threads: int = 0):
        vp, cp = ctypes.c_void_p, ctypes.c_char_p
        self._open = ref._fn("decoder_open", vp, [cp, ctypes.c_int, ctypes.POINTER(ctypes.c_int)])
        self._err = ref._fn("decoder_error", cp, [vp])
        self._free = ref._fn("decoder_free", None, [vp])
        self._cfg = ref._fn("decoder_config", None, [vp, ctypes.POINTER(ctypes.c_int)])
        self._fwd = ref._fn("decoder_forward", ctypes.c_int,
                            [vp, ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_char_p, ctypes.c_size_t])
        self._batch = ref._fn("decoder_batch", ctypes.c_int,
                              [vp, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_char_p,
                               ctypes.c_size_t])
        self._gen = ref._fn("decoder_generate", ctypes.c_int,
                            [vp, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_char_p,
                             ctypes.c_size_t])
        ok = ctypes.c_int(0)
        self.h = self._open(os.fsencode(path), threads, ctypes.byref(ok))
        if not ok.value:
            msg = self._err(self.h).decode()
            self._free(self.h)
            self.h = None
            raise RuntimeError(msg)
        c = (ctypes.c_int * 9)()
        self._cfg(self.h, c)
        self.config = dict(zip(("n_layers", "dim", "hidden_dim", "n_heads", "n_kv_heads", "head_dim", "vocab_size",
                                "max_seq_len", "rope_neox"), list(c)))

    def forward(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.config["vocab_size"], np.float32)
        err = ctypes.create_string_buffer(512)
        if self._fwd(self.h, token, pos, _ptr(out, _f32p), err, 512) != 0:
            raise RuntimeError(err.value.decode())
        return out

    def batch(self, tokens, start: int = 0) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(self.config["vocab_size"], np.float32)
        err = ctypes.create_string_buffer(512)
        if self._batch(self.h, _ptr(t), t.size, start, _ptr(out, _f32p), err, 512) != 0:
            raise RuntimeError(err.value.decode())
        return out

    def generate(self, prompt, n_new: int) -> list:
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(n_new, 1), np.int32)
        err = ctypes.create_string_buffer(512)
        if self._gen(self.h, _ptr(p), p.size, n_new, _ptr(out), err, 512) != 0:
            raise RuntimeError(err.value.decode())
        return out[:n_new].tolist()

    def __del__(self):
        if getattr(self, "h", None):
            self._free(self.h)
            self.h = None


_ORACLE: Oracle | None = None
_REF: Reference | None = None


def get() -> Oracle:
    global _ORACLE
    if _ORACLE is None:
        _ORACLE = Oracle()
    return _ORACLE


def reference() -> Reference | None:
    """The compiled reference shim, or None where it was not built."""
    global _REF
    if _REF is None and os.path.exists(REF_SO):
        _REF = Reference()
    return _REF

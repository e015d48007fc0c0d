"""A small GGUF v3 writer for the ingest tests (test infrastructure).

Layout (the published GGUF v3 format, as the reference reads it in
src/gguf.cpp:371-530): magic "GGUF", u32 version, u64 tensor count, u64
metadata count, the metadata (string key, u32 value type, value), the tensor
infos (string name, u32 n_dims, u64 dims with ne0 first, u32 GGML type, u64
offset into the data section), zero padding to general.alignment (default
32), then the data section.  Strings are u64 length + bytes; arrays are u32
element type + u64 count + elements.  Everything little-endian.
"""

from __future__ import annotations

import struct

import numpy as np

# GGUF value types and GGML tensor types (include/mini_llama/gguf.h:12-41).
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q4_1, GGML_Q8_0 = 0, 1, 2, 3, 8

_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
           U64: "<Q", I64: "<q", F64: "<d"}


def _str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value_bytes(vtype: int, value) -> bytes:
    if vtype == STRING:
        return _str(value)
    if vtype == ARRAY:
        elem, items = value
        return struct.pack("<IQ", elem, len(items)) + b"".join(value_bytes(elem, v) for v in items)
    return struct.pack(_SCALAR[vtype], value)


def build(metadata, tensors, alignment: int | None = None, version: int = 3) -> bytes:
    """metadata: [(key, vtype, value)]; tensors: [(name, dims ne0-first, ggml
    type, raw bytes)] placed in order, each at the next multiple of the
    alignment.  Returns the file bytes."""
    align = 32 if alignment is None else alignment
    meta = list(metadata)
    out = [b"GGUF", struct.pack("<IQQ", version, len(tensors), len(meta))]
    for key, vtype, value in meta:
        out.append(_str(key) + struct.pack("<I", vtype) + value_bytes(vtype, value))
    offsets, pos = [], 0
    for _, _, _, raw in tensors:
        pos = (pos + align - 1) // align * align
        offsets.append(pos)
        pos += len(raw)
    for (name, dims, gtype, _), off in zip(tensors, offsets):
        out.append(_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) +
                   struct.pack("<IQ", gtype, off))
    head = b"".join(out)
    data = bytearray()
    for (_, _, _, raw), off in zip(tensors, offsets):
        data += b"\0" * (off - len(data))
        data += bytes(raw)
    pad = (align - len(head) % align) % align
    return head + b"\0" * pad + bytes(data)


def write(path: str, metadata, tensors, alignment: int | None = None) -> None:
    meta = list(metadata)
    if alignment is not None and not any(k == "general.alignment" for k, _, _ in meta):
        meta.append(("general.alignment", U32, alignment))
    with open(path, "wb") as f:
        f.write(build(meta, tensors, alignment))


def linear_tensor(name: str, ggml_type: int, blocks: np.ndarray, rows: int, cols: int):
    """A [rows, cols] linear weight as GGUF stores it: dims (cols, rows)."""
    return (name, [cols, rows], ggml_type, np.ascontiguousarray(blocks, np.uint8).tobytes())


def f32_tensor(name: str, a: np.ndarray):
    a = np.ascontiguousarray(a, np.float32)
    dims = [a.shape[1], a.shape[0]] if a.ndim == 2 else list(a.shape)
    return (name, dims, GGML_F32, a.tobytes())


def write_stream(path: str, metadata, specs, produce, alignment: int = 32) -> None:
    """Writes a GGUF file tensor by tensor without holding it in memory:
    specs = [(name, dims ne0-first, ggml type, nbytes)], produce(i) returns
    tensor i's bytes (exactly nbytes)."""
    meta = list(metadata)
    if alignment != 32 and not any(k == "general.alignment" for k, _, _ in meta):
        meta.append(("general.alignment", U32, alignment))
    out = [b"GGUF", struct.pack("<IQQ", 3, len(specs), len(meta))]
    for key, vtype, value in meta:
        out.append(_str(key) + struct.pack("<I", vtype) + value_bytes(vtype, value))
    offsets, pos = [], 0
    for _, _, _, n in specs:
        pos = (pos + alignment - 1) // alignment * alignment
        offsets.append(pos)
        pos += n
    for (name, dims, gtype, _), off in zip(specs, offsets):
        out.append(_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) +
                   struct.pack("<IQ", gtype, off))
    head = b"".join(out)
    with open(path, "wb") as f:
        f.write(head + b"\0" * ((alignment - len(head) % alignment) % alignment))
        written = 0
        for i, ((_, _, _, n), off) in enumerate(zip(specs, offsets)):
            f.write(b"\0" * (off - written))
            raw = produce(i)
            assert len(raw) == n
            f.write(raw)
            written = off + n

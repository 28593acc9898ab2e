"""Writes GGUF files: header, metadata, tensor table, data section aligned
to 32 bytes or to ``general.alignment``.  Used to build model files from
tensors already in GGUF block layout (e.g. ``QTensor.to_numpy_bytes()``).

The layout follows the GGUF format: little-endian; strings are a uint64
length then the bytes; a metadata entry is key, uint32 value type, value
(arrays: uint32 element type, uint64 count, elements); a tensor entry is
name, uint32 n_dims, uint64 dims (dims[0] along the row), uint32 ggml type,
uint64 offset from the start of the data section.
"""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}
MAGIC = 0x46554747


def gstr(x: str) -> bytes:
    b = x.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def value_bytes(t: int, v) -> bytes:
    if t == STRING:
        return gstr(v)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += value_bytes(et, it)
        return out
    return struct.pack(_FMT[t], v)


def _head(kvs, tensors, version, alignment, offsets) -> tuple:
    """Header + metadata + tensor table, the data-section offset and each
    tensor's offset within the data section."""
    align = alignment or 32
    kvs = list(kvs) + ([("general.alignment", U32, alignment)] if alignment is not None else [])
    body = b"".join(gstr(k) + struct.pack("<I", t) + value_bytes(t, v) for k, t, v in kvs)
    offs, off = [], 0
    for _, _, _, data in tensors:
        offs.append(off)
        off = (off + len(data) + align - 1) // align * align
    if offsets is not None:
        offs = list(offsets)
    info = b"".join(gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
                    + struct.pack("<IQ", gt, o) for (name, dims, gt, _), o in zip(tensors, offs))
    meta = struct.pack("<IIQQ", MAGIC, version, len(tensors), len(kvs)) + body + info
    data_start = (len(meta) + align - 1) // align * align
    return meta, data_start, offs


def gguf_bytes(kvs, tensors, version: int = 3, alignment: int | None = None,
               offsets: list | None = None) -> tuple:
    """The file as bytes, the data-section offset and each tensor's offset.

    kvs: [(key, type, value)], arrays as (key, ARRAY, (elem_type, [items])).
    tensors: [(name, dims in GGUF order, ggml type, data bytes)].
    alignment: written as general.alignment (uint32) when given.
    version, offsets: the header version and explicit tensor offsets
    (default 3 and packed, each aligned); other values write files that a
    reader should reject, for tests of its error paths."""
    meta, data_start, offs = _head(kvs, tensors, version, alignment, offsets)
    buf = bytearray(meta) + bytearray(data_start - len(meta))
    for (_, _, _, data), o in zip(tensors, offs):
        end = data_start + o + len(data)
        if len(buf) < end:
            buf += bytearray(end - len(buf))
        buf[data_start + o: end] = data
    return bytes(buf), data_start, offs


def write_gguf(path, kvs, tensors, version: int = 3, alignment: int | None = None,
               offsets: list | None = None) -> tuple:
    """Writes the file of ``gguf_bytes`` to ``path``, streaming each
    tensor's data (bytes or any buffer) instead of building the file in
    memory.  Returns the data-section offset and the tensor offsets."""
    meta, data_start, offs = _head(kvs, tensors, version, alignment, offsets)
    end = data_start
    with open(path, "wb") as f:
        f.write(meta + bytes(data_start - len(meta)))
        for (_, _, _, data), o in zip(tensors, offs):
            f.seek(data_start + o)
            f.write(data)
            end = max(end, data_start + o + len(memoryview(data).cast("B")))
        f.truncate(end)
    return data_start, offs

"""Writes GGUF files (synthetic models for the loader tests and bench.py).

Layout (GC/loader/GGUFParser.java:17-105, GC/ = runner/gguf/gollek-gguf-core/
src/main/java/tech/kayys/gollek/gguf/): "GGUF", version i32, tensor count i64,
KV count i64; KV pairs (key string, type i32, value); tensor infos (name,
n_dims i32, dims i64..., type i32, offset i64); zero padding to the alignment;
tensor data.  Strings are an i64 byte length and UTF-8 bytes; all fields are
little-endian and unaligned.
"""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)

_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
        BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}


def string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<q", len(b)) + b


def value(kv_type: int, v) -> bytes:
    """Encoded value; an ARRAY value is (element type, list of elements)."""
    if kv_type == STRING:
        return string(v)
    if kv_type == ARRAY:
        et, items = v
        return struct.pack("<iq", et, len(items)) + b"".join(value(et, x) for x in items)
    return struct.pack(_FMT[kv_type], v)


def header(kvs, tensors, version: int = 3) -> bytes:
    """kvs: [(key, type, value)]; tensors: [(name, dims, type_id, offset)]."""
    out = [b"GGUF", struct.pack("<iqq", version, len(tensors), len(kvs))]
    for key, t, v in kvs:
        out += [string(key), struct.pack("<i", t), value(t, v)]
    for name, dims, type_id, offset in tensors:
        out += [string(name), struct.pack("<i", len(dims))]
        out += [struct.pack("<q", d) for d in dims]
        out.append(struct.pack("<iq", type_id, offset))
    return b"".join(out)


def padded(n: int, alignment: int) -> int:
    """Smallest multiple of `alignment` that is >= n."""
    return -(-n // alignment) * alignment


def gguf_file(kvs, named_blobs, alignment: int = 32, version: int = 3):
    """A file holding `named_blobs` [(name, dims, type_id, bytes)], each blob
    starting at a multiple of `alignment` from the data start.  Returns
    (file bytes, header length, data start, offsets)."""
    offsets, pos = [], 0
    for _, _, _, blob in named_blobs:
        pos = padded(pos, alignment)
        offsets.append(pos)
        pos += len(blob)
    h = header(kvs, [(n, d, t, off) for (n, d, t, _), off in zip(named_blobs, offsets)], version)
    start = padded(len(h), alignment)
    body = bytearray(pos)
    for (_, _, _, blob), off in zip(named_blobs, offsets):
        body[off:off + len(blob)] = blob
    return h + bytes(start - len(h)) + bytes(body), len(h), start, offsets

"""Synthetic GGUF v3 files for the loader tests (independent of the reader).

Layout per the GGUF v3 format: magic "GGUF", u32 version, u64 tensor count, u64
metadata count, metadata (u64-length key, u32 type, value), tensor infos
(u64-length name, u32 n_dims, u64 dims, u32 ggml type, u64 offset), padding to
the alignment, tensor data (each tensor's offset aligned within the section).
"""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}


def s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def value(t: int, v) -> bytes:
    if t == STR:
        return s(v)
    if t == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(value(et, it) for it in items)
    return struct.pack(_FMT[t], v)


def build(kvs, tensors, alignment=32, version=3, magic=b"GGUF"):
    """kvs: [(key, type, value)]; tensors: [(name, dims, ggml_type, data_bytes)].
    Returns (file bytes, data-section offset, per-tensor offsets)."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for k, t, v in kvs:
        head += s(k) + struct.pack("<I", t) + value(t, v)
    offs, data = [], b""
    for name, dims, gt, blob in tensors:
        data += b"\0" * ((-len(data)) % alignment)
        offs.append(len(data))
        data += blob
    for (name, dims, gt, blob), off in zip(tensors, offs):
        head += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", gt, off)
    data_off = len(head) + (-len(head)) % alignment
    return head + b"\0" * (data_off - len(head)) + data, data_off, offs

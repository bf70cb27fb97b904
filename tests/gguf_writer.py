"""Minimal GGUF writer for the tests (test infrastructure, not the product).

Writes the layout of reference include/gguf.h:8-56 / src/gguf.c:150-250:
u32 magic, u32 version, i64 n_tensors, i64 n_kv, the key/value pairs, the
tensor directory (name, n_dims, dims, ggml type, offset), padding to
`alignment`, then each tensor's bytes at its offset (each offset a multiple of
`alignment`, the convention of GGUF writers).
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<b",
        U64: "<Q", I64: "<q", F64: "<d"}


def _str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(ty, v) -> bytes:
    if ty == STR:
        return _str(v)
    if ty == ARR:
        ety, items = v
        out = struct.pack("<iQ", ety, len(items))
        return out + b"".join(_str(x) if ety == STR else struct.pack(_FMT[ety], x) for x in items)
    return struct.pack(_FMT[ty], v)


def header_bytes(kvs, tensors, version=3, n_tensors=None, n_kv=None, alignment=32):
    """kvs: [(key, type, value)]; tensors: [(name, dims, ggml_type, data_bytes)].
    Returns (header bytes, tensor offsets)."""
    out = bytearray(struct.pack("<IIqq", 0x46554747, version,
                                len(tensors) if n_tensors is None else n_tensors,
                                len(kvs) if n_kv is None else n_kv))
    for key, ty, v in kvs:
        out += _str(key) + struct.pack("<i", ty) + _value(ty, v)
    offs, off = [], 0
    for name, dims, gt, data in tensors:
        offs.append(off)
        out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<q", d) for d in dims)
        out += struct.pack("<iQ", gt, off)
        n = data.nbytes if isinstance(data, np.ndarray) else len(data)
        off += (n + alignment - 1) // alignment * alignment
    return bytes(out), offs


def write_gguf(path, kvs, tensors, version=3, alignment=32):
    """Write a GGUF file; returns (absolute data offset, per-tensor offsets)."""
    if alignment != 32 and not any(k == "general.alignment" for k, _, _ in kvs):
        kvs = list(kvs) + [("general.alignment", U32, alignment)]
    hdr, offs = header_bytes(kvs, tensors, version=version, alignment=alignment)
    data_off = (len(hdr) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(hdr)
        f.write(b"\0" * (data_off - len(hdr)))
        pos = 0
        for (_, _, _, data), o in zip(tensors, offs):
            f.write(b"\0" * (o - pos))
            b = np.ascontiguousarray(data).view(np.uint8).tobytes() if isinstance(data, np.ndarray) else data
            f.write(b)
            pos = o + len(b)
    return data_off, offs

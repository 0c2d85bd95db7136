"""Minimal GGUF v3 writer for tests (the published container layout): header,
metadata, tensor infos, data section at general.alignment. Test infrastructure only."""
from __future__ import annotations

import struct

import numpy as np

_SCALAR = {np.uint8: (0, "<B"), np.int8: (1, "<b"), np.uint16: (2, "<H"), np.int16: (3, "<h"),
           np.uint32: (4, "<I"), np.int32: (5, "<i"), np.float32: (6, "<f"),
           np.uint64: (10, "<Q"), np.int64: (11, "<q"), np.float64: (12, "<d")}


def _s(b: bytearray, text: str) -> None:
    raw = text.encode()
    b += struct.pack("<Q", len(raw)) + raw


def _value(b: bytearray, v) -> None:
    if isinstance(v, bool):
        b += struct.pack("<I?", 7, v)
    elif isinstance(v, str):
        b += struct.pack("<I", 8)
        _s(b, v)
    elif isinstance(v, np.ndarray):
        t, fmt = _SCALAR[v.dtype.type]
        b += struct.pack("<IIQ", 9, t, v.size) + np.ascontiguousarray(v).astype(fmt).tobytes()
    elif isinstance(v, list):  # list of strings
        b += struct.pack("<IIQ", 9, 8, len(v))
        for x in v:
            _s(b, x)
    elif isinstance(v, np.generic):
        t, fmt = _SCALAR[type(v)]
        b += struct.pack("<I", t) + struct.pack(fmt, v)
    elif isinstance(v, int):
        b += struct.pack("<Iq", 11, v)
    elif isinstance(v, float):
        b += struct.pack("<Id", 12, v)
    else:
        raise TypeError(type(v))


def write_gguf(path, metadata: dict, tensors: list, *, alignment: int = 32, version: int = 3):
    """tensors: [(name, ggml_type, shape in GGUF order, raw bytes)]."""
    meta = dict(metadata)
    if alignment != 32:
        meta["general.alignment"] = np.uint32(alignment)
    b = bytearray(b"GGUF")
    b += struct.pack("<IQQ", version, len(tensors), len(meta))
    for k, v in meta.items():
        _s(b, k)
        _value(b, v)
    offs, off = [], 0
    for _, _, _, raw in tensors:
        offs.append(off)
        off = (off + len(raw) + alignment - 1) // alignment * alignment
    for (name, ttype, shape, _), o in zip(tensors, offs):
        _s(b, name)
        b += struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        b += struct.pack("<IQ", ttype, o)
    b += b"\0" * ((-len(b)) % alignment)
    data = bytearray()
    for (_, _, _, raw), o in zip(tensors, offs):
        data += b"\0" * (o - len(data))
        data += bytes(raw)
    with open(path, "wb") as f:
        f.write(b + data)

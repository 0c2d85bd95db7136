"""GGUF reader feeding native k-quant bytes to the fused linears.

Replaces the reference's loader (superl8/gguf.py:106-235), which reads files
through llama.cpp's ``gguf`` Python package (a third-party dependency absent
here). This module parses the GGUF container itself, following the published
format (llama.cpp docs/gguf.md, version 2 and 3):

  header   : magic "GGUF", uint32 version, uint64 tensor_count, uint64 kv_count
  metadata : kv_count x (string key, uint32 value_type, value); strings are
             uint64 length + bytes; arrays are uint32 elem_type, uint64 n, values
  tensors  : tensor_count x (string name, uint32 n_dims, uint64 dims[n_dims]
             (dims[0] fastest), uint32 ggml_type, uint64 offset)
  data     : starts at the first multiple of general.alignment (default 32)
             after the tensor infos; each offset is relative to it.

The file is memory-mapped; a 2-D Q4_K / Q5_K / Q6_K weight whose input
dimension is a multiple of 256 becomes a ``gguf_kquant`` QTensor holding the
file's bytes unchanged ([out, (in/256) * type_size] uint8), which
``superl8_amd.ops.linear`` runs on the fused kernels. Other tensor types are
reported (type histogram) but not converted: the requantisation fallback of
the reference is outside this hot path.
"""
from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass, field

import numpy as np
import torch

from .format import GGUF_KQUANT_BLOCK, QK_K, QTensor

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32

# ggml_type ids and names (ggml.h enum ggml_type), with (block elements, block bytes)
# for the types whose byte size this reader needs.
GGML_TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20),
    6: ("Q5_0", 32, 22), 7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 36),
    10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144),
    13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210), 15: ("Q8_K", 256, 292),
    16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98),
    19: ("IQ1_S", 256, 50), 20: ("IQ4_NL", 32, 18), 21: ("IQ3_S", 256, 110),
    22: ("IQ2_S", 256, 82), 23: ("IQ4_XS", 256, 136), 24: ("I8", 1, 1), 25: ("I16", 1, 2),
    26: ("I32", 1, 4), 27: ("I64", 1, 8), 28: ("F64", 1, 8), 29: ("IQ1_M", 256, 56),
    30: ("BF16", 1, 2), 34: ("TQ1_0", 256, 54), 35: ("TQ2_0", 256, 66),
}
GGML_TYPE_ID = {v[0]: k for k, v in GGML_TYPES.items()}
# the native-fused types of this build (reference gguf.py:46-55, the subset with kernels here)
NATIVE_FUSED = {"Q4_K": "q4_k", "Q5_K": "q5_k", "Q6_K": "q6_k"}

# metadata value types
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?",
           10: "<Q", 11: "<q", 12: "<d"}
_STRING, _ARRAY = 8, 9


class GGUFError(ValueError):
    """A malformed or unsupported GGUF file."""


@dataclass
class GGUFTensorInfo:
    name: str
    shape: tuple          # GGUF order: shape[0] is the fastest-varying dimension
    ggml_type: int
    offset: int           # absolute byte offset in the file
    nbytes: int

    @property
    def type_name(self) -> str:
        return GGML_TYPES.get(self.ggml_type, (f"ggml_type_{self.ggml_type}",))[0]


@dataclass
class GGUFFile:
    """A parsed, memory-mapped GGUF file (close() or use as a context manager)."""
    path: str
    version: int
    metadata: dict = field(default_factory=dict)
    tensors: list = field(default_factory=list)
    alignment: int = DEFAULT_ALIGNMENT
    _mm: object = None
    _f: object = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def close(self) -> None:
        if self._mm is not None:
            try:
                self._mm.close()
            except BufferError:  # arrays from tensor_bytes() still alive: unmapped with them
                pass
            self._mm = None
        if self._f is not None:
            self._f.close()
            self._f = None

    def tensor_bytes(self, t: GGUFTensorInfo) -> np.ndarray:
        """The tensor's bytes as a read-only uint8 view of the mapping."""
        return np.frombuffer(self._mm, dtype=np.uint8, count=t.nbytes, offset=t.offset)


class _Cursor:
    def __init__(self, buf, pos=0):
        self.buf, self.pos = buf, pos

    def take(self, n):
        if self.pos + n > len(self.buf):
            raise GGUFError("truncated GGUF file")
        b = self.buf[self.pos:self.pos + n]  # mmap slices are bytes copies (no buffer export)
        self.pos += n
        return b

    def unpack(self, fmt):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self):
        n = self.unpack("<Q")
        return self.take(n).decode("utf-8", errors="replace")

    def value(self, vtype):
        if vtype in _SCALAR:
            return self.unpack(_SCALAR[vtype])
        if vtype == _STRING:
            return self.string()
        if vtype == _ARRAY:
            etype, n = self.unpack("<I"), self.unpack("<Q")
            if etype in _SCALAR and etype != 7:
                dt = np.dtype(_SCALAR[etype])
                return np.frombuffer(self.take(n * dt.itemsize), dtype=dt).copy()
            return [self.value(etype) for _ in range(n)]
        raise GGUFError(f"unknown GGUF metadata value type {vtype}")


def _nbytes(ggml_type: int, shape) -> int:
    if ggml_type not in GGML_TYPES:
        raise GGUFError(f"unknown ggml_type {ggml_type}")
    _, blk, bsz = GGML_TYPES[ggml_type]
    n = int(np.prod(shape)) if len(shape) else 1
    if shape and shape[0] % blk:
        raise GGUFError(f"row of {shape[0]} not a multiple of the {blk}-element block")
    return n // blk * bsz


def open_gguf(path: str) -> GGUFFile:
    """Parse the header, metadata and tensor table of a GGUF file (v2 / v3)."""
    f = open(path, "rb")
    try:
        mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    except ValueError as e:  # empty file
        f.close()
        raise GGUFError("empty GGUF file") from e
    try:
        c = _Cursor(mm)
        if c.take(4) != GGUF_MAGIC:
            raise GGUFError("not a GGUF file (bad magic)")
        version = c.unpack("<I")
        if version not in (2, 3):
            raise GGUFError(f"unsupported GGUF version {version}")
        n_tensors, n_kv = c.unpack("<Q"), c.unpack("<Q")
        meta = {}
        for _ in range(n_kv):
            key = c.string()
            meta[key] = c.value(c.unpack("<I"))
        infos = []
        for _ in range(n_tensors):
            name = c.string()
            nd = c.unpack("<I")
            shape = tuple(int(c.unpack("<Q")) for _ in range(nd))
            infos.append((name, shape, c.unpack("<I"), c.unpack("<Q")))
        align = int(meta.get("general.alignment", DEFAULT_ALIGNMENT))
        if align <= 0 or align & (align - 1):
            raise GGUFError(f"bad general.alignment {align}")
        data0 = (c.pos + align - 1) // align * align
        tensors = []
        for name, shape, ttype, off in infos:
            nb = _nbytes(ttype, shape)
            if off % align or data0 + off + nb > len(mm):
                raise GGUFError(f"tensor {name!r} out of bounds or misaligned")
            tensors.append(GGUFTensorInfo(name, shape, ttype, data0 + off, nb))
        del c
        return GGUFFile(path, version, meta, tensors, align, mm, f)
    except Exception:
        mm.close()
        f.close()
        raise


def kquant_qtensor(raw_bytes: np.ndarray, out_features: int, in_features: int, tag: str) -> QTensor:
    """Native k-quant bytes -> ``gguf_kquant`` QTensor [out, (in/256) * type_size]
    uint8, byte-identical (reference gguf.py:106-126)."""
    if tag not in GGUF_KQUANT_BLOCK:
        raise ValueError(f"unsupported native-fused tag {tag!r}")
    if in_features % QK_K:
        raise ValueError(f"{tag} needs in%256==0, got {in_features}")
    row_bytes = in_features // QK_K * GGUF_KQUANT_BLOCK[tag]
    u8 = np.ascontiguousarray(raw_bytes).view(np.uint8).reshape(-1)
    if u8.size != out_features * row_bytes:
        raise ValueError(f"gguf {tag}: {u8.size} bytes != {out_features}*{row_bytes}")
    data = torch.from_numpy(u8.reshape(out_features, row_bytes).copy())
    qt = QTensor(data, None, scheme="gguf_kquant", group_size=QK_K, codebook=tag)
    qt.validate()
    return qt


def load_gguf_kquant_tensors(path: str, *, device=None):
    """Yield ``(name, qtensor_or_None, type_name)`` for every tensor of a GGUF file:
    2-D Q4_K / Q5_K / Q6_K weights with in%256==0 as ``gguf_kquant`` QTensors
    (moved to ``device`` when given), anything else as None (reference
    gguf.py:213-235)."""
    with open_gguf(path) as g:
        for t in g.tensors:
            tag = NATIVE_FUSED.get(t.type_name)
            if len(t.shape) == 2 and tag and t.shape[0] % QK_K == 0:
                qt = kquant_qtensor(g.tensor_bytes(t), t.shape[1], t.shape[0], tag)
                if device is not None:
                    qt.data = qt.data.to(device)
                yield t.name, qt, t.type_name
            else:
                yield t.name, None, t.type_name


def gguf_type_histogram(path: str) -> dict:
    """``{type_name: {"count": n, "path": "native_fused" | "unsupported"}}`` over the
    file's tensors (reference gguf.py:189-210, with this build's coverage)."""
    hist: dict = {}
    with open_gguf(path) as g:
        for t in g.tensors:
            native = t.type_name in NATIVE_FUSED and len(t.shape) == 2
            e = hist.setdefault(t.type_name, {"count": 0,
                                              "path": "native_fused" if native else "unsupported"})
            e["count"] += 1
    return hist

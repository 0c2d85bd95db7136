"""Weight container of the k-quant linear path and the `.superl8` checkpoint file.

QTensor (reference superl8/format.py:219-303) describes a stored weight; the
schemes this hot path computes on are ``gguf_kquant`` (native GGUF k-quant
bytes kept resident, byte-identical to the GGUF file; the sub-block scales
live inside the bytes) for the Q4_K / Q5_K / Q6_K kernels and ``raw`` (a
tensor used as is). ``per_row_i8`` / ``per_chan_i8`` (int8 + fp32 scale) are
carried by the file format so checkpoints holding them load, but no kernel of
this path consumes them.

`.superl8` file (reference superl8/format.py:306-625; the layout below is the
file format, kept identical so files move between the two builds):

    "FNI8QCK1" | u64 header length H | header JSON (H bytes) | zero pad to 128 |
    blobs, each starting on a 128-byte boundary of the blob area

or, from the streaming writer (H = 0 marks it):

    "FNI8QCK1" | u64 0 | zero pad to 128 | blobs ... | header JSON |
    u64 header offset | u64 header length | "FNI8FOOT"

Blob offsets in the header are relative to the blob area (byte 128 of a
streaming file, pad128(16 + H) otherwise). Every tensor entry records dtype,
shape, offset, nbytes, crc32, the quant scheme and its scale blob's name
(``<name>.scale``), the baked-transform flags and a derived recipe. The bytes
of a blob are the tensor's resident device layout: loading is an mmap slice
plus one host-to-device copy, with no transcode.

Byte layouts this build shares with the reference (row-major int8 with an fp32
scale per row or channel, raw GGUF k-quant super-blocks) are tagged with the
reference's layout name "cuda-dp4a"; the reader accepts files written for
either build's arch/quant tags, since the bytes it hands to the kernels are
the same.
"""
from __future__ import annotations

import hashlib
import json
import math
import mmap
import os
import struct
import zlib
from dataclasses import asdict, dataclass, is_dataclass

import numpy as np
import torch

# Bytes per 256-weight super-block of the k-quant types served natively
# (reference format.py:209-214, the GGUF block sizes).
GGUF_KQUANT_BLOCK = {"q4_k": 144, "q5_k": 176, "q6_k": 210}
QK_K = 256

SCHEMES = ("gguf_kquant", "raw", "per_row_i8", "per_chan_i8")


@dataclass
class QTensor:
    """A stored weight: ``data`` plus how to read it.

    ``gguf_kquant``: uint8 ``data`` [out, (in/256) * type_size], ``codebook`` the
    GGML type tag ('q4_k' / 'q5_k' / 'q6_k'), ``group_size`` 256, no scale.
    ``per_row_i8``: int8 ``data`` [out, in] (in % 4 == 0) + fp32 ``scale`` [out].
    ``per_chan_i8``: int8 ``data`` + fp32 ``scale`` [..., 1, d].
    ``raw``: ``data`` used as is (norms, embeddings, float weights), no scale.
    ``rotated`` / ``hadamard_dim`` / ``smoothed`` record transforms baked in
    offline (a Hadamard rotation, the K-smoothing mean).
    """
    data: torch.Tensor
    scale: torch.Tensor | None = None
    scheme: str = "per_row_i8"   # field order and default as the reference's QTensor
    rotated: bool = False
    hadamard_dim: int = 0
    smoothed: bool = False
    group_size: int = 0
    codebook: str = ""

    def validate(self) -> None:
        if self.scheme == "gguf_kquant":
            assert self.data.dtype == torch.uint8 and self.data.dim() == 2, \
                "gguf_kquant needs uint8 data [out, n_superblocks * type_size]"
            assert self.scale is None, "gguf_kquant carries no separate scale"
            assert self.codebook in GGUF_KQUANT_BLOCK, (
                f"gguf_kquant type tag {self.codebook!r} "
                f"(expect one of {', '.join(sorted(GGUF_KQUANT_BLOCK))})")
            assert self.group_size == QK_K, f"gguf_kquant group_size must be {QK_K}"
            assert self.data.shape[-1] % GGUF_KQUANT_BLOCK[self.codebook] == 0, \
                f"{self.codebook} row bytes must be a multiple of {GGUF_KQUANT_BLOCK[self.codebook]}"
        elif self.scheme in ("per_row_i8", "per_chan_i8"):
            assert self.data.dtype == torch.int8, f"{self.scheme} needs int8 data"
            assert self.scale is not None and self.scale.dtype == torch.float32, \
                f"{self.scheme} needs an fp32 scale"
            assert self.data.shape[-1] % 4 == 0, \
                f"{self.scheme}: the contraction dim must be a multiple of 4"
        elif self.scheme == "raw":
            assert self.scale is None, "raw tensors carry no scale"
        else:
            raise AssertionError(f"unsupported scheme {self.scheme!r} on this path")

    @property
    def in_features(self) -> int:
        if self.scheme == "gguf_kquant":
            return self.data.shape[-1] // GGUF_KQUANT_BLOCK[self.codebook] * QK_K
        return self.data.shape[-1]

    @property
    def out_features(self) -> int:
        return self.data.shape[0]


# ---------------------------------------------------------------------------
# .superl8 framing constants (the file format)
# ---------------------------------------------------------------------------
MAGIC = b"FNI8QCK1"
FOOTER_MAGIC = b"FNI8FOOT"
ALIGN = 128
FORMAT_VERSION = 1
KERNEL_ABI_VERSION = 1
LAYOUT = "cuda-dp4a"            # the shared resident byte layout (see module doc)
ARCH = "gfx950"
QUANT = "mfma_w8a8"
# arch/quant tags whose blobs this build reads: its own and the reference's
READ_TARGETS = {("gfx950", "mfma_w8a8"), ("sm70", "dp4a_w8a8")}
WRITE_TARGETS = {"gfx950": ("gfx950", "mfma_w8a8"), "sm70": ("sm70", "dp4a_w8a8")}
SUPPORTED_VERSIONS = (1,)
SUPPORTED_ABIS = (1,)
SUPPORTED_LAYOUTS = ("cuda-dp4a",)

# file dtype name <-> (torch dtype, numpy dtype used to view the bytes)
_DTYPES = {
    "int8": (torch.int8, np.int8), "uint8": (torch.uint8, np.uint8),
    "int32": (torch.int32, np.int32), "float16": (torch.float16, np.float16),
    "float32": (torch.float32, np.float32),
    "bfloat16": (torch.bfloat16, np.uint16),  # numpy has no bf16: the bits as uint16
}
_DTYPE_OF_TORCH = {tdt: name for name, (tdt, _) in _DTYPES.items()}


def _align(n: int) -> int:
    return -(-n // ALIGN) * ALIGN


def _payload(t: torch.Tensor) -> bytes:
    """The tensor's bytes in memory order (little-endian, row-major), no conversion."""
    return t.detach().contiguous().cpu().reshape(-1).view(torch.uint8).numpy().tobytes()


def _dtype_name(t: torch.Tensor) -> str:
    name = _DTYPE_OF_TORCH.get(t.dtype)
    if name is None:
        raise ValueError(f"superl8 format: unsupported dtype {t.dtype} "
                         f"(one of {', '.join(_DTYPES)})")
    return name


def recipe_of(entry: dict) -> dict:
    """Logical quant recipe of a tensor entry, derived from its stored fields
    (reference format.py:137-179): dtype, per-row symmetry, group size, baked
    transforms and an id string such as 'int8-perrow-sym-had-ksmooth'."""
    scheme = entry.get("scheme", "raw")
    if scheme == "raw":
        dt = entry.get("dtype", "raw")
        dtype = {"float16": "fp16", "float32": "fp32"}.get(dt, dt)
    else:
        dtype = {"per_row_i8": "int8", "per_chan_i8": "int8"}.get(scheme, scheme)
    gs = int(entry.get("group_size") or 0)
    parts = [dtype]
    if scheme == "per_row_i8":
        parts.append("perrow-sym")
    elif scheme == "per_chan_i8":
        parts.append("perchan-sym")
    if gs:
        parts.append(f"g{gs}")
    if entry.get("codebook"):
        parts.append(entry["codebook"])
    if entry.get("rotated"):
        parts.append("had")
    if entry.get("smoothed"):
        parts.append("ksmooth")
    transforms = (["k-smoothing"] if entry.get("smoothed") else []) + \
        (["hadamard"] if entry.get("rotated") else [])
    return {"dtype": dtype, "per_row_symmetric": scheme == "per_row_i8", "group_size": gs,
            "transforms": transforms, "recipe_id": "-".join(parts)}


def content_hash(entries: dict) -> str:
    """Digest of the blobs from their CRCs and sizes (sorted by name): equal
    weights give equal hashes without re-reading any blob."""
    text = "|".join(f"{n}:{e['crc32']:08x}:{e['nbytes']}" for n, e in sorted(entries.items()))
    return "superl8-crc:" + hashlib.sha256(text.encode("utf-8")).hexdigest()[:32]


def _jsonable(o):
    """json.dumps fallback for metadata objects (configs, dataclasses): never raises."""
    if callable(getattr(o, "to_dict", None)):
        try:
            return o.to_dict()
        except Exception:
            pass
    if is_dataclass(o) and not isinstance(o, type):
        return asdict(o)
    if hasattr(o, "__dict__"):
        return {k: v for k, v in vars(o).items() if not k.startswith("_")}
    return str(o)


def _provenance(source_model, weight_hash, calibration_fingerprint) -> dict:
    """Writer stamp: deterministic (no time, no randomness) so equal inputs give
    byte-identical files."""
    return {"tool": "superl8_amd.format", "format_version": FORMAT_VERSION,
            "superl8_version": _package_version(), "kernel_abi_version": KERNEL_ABI_VERSION,
            "layout": LAYOUT, "source_model": source_model, "weight_hash": weight_hash,
            "calibration_fingerprint": calibration_fingerprint}


def _package_version() -> str:
    try:
        from . import __version__
        return str(__version__)
    except Exception:
        return "unknown"


def _blob_entries(name: str, qt: QTensor):
    """(blob name, tensor, entry fields) for a QTensor's data and its scale."""
    qt.validate()
    fields = {"scheme": qt.scheme, "scale": f"{name}.scale" if qt.scale is not None else None,
              "rotated": bool(qt.rotated), "hadamard_dim": int(qt.hadamard_dim),
              "smoothed": bool(qt.smoothed), "group_size": int(qt.group_size),
              "codebook": qt.codebook}
    yield name, qt.data, fields
    if qt.scale is not None:
        yield f"{name}.scale", qt.scale, {"scheme": "raw", "scale": None, "rotated": False,
                                          "hadamard_dim": 0, "smoothed": False,
                                          "group_size": 0, "codebook": ""}


def _header(entries, target, shards, meta, source_model, weight_hash, calib) -> bytes:
    arch, quant = WRITE_TARGETS[target]
    for e in entries.values():
        e["recipe"] = recipe_of(e)
    hdr = {"arch": arch, "quant": quant, "version": FORMAT_VERSION,
           "kernel_abi_version": KERNEL_ABI_VERSION, "layout": LAYOUT,
           "provenance": _provenance(source_model,
                                     weight_hash if weight_hash is not None else content_hash(entries),
                                     calib),
           "align": ALIGN, "tensors": entries, "shards": shards or {}, "__meta__": meta or {}}
    return json.dumps(hdr, default=_jsonable).encode("utf-8")


def save_superl8(path: str, tensors: dict, *, shards: dict | None = None, meta: dict | None = None,
                 source_model: str | None = None, weight_hash: str | None = None,
                 calibration_fingerprint: str | None = None, target: str = ARCH) -> None:
    """Write a header-first `.superl8` file from a dict of QTensors. Two passes:
    sizes and CRCs first (each payload built, summed and dropped), then the blobs
    are streamed, so at most one extra payload is in memory at a time.
    `target` selects the arch/quant tags ('gfx950', or 'sm70' for files the
    reference build reads)."""
    order, entries, pos = [], {}, 0
    for name, qt in tensors.items():
        for bname, t, fields in _blob_entries(name, qt):
            raw = _payload(t)
            pos = _align(pos)
            entries[bname] = {"dtype": _dtype_name(t), "shape": list(t.shape), "offset": pos,
                              "nbytes": len(raw), "crc32": zlib.crc32(raw) & 0xFFFFFFFF, **fields}
            pos += len(raw)
            order.append((bname, t))
    hdr = _header(entries, target, shards, meta, source_model, weight_hash, calibration_fingerprint)
    blob0 = _align(16 + len(hdr))
    with open(path, "wb") as f:
        f.write(MAGIC + struct.pack("<Q", len(hdr)) + hdr)
        for bname, t in order:
            f.write(b"\0" * (blob0 + entries[bname]["offset"] - f.tell()))
            f.write(_payload(t))


class FQWriter:
    """Streaming `.superl8` writer: each tensor is written when added, the header
    and footer at finalize(), so a converter holds one tensor at a time."""

    def __init__(self, path: str, *, target: str = ARCH):
        if target not in WRITE_TARGETS:
            raise ValueError(f"superl8 format: unknown target {target!r}")
        self._target = target
        self._f = open(path, "wb")
        self._f.write(MAGIC + struct.pack("<Q", 0))  # header length 0: footer format
        self._blob0 = _align(self._f.tell())
        self._f.write(b"\0" * (self._blob0 - self._f.tell()))
        self._entries: dict[str, dict] = {}

    def add(self, name: str, qt: QTensor) -> None:
        for bname, t, fields in _blob_entries(name, qt):
            if bname in self._entries:
                raise ValueError(f"superl8 format: duplicate tensor {bname!r}")
            raw = _payload(t)
            at = self._blob0 + _align(self._f.tell() - self._blob0)
            self._f.write(b"\0" * (at - self._f.tell()))
            self._entries[bname] = {"dtype": _dtype_name(t), "shape": list(t.shape),
                                    "offset": at - self._blob0, "nbytes": len(raw),
                                    "crc32": zlib.crc32(raw) & 0xFFFFFFFF, **fields}
            self._f.write(raw)

    def finalize(self, *, shards: dict | None = None, meta: dict | None = None,
                 source_model: str | None = None, weight_hash: str | None = None,
                 calibration_fingerprint: str | None = None) -> None:
        hdr = _header(self._entries, self._target, shards, meta, source_model, weight_hash,
                      calibration_fingerprint)
        off = self._f.tell()
        self._f.write(hdr + struct.pack("<QQ", off, len(hdr)) + FOOTER_MAGIC)
        self._f.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        if not self._f.closed:
            self._f.close()


class FQReader:
    """mmap reader of a `.superl8` file (either framing). Opening parses and
    checks the header (version, arch/quant, layout and kernel-ABI tags, every
    blob inside the file and its size equal to shape x dtype); tensors are read
    lazily, so only the pages of the tensors fetched are touched."""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        try:
            self._open()
        except Exception:
            self._f.close()
            raise

    def _open(self) -> None:
        f = self._f
        size = os.fstat(f.fileno()).st_size
        pre = f.read(16)
        if len(pre) < 16 or pre[:8] != MAGIC:
            raise ValueError(f"superl8 format: bad magic {pre[:8]!r} (not a .superl8 checkpoint)")
        (hlen,) = struct.unpack("<Q", pre[8:])
        if hlen == 0:
            if size < 16 + 24:
                raise ValueError("superl8 format: bad footer magic (truncated streaming .superl8?)")
            f.seek(size - 24)
            off, n = struct.unpack("<QQ", f.read(16))
            if f.read(8) != FOOTER_MAGIC:
                raise ValueError("superl8 format: bad footer magic (truncated streaming .superl8?)")
            if off + n > size - 24:
                raise ValueError("superl8 format: footer points past the end of the file")
            f.seek(off)
            raw = f.read(n)
            self._blob0 = _align(16)
        else:
            if 16 + hlen > size:
                raise ValueError("superl8 format: header length past the end of the file")
            raw = f.read(hlen)
            self._blob0 = _align(16 + hlen)
        self.header = json.loads(raw)
        self._check_tags()
        self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) if size else None
        for name, e in self.header["tensors"].items():
            if e["dtype"] not in _DTYPES:
                raise ValueError(f"superl8 format: tensor {name!r} has unknown dtype {e['dtype']!r}")
            if e["offset"] < 0:
                raise ValueError(f"superl8 format: negative offset {e['offset']} for tensor {name!r}")
            end = self._blob0 + e["offset"] + e["nbytes"]
            if end > size:
                raise ValueError(f"superl8 format: tensor {name!r} offset+{e['nbytes']}B exceeds "
                                 f"file size ({end} > {size})")
            want = math.prod(e["shape"]) * np.dtype(_DTYPES[e["dtype"]][1]).itemsize
            if want != e["nbytes"]:
                raise ValueError(f"superl8 format: tensor {name!r} shape {e['shape']} * "
                                 f"{e['dtype']} = {want}B, but header declares {e['nbytes']}B")

    def _check_tags(self) -> None:
        h = self.header
        ver = h.get("version", 1)
        if ver not in SUPPORTED_VERSIONS:
            raise ValueError(f"superl8 format: unsupported format version {ver} (this build "
                             f"reads {list(SUPPORTED_VERSIONS)}) — upgrade superl8 to read this file")
        if (h.get("arch"), h.get("quant")) not in READ_TARGETS:
            raise ValueError(f"superl8 format: arch/quant mismatch ({h.get('arch')}/"
                             f"{h.get('quant')} is not one of {sorted(READ_TARGETS)})")
        layout = h.get("layout", LAYOUT)  # absent: a legacy file, always this layout
        if layout not in SUPPORTED_LAYOUTS:
            raise ValueError(f"superl8 format: unsupported backend layout {layout!r} "
                             f"(this build reads {list(SUPPORTED_LAYOUTS)})")
        abi = h.get("kernel_abi_version", KERNEL_ABI_VERSION)
        if abi not in SUPPORTED_ABIS:
            raise ValueError(f"superl8 format: unsupported kernel-ABI / resident-layout version "
                             f"{abi} (this build reads {list(SUPPORTED_ABIS)})")

    # -- introspection -------------------------------------------------------
    @property
    def names(self) -> list[str]:
        return [n for n in self.header["tensors"] if not n.endswith(".scale")]

    @property
    def shards(self) -> dict:
        return self.header.get("shards", {})

    @property
    def provenance(self) -> dict:
        return self.header.get("provenance", {})

    def info(self, name: str) -> dict:
        return self.header["tensors"][name]

    def recipe(self, name: str) -> dict:
        e = self.header["tensors"][name]
        return e.get("recipe") or recipe_of(e)

    # -- loads ---------------------------------------------------------------
    def _array(self, name: str) -> np.ndarray:
        e = self.header["tensors"][name]
        start = self._blob0 + e["offset"]
        buf = self._mm[start:start + e["nbytes"]] if e["nbytes"] else b""
        return np.frombuffer(buf, dtype=_DTYPES[e["dtype"]][1]).reshape(e["shape"])

    def get(self, name: str, device="cpu", *, verify: bool = False) -> torch.Tensor:
        """One tensor on `device`: the blob's bytes, one host-to-device copy."""
        e = self.header["tensors"][name]
        arr = self._array(name)
        if verify and (zlib.crc32(arr.tobytes()) & 0xFFFFFFFF) != e["crc32"]:
            raise ValueError(f"superl8 format: crc mismatch on {name!r} (corrupt file)")
        t = torch.from_numpy(arr.copy())
        if e["dtype"] == "bfloat16":
            t = t.view(torch.bfloat16)
        return t.to(device)

    def get_qtensor(self, name: str, device="cpu") -> QTensor:
        e = self.header["tensors"][name]
        scheme, codebook = e.get("scheme", "raw"), e.get("codebook", "")
        if scheme not in SCHEMES:
            raise ValueError(f"superl8 format: unsupported scheme {scheme!r} on {name!r} "
                             f"(this build runs {', '.join(SCHEMES)})")
        if scheme == "gguf_kquant" and codebook not in GGUF_KQUANT_BLOCK:
            raise ValueError(f"superl8 format: unsupported gguf_kquant type {codebook!r} on "
                             f"{name!r} (this build runs {', '.join(GGUF_KQUANT_BLOCK)})")
        scale = self.get(e["scale"], device) if e.get("scale") else None
        return QTensor(self.get(name, device), scale, e["scheme"], bool(e.get("rotated", False)),
                       int(e.get("hadamard_dim", 0)), bool(e.get("smoothed", False)),
                       int(e.get("group_size", 0)), e.get("codebook", ""))

    def load_many(self, names, device="cpu") -> dict:
        return {n: self.get_qtensor(n, device) for n in names}

    def verify(self) -> bool:
        for name in self.header["tensors"]:
            self.get(name, verify=True)
        return True

    def close(self) -> None:
        if getattr(self, "_mm", None) is not None:
            self._mm.close()
        self._f.close()

    def __enter__(self) -> "FQReader":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

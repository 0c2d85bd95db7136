"""The `.superl8` container (superl8_amd.format): both framings, literal files
built byte by byte from the format description, the reader's checks, and the
GPU load into the k-quant linear (reference superl8/format.py:306-625 and its
tests/test_format*.py)."""
import json
import struct
import zlib

import numpy as np
import pytest
import torch

from oracle import q4k as oq
from superl8_amd import format as fmt
from superl8_amd.format import FQReader, FQWriter, QTensor, save_superl8

RNG = np.random.default_rng(7)


def _tensors():
    w = torch.from_numpy(oq.random_weights(8, 512, seed=3))
    i8 = torch.from_numpy(RNG.integers(-127, 128, (6, 16), dtype=np.int8))
    return {
        "blk.0.ffn_up.weight": QTensor(w, None, "gguf_kquant", group_size=256, codebook="q4_k"),
        "blk.0.attn_q.weight": QTensor(i8, torch.rand(6), "per_row_i8", rotated=True,
                                       hadamard_dim=16, smoothed=True),
        "norm.weight": QTensor(torch.randn(5, dtype=torch.float16), None, "raw"),
        "emb.bf16": QTensor(torch.randn(3, 4).to(torch.bfloat16), None, "raw"),
    }


def _write(path, tensors, streaming, **kw):
    if streaming:
        with FQWriter(str(path), target=kw.pop("target", "gfx950")) as w:
            for n, qt in tensors.items():
                w.add(n, qt)
            w.finalize(**kw)
    else:
        save_superl8(str(path), tensors, **kw)


@pytest.mark.parametrize("streaming", [False, True])
def test_roundtrip(tmp_path, streaming):
    ts = _tensors()
    p = tmp_path / "m.superl8"
    _write(p, ts, streaming, shards={"pp_stages": [["norm.weight"]]}, meta={"arch": "demo"},
           source_model="demo/model")
    with FQReader(str(p)) as r:
        assert sorted(r.names) == sorted(ts)
        assert r.shards == {"pp_stages": [["norm.weight"]]}
        assert r.provenance["source_model"] == "demo/model"
        assert r.provenance["weight_hash"].startswith("superl8-crc:")
        for n, qt in ts.items():
            got = r.get_qtensor(n)
            assert got.scheme == qt.scheme and got.codebook == qt.codebook
            assert got.rotated == qt.rotated and got.smoothed == qt.smoothed
            assert got.data.dtype == qt.data.dtype and torch.equal(
                got.data.view(torch.uint8), qt.data.view(torch.uint8))
            if qt.scale is not None:
                assert torch.equal(got.scale, qt.scale)
        assert r.recipe("blk.0.attn_q.weight")["recipe_id"] == "int8-perrow-sym-had-ksmooth"
        assert r.recipe("blk.0.attn_q.weight")["transforms"] == ["k-smoothing", "hadamard"]
        assert r.recipe("blk.0.ffn_up.weight")["recipe_id"] == "gguf_kquant-g256-q4_k"
        assert r.verify()


def test_both_framings_same_blobs_and_deterministic(tmp_path):
    ts = _tensors()
    a, b, c = tmp_path / "a", tmp_path / "b", tmp_path / "c"
    _write(a, ts, False)
    _write(b, ts, True)
    _write(c, ts, False)
    assert a.read_bytes() == c.read_bytes()  # no timestamps or randomness
    with FQReader(str(a)) as ra, FQReader(str(b)) as rb:
        assert ra.header["tensors"] == rb.header["tensors"]
        assert ra.provenance == rb.provenance


def test_writer_output_parses_per_format_description(tmp_path):
    """Read the header-first file by hand: magic, u64 header length, JSON, blobs at
    pad128(16 + H) + offset, each offset a multiple of 128, CRC32 of the bytes."""
    ts = _tensors()
    p = tmp_path / "m.superl8"
    _write(p, ts, False)
    raw = p.read_bytes()
    assert raw[:8] == b"FNI8QCK1"
    (h,) = struct.unpack("<Q", raw[8:16])
    hdr = json.loads(raw[16:16 + h])
    assert hdr["align"] == 128 and hdr["version"] == 1 and hdr["layout"] == "cuda-dp4a"
    blob0 = (16 + h + 127) // 128 * 128
    for name, e in hdr["tensors"].items():
        assert e["offset"] % 128 == 0
        blob = raw[blob0 + e["offset"]: blob0 + e["offset"] + e["nbytes"]]
        assert zlib.crc32(blob) & 0xFFFFFFFF == e["crc32"]
    w = ts["blk.0.ffn_up.weight"].data.numpy().tobytes()
    e = hdr["tensors"]["blk.0.ffn_up.weight"]
    assert raw[blob0 + e["offset"]: blob0 + e["offset"] + e["nbytes"]] == w


def _literal(hdr_tensors, blobs, *, streaming, arch="sm70", quant="dp4a_w8a8", extra=None):
    """A file assembled from the format description alone (no writer code)."""
    hdr = {"arch": arch, "quant": quant, "version": 1, "align": 128, "tensors": hdr_tensors,
           "shards": {}, "__meta__": {}}
    hdr.update(extra or {})
    hb = json.dumps(hdr).encode()
    area = bytearray()
    for off, payload in blobs:
        area += b"\0" * (off - len(area))
        area += payload
    if streaming:
        out = bytearray(b"FNI8QCK1" + struct.pack("<Q", 0)) + b"\0" * 112 + area
        hoff = len(out)
        out += hb + struct.pack("<QQ", hoff, len(hb)) + b"FNI8FOOT"
    else:
        out = bytearray(b"FNI8QCK1" + struct.pack("<Q", len(hb)) + hb)
        out += b"\0" * ((-len(out)) % 128) + area
    return bytes(out)


@pytest.mark.parametrize("streaming", [False, True])
def test_literal_reference_tagged_file(tmp_path, streaming):
    """A file with the reference build's tags (sm70 / dp4a_w8a8, no layout field:
    a legacy v1 file) and two blobs: int8 [2,4] + its fp32 scale at offset 128."""
    codes = np.array([[1, -2, 3, -4], [5, 6, -7, 127]], np.int8)
    scale = np.array([0.5, 0.25], np.float32)
    ent = {
        "w": {"dtype": "int8", "shape": [2, 4], "offset": 0, "nbytes": 8,
              "crc32": zlib.crc32(codes.tobytes()), "scheme": "per_row_i8", "scale": "w.scale",
              "rotated": False, "hadamard_dim": 0, "smoothed": False, "group_size": 0,
              "codebook": ""},
        "w.scale": {"dtype": "float32", "shape": [2], "offset": 128, "nbytes": 8,
                    "crc32": zlib.crc32(scale.tobytes()), "scheme": "raw", "scale": None},
    }
    p = tmp_path / "ref.superl8"
    p.write_bytes(_literal(ent, [(0, codes.tobytes()), (128, scale.tobytes())], streaming=streaming))
    with FQReader(str(p)) as r:
        assert r.names == ["w"]
        qt = r.get_qtensor("w")
        np.testing.assert_array_equal(qt.data.numpy(), codes)
        np.testing.assert_array_equal(qt.scale.numpy(), scale)
        assert r.recipe("w")["recipe_id"] == "int8-perrow-sym"  # derived (no stored recipe)
        assert r.verify()


@pytest.mark.parametrize("scheme,codebook,msg", [
    ("per_group_i4", "", "unsupported scheme 'per_group_i4'"),
    ("gguf_kquant", "q2_k", "unsupported gguf_kquant type 'q2_k'"),
])
def test_reference_tagged_unsupported_scheme_rejected(tmp_path, scheme, codebook, msg):
    """A reference-tagged file whose tensor uses a scheme this build does not run
    reads (header, raw blobs) but get_qtensor refuses it with a clear error."""
    data = np.arange(16, dtype=np.uint8)
    ent = {"w": {"dtype": "uint8", "shape": [2, 8], "offset": 0, "nbytes": 16,
                 "crc32": zlib.crc32(data.tobytes()), "scheme": scheme, "scale": None,
                 "rotated": False, "hadamard_dim": 0, "smoothed": False, "group_size": 32,
                 "codebook": codebook}}
    p = tmp_path / "unsup.superl8"
    p.write_bytes(_literal(ent, [(0, data.tobytes())], streaming=False))
    with FQReader(str(p)) as r:
        np.testing.assert_array_equal(r.get("w").numpy().ravel(), data)
        with pytest.raises(ValueError, match=msg):
            r.get_qtensor("w")


def test_sm70_target_writes_reference_tags(tmp_path):
    p = tmp_path / "m.superl8"
    _write(p, _tensors(), True, target="sm70")
    with FQReader(str(p)) as r:
        assert (r.header["arch"], r.header["quant"]) == ("sm70", "dp4a_w8a8")


def _entry(shape=(2,), dtype="float32", offset=0, nbytes=8):
    return {"dtype": dtype, "shape": list(shape), "offset": offset, "nbytes": nbytes, "crc32": 0,
            "scheme": "raw", "scale": None}


@pytest.mark.parametrize("case,msg", [
    ("magic", "bad magic"), ("footer", "bad footer magic"), ("version", "format version"),
    ("arch", "arch/quant mismatch"), ("layout", "backend layout"), ("abi", "kernel-ABI"),
    ("size", "declares"), ("past_eof", "exceeds file size"), ("neg", "negative offset"),
])
def test_reader_rejects(tmp_path, case, msg):
    p = tmp_path / "bad.superl8"
    blobs = [(0, b"\0" * 8)]
    if case == "magic":
        data = b"GGUF" + b"\0" * 60
    elif case == "footer":
        data = _literal({"x": _entry()}, blobs, streaming=True)[:-3]
    else:
        ent, extra = {"x": _entry()}, {}
        if case == "version":
            extra = {"version": 2}
        elif case == "arch":
            extra = {"arch": "sm90"}
        elif case == "layout":
            extra = {"layout": "vulkan-dp4a"}
        elif case == "abi":
            extra = {"kernel_abi_version": 2}
        elif case == "size":
            ent = {"x": _entry(shape=(3,))}
        elif case == "past_eof":
            ent = {"x": _entry(offset=4096)}
        elif case == "neg":
            ent = {"x": _entry(offset=-128)}
        data = _literal(ent, blobs, streaming=False, extra=extra)
    p.write_bytes(data)
    with pytest.raises(ValueError, match=msg):
        FQReader(str(p))


def test_crc_detects_corruption(tmp_path):
    p = tmp_path / "m.superl8"
    _write(p, _tensors(), False)
    raw = bytearray(p.read_bytes())
    raw[-1] ^= 0xFF  # last byte of the last blob
    p.write_bytes(bytes(raw))
    with FQReader(str(p)) as r:
        with pytest.raises(ValueError, match="crc mismatch"):
            r.verify()


def test_validate_rejects_bad_qtensors():
    with pytest.raises(AssertionError):
        QTensor(torch.zeros(4, 100, dtype=torch.uint8), None, "gguf_kquant", group_size=256,
                codebook="q4_k").validate()
    with pytest.raises(AssertionError):
        QTensor(torch.zeros(4, 6, dtype=torch.int8), torch.ones(4), "per_row_i8").validate()
    with pytest.raises(AssertionError):
        QTensor(torch.zeros(4, 8, dtype=torch.int8), torch.ones(4).half(), "per_row_i8").validate()
    with pytest.raises(ValueError):
        save_superl8("/dev/null", {"x": QTensor(torch.zeros(2, dtype=torch.float64), None, "raw")})


@pytest.mark.gpu
def test_superl8_feeds_the_kquant_linear(tmp_path, device):
    """Native Q4_K bytes written to a .superl8 file, loaded straight to the GPU and
    run through superl8.linear: identical to the same bytes used directly."""
    import superl8_amd

    w = oq.random_weights(96, 1024, seed=11)
    qt = QTensor(torch.from_numpy(w), None, "gguf_kquant", group_size=256, codebook="q4_k")
    p = tmp_path / "m.superl8"
    _write(p, {"w": qt}, True)
    x = torch.randn(3, 1024, device=device, dtype=torch.float16)
    with FQReader(str(p)) as r:
        loaded = r.get_qtensor("w", device)
    assert loaded.data.is_cuda
    y = superl8_amd.linear(x, loaded)
    y0 = superl8_amd.linear_q4k(x, torch.from_numpy(w).to(device))
    assert torch.equal(y, y0)

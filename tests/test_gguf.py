"""The GGUF reader (superl8_amd.gguf): container parsing, byte-identical native
k-quant tensors, dispatch and error handling (reference superl8/gguf.py:106-235;
the reference reads files through llama.cpp's `gguf` package, absent here, so the
files are made by tests/gguf_writer.py and by a literal byte string)."""
import struct

import numpy as np
import pytest
import torch

from oracle import kquant as okq
from oracle import q4k as oq
from superl8_amd import gguf
from superl8_amd.format import QTensor
from tests.gguf_writer import write_gguf

RNG = np.random.default_rng(0)


def _kq(tag, N, K, seed):
    return {"q4_k": oq.random_weights, "q5_k": okq.q5k_random, "q6_k": okq.q6k_random}[tag](N, K, seed)


def test_literal_minimal_file(tmp_path):
    """A file written byte by byte from the format description: one u32 key, one
    F32 tensor [3] at offset 0 after 32-byte alignment."""
    b = bytearray(b"GGUF") + struct.pack("<IQQ", 3, 1, 1)
    b += struct.pack("<Q", 11) + b"test.answer" + struct.pack("<II", 4, 42)
    b += struct.pack("<Q", 1) + b"w" + struct.pack("<IQIQ", 1, 3, 0, 0)
    b += b"\0" * ((-len(b)) % 32)
    start = len(b)
    b += np.array([1.5, -2.0, 3.25], np.float32).tobytes()
    p = tmp_path / "m.gguf"
    p.write_bytes(bytes(b))
    with gguf.open_gguf(str(p)) as g:
        assert g.version == 3 and g.metadata == {"test.answer": 42}
        (t,) = g.tensors
        assert (t.name, t.shape, t.type_name, t.offset, t.nbytes) == ("w", (3,), "F32", start, 12)
        np.testing.assert_array_equal(g.tensor_bytes(t).view(np.float32), [1.5, -2.0, 3.25])


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_roundtrip_metadata_and_tensors(tmp_path, alignment):
    meta = {"general.architecture": "llama", "general.name": "tiny",
            "a.u8": np.uint8(7), "a.i16": np.int16(-3), "a.f32": np.float32(0.5),
            "a.u64": np.uint64(1 << 40), "a.f64": 2.5, "a.i64": -9, "a.flag": True,
            "a.arr_i32": np.arange(5, dtype=np.int32), "a.arr_f32": np.ones(3, np.float32),
            "tok.list": ["<s>", "</s>", "héllo"]}
    w4 = _kq("q4_k", 6, 512, 1)
    w5 = _kq("q5_k", 3, 256, 2)
    w6 = _kq("q6_k", 5, 768, 3)
    norm = RNG.standard_normal(512).astype(np.float32)
    q80 = RNG.integers(0, 256, 4 * 34, dtype=np.uint8)          # Q8_0 [128, 1]
    emb = RNG.standard_normal((4, 8)).astype(np.float16)
    tensors = [("blk.0.attn_q.weight", 12, (512, 6), w4.tobytes()),
               ("blk.0.ffn_up.weight", 13, (256, 3), w5.tobytes()),
               ("output.weight", 14, (768, 5), w6.tobytes()),
               ("blk.0.attn_norm.weight", 0, (512,), norm.tobytes()),
               ("blk.0.other.weight", 8, (128, 1), q80.tobytes()),
               ("token_embd.weight", 1, (8, 4), emb.tobytes())]
    p = tmp_path / "t.gguf"
    write_gguf(str(p), meta, tensors, alignment=alignment)
    with gguf.open_gguf(str(p)) as g:
        assert g.alignment == alignment
        for k, v in meta.items():
            got = g.metadata[k]
            if isinstance(v, np.ndarray):
                np.testing.assert_array_equal(got, v)
            else:
                assert got == v, k
        assert [t.name for t in g.tensors] == [t[0] for t in tensors]
        for t, (_, ty, shape, raw) in zip(g.tensors, tensors):
            assert t.ggml_type == ty and t.shape == shape and t.offset % alignment == 0
            assert g.tensor_bytes(t).tobytes() == raw
    got = {n: (qt, tn) for n, qt, tn in gguf.load_gguf_kquant_tensors(str(p))}
    for name, w, tag, K in (("blk.0.attn_q.weight", w4, "q4_k", 512),
                            ("blk.0.ffn_up.weight", w5, "q5_k", 256),
                            ("output.weight", w6, "q6_k", 768)):
        qt, _ = got[name]
        assert isinstance(qt, QTensor) and qt.codebook == tag and qt.scheme == "gguf_kquant"
        assert qt.data.dtype == torch.uint8 and qt.in_features == K
        np.testing.assert_array_equal(qt.data.numpy(), w)
    assert got["blk.0.attn_norm.weight"] == (None, "F32")
    assert got["blk.0.other.weight"] == (None, "Q8_0")
    hist = gguf.gguf_type_histogram(str(p))
    assert hist["Q4_K"] == {"count": 1, "path": "native_fused"}
    assert hist["Q8_0"]["path"] == "unsupported" and hist["F16"]["count"] == 1


def test_kquant_qtensor_checks():
    w = _kq("q6_k", 4, 512, 5)
    qt = gguf.kquant_qtensor(w, 4, 512, "q6_k")
    assert qt.data.shape == (4, 420) and qt.out_features == 4
    with pytest.raises(ValueError):
        gguf.kquant_qtensor(w, 4, 500, "q6_k")
    with pytest.raises(ValueError):
        gguf.kquant_qtensor(w, 5, 512, "q6_k")
    with pytest.raises(ValueError):
        gguf.kquant_qtensor(w, 4, 512, "iq4_xs")


def test_rejects_malformed(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGML" + b"\0" * 28)
    with pytest.raises(gguf.GGUFError, match="magic"):
        gguf.open_gguf(str(p))
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 1, 0, 0))
    with pytest.raises(gguf.GGUFError, match="version"):
        gguf.open_gguf(str(p))
    w = _kq("q4_k", 2, 256, 1)
    write_gguf(str(p), {}, [("w", 12, (256, 2), w.tobytes())])
    raw = p.read_bytes()
    p.write_bytes(raw[:-10])                                  # data cut short
    with pytest.raises(gguf.GGUFError, match="bounds"):
        gguf.open_gguf(str(p))
    p.write_bytes(raw[:30])                                   # header cut short
    with pytest.raises(gguf.GGUFError, match="truncated"):
        gguf.open_gguf(str(p))
    write_gguf(str(p), {}, [("w", 12, (200, 2), b"\0" * 288)])  # row not a block multiple
    with pytest.raises(gguf.GGUFError, match="block"):
        gguf.open_gguf(str(p))

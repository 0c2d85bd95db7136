"""A GGUF file's native k-quant tensors run on the fused kernels through
superl8_amd.linear exactly as the direct linear_q{4,5,6}k calls (reference
tests/test_gemm_q4k.py:415-428,498-512)."""
import numpy as np
import pytest
import torch

import superl8_amd
from oracle import kquant as okq
from oracle import q4k as oq
from superl8_amd import gguf
from tests.gguf_writer import write_gguf

pytestmark = pytest.mark.gpu


def test_gguf_linear_matches_direct(device, tmp_path):
    w4 = oq.random_weights(64, 512, seed=1)
    w5 = okq.q5k_random(96, 512, seed=2)
    w6 = okq.q6k_random(130, 512, seed=3)
    p = tmp_path / "m.gguf"
    write_gguf(str(p), {"general.architecture": "test"},
               [("a", 12, (512, 64), w4.tobytes()), ("b", 13, (512, 96), w5.tobytes()),
                ("c", 14, (512, 130), w6.tobytes())])
    qts = {n: qt for n, qt, _ in gguf.load_gguf_kquant_tensors(str(p), device=device)}
    for M in (1, 6, 40):
        x = torch.randn(M, 512, device=device, dtype=torch.float16)
        for name, w, lin in (("a", w4, superl8_amd.linear_q4k), ("b", w5, superl8_amd.linear_q5k),
                             ("c", w6, superl8_amd.linear_q6k)):
            y = superl8_amd.linear(x, qts[name])
            assert torch.equal(y, lin(x, torch.from_numpy(w).to(device)))


def test_linear_rejects_unknown(device):
    from superl8_amd.format import QTensor

    x = torch.randn(2, 256, device=device, dtype=torch.float16)
    with pytest.raises(ValueError):
        superl8_amd.linear(x, QTensor(torch.zeros(4, 144, dtype=torch.uint8, device=device),
                                      scheme="gguf_kquant", group_size=256, codebook="q3_k"))
    with pytest.raises(ValueError):
        superl8_amd.linear(x, QTensor(torch.zeros(4, 256, device=device), scheme="raw"))

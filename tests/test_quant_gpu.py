"""GPU parity of the quantisation prologue against the oracle (bit-exact)."""
import math

import numpy as np
import pytest
import torch

from oracle import quant as oqn
from superl8_amd import _C, quant

pytestmark = pytest.mark.gpu

SHAPES = [(1, 896), (3, 896), (8, 896), (16, 4864), (4096, 896), (2, 17), (5, 4097), (7, 64),
          (33, 128), (1, 5120), (8, 5120),
          # vectorised paths: 1..8 vectors per lane, one workgroup per row
          (2, 16384), (3, 12288), (4, 8), (9, 2048), (17, 1024), (1000, 256)]


def _np(x):
    return x.detach().cpu().numpy()


def _as_oracle(x):
    if x.dtype == torch.bfloat16:
        return oqn.bf16_bits_to_f32(_np(x.view(torch.int16)).view(np.uint16))
    return _np(x.float())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,K", SHAPES)
def test_quantize_rowwise_bit_exact(device, M, K, dtype):
    torch.manual_seed(M * 7 + K)
    x = torch.randn(M, K, device=device, dtype=dtype) * 3.0
    q, s = _C.quantize_i8_rowwise(x)
    rq, rs = oqn.quantize_rows(_as_oracle(x))
    assert q.dtype == torch.int8 and q.shape == (M, K) and s.shape == (M,)
    np.testing.assert_array_equal(_np(q), rq)
    np.testing.assert_array_equal(_np(s), rs)


def test_quantize_zero_row_and_outlier(device):
    x = torch.zeros(3, 128, device=device, dtype=torch.float16)
    x[1, 40] = 50.0
    q, s = _C.quantize_i8_rowwise(x)
    assert s[0].item() == 1.0 and not q[0].any()
    rq, rs = oqn.quantize_rows(_np(x.float()))
    np.testing.assert_array_equal(_np(q), rq)
    np.testing.assert_array_equal(_np(s), rs)


def test_quantize_deterministic(device):
    x = torch.randn(8, 896, device=device, dtype=torch.float16) * 4
    outs = [_C.quantize_i8_rowwise(x) for _ in range(3)]
    for q, s in outs[1:]:
        assert torch.equal(q, outs[0][0]) and torch.equal(s, outs[0][1])


@pytest.mark.parametrize("dtype,tag", [(torch.float16, "f16"), (torch.bfloat16, "bf16"),
                                       (torch.float32, "f32")])
@pytest.mark.parametrize("shape", [(1, 8, 4096, 128), (2, 3, 777, 64), (1, 1, 5, 256),
                                   (1, 2, 70000, 64)])
def test_k_mean_bit_exact(device, dtype, tag, shape):
    k = (torch.randn(shape, device=device) * 2).to(dtype)
    m = _C.k_mean(k)
    raw = _np(k.view(torch.int16)).view(np.uint16) if tag == "bf16" else _np(k)
    np.testing.assert_array_equal(_np(m), oqn.k_mean(raw, tag))


@pytest.mark.parametrize("shape", [(1, 8, 512, 64), (1, 32, 333, 128), (2, 4, 257, 64)])
def test_quantize_qk_bit_exact(device, shape):
    B, H, S, D = shape
    q = torch.randn(B, H, S, D, device=device, dtype=torch.float16)
    k = torch.randn(B, max(1, H // 4), S + 5, D, device=device, dtype=torch.float16)
    k[..., 3] += 6.0  # channel outlier: smoothing must remove it identically
    q_i8, qs, k_i8, ks, km = quant.quantize_qk(q, k)
    rq, rqs, rk, rks, rm = oqn.quantize_qk(_np(q), _np(k))
    np.testing.assert_array_equal(_np(km), rm)
    np.testing.assert_array_equal(_np(q_i8), rq)
    np.testing.assert_array_equal(_np(qs)[..., 0], rqs)
    np.testing.assert_array_equal(_np(k_i8), rk)
    np.testing.assert_array_equal(_np(ks)[..., 0], rks)


def test_smooth_k_matches_oracle(device):
    k = torch.randn(1, 2, 300, 64, device=device, dtype=torch.float16)
    ks, km = quant.smooth_k(k)
    rks, rm = oqn.smooth_k(_np(k))
    np.testing.assert_array_equal(_np(ks.float()), rks)
    np.testing.assert_array_equal(_np(km), rm)

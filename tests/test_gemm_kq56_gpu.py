"""GPU parity of the Q5_K / Q6_K linears: dequant bit-exact against the oracle,
GEMM / GEMV against the oracle's exact integer sums (reference
tests/test_gemm_q4k.py:430-528)."""
import numpy as np
import pytest
import torch

import superl8_amd
from oracle import kquant as okq
from superl8_amd import _C
from tests.tolerances import assert_close_abs, assert_int8_quality

pytestmark = pytest.mark.gpu

FMT = {
    "q5k": (okq.q5k_random, okq.q5k_dequant, okq.q5k_gemv, okq.q5k_quantize,
            "gemm_q5k", "gemm_decode_q5k", "dequant_q5k", "linear_q5k", 176),
    "q6k": (okq.q6k_random, okq.q6k_dequant, okq.q6k_gemv, okq.q6k_quantize,
            "gemm_q6k", "gemm_decode_q6k", "dequant_q6k", "linear_q6k", 210),
}
RTOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2, torch.float32: 1e-5}


def _np(x):
    return x.detach().cpu().numpy()


def _case(fmt, M, N, K, seed, device):
    w = FMT[fmt][0](N, K, seed)
    r = np.random.default_rng(seed + 1)
    x = torch.from_numpy(r.standard_normal((M, K)).astype(np.float16)).to(device)
    return x, w, torch.from_numpy(w).to(device)


def _check_exact_sum(y, ref, odt):
    err = np.abs(_np(y.float()).astype(np.float64) - ref)
    scale = np.abs(ref).max()
    assert (err <= RTOL[odt] * np.abs(ref) + 1e-5 * scale).all(), f"max err {err.max():.3e}"


@pytest.mark.parametrize("fmt", ["q5k", "q6k"])
@pytest.mark.parametrize("N,K", [(64, 256), (130, 512), (33, 768), (4096, 5120)])
def test_dequant_bit_exact(device, fmt, N, K):
    w = FMT[fmt][0](N, K, N)
    got = getattr(_C, FMT[fmt][6])(torch.from_numpy(w).to(device), K)
    np.testing.assert_array_equal(_np(got), FMT[fmt][1](w, K))


TILE_SHAPES = [(17, 130, 512), (40, 256, 1024), (128, 128, 256), (300, 1000, 2048),
               (257, 17, 768), (512, 4864, 5120), (33, 129, 768), (1, 64, 256), (7, 128, 256)]


@pytest.mark.parametrize("odt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,K", TILE_SHAPES)
@pytest.mark.parametrize("fmt", ["q5k", "q6k"])
def test_tile_gemm_matches_exact_sum(device, fmt, M, N, K, odt):
    x, w, wd = _case(fmt, M, N, K, seed=M * 7 + N, device=device)
    x_i8, xs = _C.quantize_i8_rowwise(x)
    y = getattr(_C, FMT[fmt][4])(x_i8, xs, wd, odt)
    assert y.shape == (M, N) and y.dtype == odt
    _check_exact_sum(y, FMT[fmt][2](_np(x_i8), _np(xs), w, K), odt)


# at least one full round of 128 x 128 tiles on 256 CUs plus a short last
# round (260 and 258 tiles): the last tiles run as row quarters in a second
# launch; (257, 10890): the split tiles are the ragged last ones in M and N
SPLIT_SHAPES = [(160, 16635, 512), (257, 10890, 256)]


@pytest.mark.parametrize("M,N,K", SPLIT_SHAPES)
@pytest.mark.parametrize("fmt", ["q5k", "q6k"])
def test_tile_gemm_last_round_split(device, fmt, M, N, K):
    x, w, wd = _case(fmt, M, N, K, seed=M + N, device=device)
    x_i8, xs = _C.quantize_i8_rowwise(x)
    y = getattr(_C, FMT[fmt][4])(x_i8, xs, wd, torch.float32)
    xn, xsn = _np(x_i8), _np(xs)
    ref = np.concatenate([FMT[fmt][2](xn, xsn, w[n:n + 1024], K) for n in range(0, N, 1024)], axis=1)
    _check_exact_sum(y, ref, torch.float32)


@pytest.mark.parametrize("fmt", ["q5k", "q6k"])
def test_tile_quarters_bit_match_full_tiles(device, fmt):
    """The quarter tiles of the short last round (rows 128..159, columns 16128..
    at M = 160, N = 16635) match the same columns computed in full tiles bit
    for bit (same per-element operations in the same order)."""
    M, N, K, c0 = 160, 16635, 512, 126 * 128
    x, w, wd = _case(fmt, M, N, K, seed=31, device=device)
    x_i8, xs = _C.quantize_i8_rowwise(x)
    fn = getattr(_C, FMT[fmt][4])
    y = fn(x_i8, xs, wd, torch.float32)
    y_sub = fn(x_i8, xs, wd[c0:].contiguous(), torch.float32)
    assert torch.equal(y[:, c0:], y_sub)


DEC_SHAPES = [(1, 4096, 3072), (1, 130, 256), (2, 4096, 5120), (4, 512, 768), (8, 17408, 5120),
              (16, 1000, 2048), (3, 33, 768), (1, 64, 16384),
              # long K: the M >= 3 MFMA kernels loop over several super-block
              # chunks per wave (K > 5120 for Q5_K, K > 6144 for Q6_K)
              (3, 40, 17408), (8, 256, 17408), (16, 130, 12544), (9, 64, 8192), (12, 96, 6400)]


@pytest.mark.parametrize("odt", [torch.float16, torch.float32])
@pytest.mark.parametrize("M,N,K", DEC_SHAPES)
@pytest.mark.parametrize("fmt", ["q5k", "q6k"])
def test_decode_matches_exact_sum(device, fmt, M, N, K, odt):
    x, w, wd = _case(fmt, M, N, K, seed=M * 131 + N, device=device)
    x_i8, xs = _C.quantize_i8_rowwise(x)
    y = getattr(_C, FMT[fmt][5])(x_i8, xs, wd, odt)
    assert y.shape == (M, N) and y.dtype == odt
    _check_exact_sum(y, FMT[fmt][2](_np(x_i8), _np(xs), w, K), odt)


@pytest.mark.parametrize("fmt", ["q5k", "q6k"])
@pytest.mark.parametrize("m,n,k", [(1, 64, 256), (7, 128, 256), (64, 64, 512), (257, 128, 768),
                                   (33, 512, 1024), (5, 130, 256), (200, 96, 512)])
def test_reproduces_dequant_reference_encoder(device, fmt, m, n, k):
    """reference test_gemm_q4k.py:451-480: the fused op equals dequant -> matmul of the
    same native bytes made by the reference's own encoder."""
    torch.manual_seed(m * 17 + n)
    x = torch.randn(m, k, device=device, dtype=torch.float16)
    w = (np.random.default_rng(m + n).standard_normal((n, k)) * 0.1).astype(np.float32)
    blk, deq = FMT[fmt][3](w)
    x_i8, xs = _C.quantize_i8_rowwise(x)
    ref = (_np(x_i8).astype(np.float64) @ deq.astype(np.float64).T) * _np(xs)[:, None]
    y = getattr(_C, FMT[fmt][4])(x_i8, xs, torch.from_numpy(blk).to(device), torch.float16)
    assert_int8_quality(y, ref, min_cos=0.999, max_rel_l1=0.01, min_sqnr_db=40.0,
                        what=f"{fmt} dequant-exact {m}x{n}x{k}")


def test_error_ladder_vs_fp32(device):
    """reference test_gemm_q4k.py:482-496: Q6_K tighter than Q5_K against fp32."""
    torch.manual_seed(2)
    m, n, k = 128, 512, 1024
    x = torch.randn(m, k, device=device, dtype=torch.float16)
    w = (np.random.default_rng(2).standard_normal((n, k)) * 0.1).astype(np.float32)
    ref = _np(x.float()).astype(np.float64) @ w.astype(np.float64).T
    y5 = superl8_amd.linear_q5k(x, torch.from_numpy(okq.q5k_quantize(w)[0]).to(device))
    y6 = superl8_amd.linear_q6k(x, torch.from_numpy(okq.q6k_quantize(w)[0]).to(device))
    assert_int8_quality(y5, ref, min_cos=0.995, max_rel_l1=0.09, min_sqnr_db=24.0, what="q5k fp32")
    assert_int8_quality(y6, ref, min_cos=0.999, max_rel_l1=0.05, min_sqnr_db=30.0, what="q6k fp32")
    e5 = np.abs(_np(y5.float()) - ref).mean()
    e6 = np.abs(_np(y6.float()) - ref).mean()
    assert e6 < e5


@pytest.mark.parametrize("fmt", ["q5k", "q6k"])
def test_linear_routes_and_is_deterministic(device, fmt, monkeypatch):
    x, w, wd = _case(fmt, 1, 4096, 1024, seed=7, device=device)
    called = {}
    orig = getattr(_C, FMT[fmt][5])

    def spy(*a, **k):
        called["decode"] = True
        return orig(*a, **k)

    monkeypatch.setattr(_C, FMT[fmt][5], spy)
    lin = getattr(superl8_amd, FMT[fmt][7])
    y = lin(x, wd)
    assert called.get("decode")
    monkeypatch.undo()
    for _ in range(3):
        assert torch.equal(lin(x, wd), y)
    xt, _, _ = _case(fmt, 40, 4096, 1024, seed=8, device=device)
    yt = lin(xt, wd)
    y16 = getattr(_C, FMT[fmt][5])(*_C.quantize_i8_rowwise(xt[:16].contiguous()), wd)
    assert_close_abs(y16, _np(yt[:16].float()), atol=2e-3 * float(yt.abs().max()), rtol=2e-3,
                     what="decode vs tile")


@pytest.mark.parametrize("fmt", ["q5k", "q6k"])
def test_rejects(device, fmt):
    ts = FMT[fmt][8]
    x_i8 = torch.randint(-127, 128, (4, 128), device=device, dtype=torch.int8)
    xs = torch.ones(4, device=device)
    blk = torch.zeros(8, ts, device=device, dtype=torch.uint8)
    with pytest.raises(RuntimeError):
        getattr(_C, FMT[fmt][4])(x_i8, xs, blk, torch.float16)
    with pytest.raises(RuntimeError, match="M<=16"):
        getattr(_C, FMT[fmt][5])(torch.zeros(17, 256, device=device, dtype=torch.int8),
                                 torch.ones(17, device=device), blk)
    with pytest.raises(RuntimeError):  # wrong type size
        getattr(_C, FMT[fmt][4])(torch.zeros(2, 256, device=device, dtype=torch.int8),
                                 torch.ones(2, device=device),
                                 torch.zeros(8, 144, device=device, dtype=torch.uint8))

"""GPU parity of the Q4_K path: dequant bit-exact, GEMV vs the oracle's exact sum."""
import numpy as np
import pytest
import torch

import superl8_amd
from oracle import q4k as oq
from oracle import quant as oqn
from superl8_amd import _C
from tests.tolerances import assert_close_abs, assert_int8_quality

pytestmark = pytest.mark.gpu


def _np(x):
    return x.detach().cpu().numpy()


def _case(M, N, K, seed, device):
    w = oq.random_weights(N, K, seed)
    r = np.random.default_rng(seed + 1)
    x = torch.from_numpy(r.standard_normal((M, K)).astype(np.float16)).to(device)
    return x, w, torch.from_numpy(w).to(device)


@pytest.mark.parametrize("N,K", [(64, 256), (130, 512), (17408, 5120), (33, 4096)])
def test_dequant_bit_exact(device, N, K):
    w = oq.random_weights(N, K, seed=N)
    got = _C.dequant_q4k(torch.from_numpy(w).to(device), K)
    np.testing.assert_array_equal(_np(got), oq.dequant(w, K))


SHAPES = [(1, 4096, 3072), (1, 1024, 4096), (4, 4096, 4096), (8, 512, 768), (16, 4096, 3072),
          (1, 130, 256), (1, 4864, 1024), (1, 17408, 5120), (8, 17408, 5120), (5, 7, 256),
          (11, 96, 512),
          # M <= 2 (VALU path), partial and multi-chunk K splits
          (2, 4096, 3072), (2, 130, 256), (1, 64, 16384), (2, 50, 12544), (3, 40, 16384),
          # 5 <= M <= 8 (activation copies first): the K = 5120 straight-line
          # chunk with a ragged N, and several chunks per wave
          (6, 130, 5120), (6, 40, 16384), (8, 64, 12544)]


@pytest.mark.parametrize("odt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemv_matches_exact_sum(device, M, N, K, odt):
    x, w, wd = _case(M, N, K, seed=M * 131 + N, device=device)
    x_i8, xs = _C.quantize_i8_rowwise(x)
    y = _C.gemm_decode_q4k(x_i8, xs, wd, odt)
    assert y.shape == (M, N) and y.dtype == odt
    ref = oq.gemv(_np(x_i8), _np(xs), w, K)
    # one fp32 accumulation per super-block, then the output rounding of odt
    rtol = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2, torch.float32: 1e-5}[odt]
    err = np.abs(_np(y.float()).astype(np.float64) - ref)
    scale = np.abs(ref).max()
    assert (err <= rtol * np.abs(ref) + 1e-5 * scale).all(), f"max err {err.max():.3e}"
    assert_int8_quality(y, ref, min_cos=0.9999, max_rel_l1=1e-3 if odt != torch.bfloat16 else 1e-2,
                        min_sqnr_db=40.0)


XB_SHAPES = [(1, 17408, 5120), (8, 17408, 5120), (2, 130, 256), (3, 40, 16384), (16, 96, 512),
             (5, 64, 1024), (1, 64, 16384), (7, 48, 12288), (6, 130, 5120)]


@pytest.mark.parametrize("odt", [torch.float16, torch.float32])
@pytest.mark.parametrize("M,N,K", XB_SHAPES)
def test_gemv_block_scales_matches_exact_sum(device, M, N, K, odt):
    """BASELINE config 4's activation format: int8 per 256-element block with an
    fp32 scale each (x_scale [M, K/256]) against the oracle's exact sums."""
    x, w, wd = _case(M, N, K, seed=M * 17 + N, device=device)
    x[:, :256] *= 30  # blocks of one row at very different scales
    x_i8, xb = _C.quantize_i8_blockwise(x, 256)
    assert xb.shape == (M, K // 256)
    # the block quantiser is the row quantiser on each 256-slice: codes bit-exact
    rq, rs = oqn.quantize_rows(_np(x.float()).reshape(-1, 256))
    np.testing.assert_array_equal(_np(x_i8).reshape(-1, 256), rq)
    np.testing.assert_array_equal(_np(xb).reshape(-1), rs)
    y = _C.gemm_decode_q4k(x_i8, xb, wd, odt)
    ref = oq.gemv_xblock(_np(x_i8), _np(xb), w, K)
    rtol = {torch.float16: 2e-3, torch.float32: 1e-5}[odt]
    err = np.abs(_np(y.float()).astype(np.float64) - ref)
    assert (err <= rtol * np.abs(ref) + 1e-5 * np.abs(ref).max()).all(), f"max err {err.max():.3e}"


TILE_SHAPES = [(17, 130, 512), (40, 256, 1024), (128, 128, 256), (300, 1000, 2048),
               (257, 17, 768), (512, 4864, 5120)]


@pytest.mark.parametrize("odt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,K", TILE_SHAPES)
def test_tile_gemm_matches_exact_sum(device, M, N, K, odt):
    """M > 16: the tiled MFMA GEMM (exact integer sub-block sums, fp32 per super-block)."""
    x, w, wd = _case(M, N, K, seed=M * 7 + N, device=device)
    x_i8, xs = _C.quantize_i8_rowwise(x)
    y = _C.gemm_q4k(x_i8, xs, wd, odt)
    assert y.shape == (M, N) and y.dtype == odt
    ref = oq.gemv(_np(x_i8), _np(xs), w, K)
    rtol = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2, torch.float32: 1e-5}[odt]
    err = np.abs(_np(y.float()).astype(np.float64) - ref)
    scale = np.abs(ref).max()
    assert (err <= rtol * np.abs(ref) + 1e-5 * scale).all(), f"max err {err.max():.3e}"


# at least one full round of 128 x 128 tiles on 256 CUs plus a short last
# round (260 and 258 tiles): the last tiles run as row quarters in a second
# launch; (257, 10890): the split tiles are the ragged last ones in M and N
@pytest.mark.parametrize("M,N,K", [(160, 16635, 512), (257, 10890, 256)])
def test_tile_gemm_last_round_split(device, M, N, K):
    x, w, wd = _case(M, N, K, seed=M + N, device=device)
    x_i8, xs = _C.quantize_i8_rowwise(x)
    y = _C.gemm_q4k(x_i8, xs, wd, torch.float32)
    xn, xsn = _np(x_i8), _np(xs)
    ref = np.concatenate([oq.gemv(xn, xsn, w[n:n + 1024], K) for n in range(0, N, 1024)], axis=1)
    err = np.abs(_np(y).astype(np.float64) - ref)
    assert (err <= 1e-5 * np.abs(ref) + 1e-5 * np.abs(ref).max()).all(), f"max err {err.max():.3e}"


def test_tile_quarters_bit_match_full_tiles(device):
    """The last-round quarter launch applies the full tiles' per-element
    operations in the same order: at M = 160, N = 16635 (260 tiles in row-major
    order on 256 CUs) tiles 256..259 -- rows 128..159, columns 16128.. -- run as
    quarters; the same columns computed alone (130 full tiles over the sliced
    weights) must match them bit for bit."""
    M, N, K, c0 = 160, 16635, 512, 126 * 128
    x, w, wd = _case(M, N, K, seed=31, device=device)
    x_i8, xs = _C.quantize_i8_rowwise(x)
    y = _C.gemm_q4k(x_i8, xs, wd, torch.float32)
    y_sub = _C.gemm_q4k(x_i8, xs, wd[c0:].contiguous(), torch.float32)
    assert torch.equal(y[:, c0:], y_sub)


def test_tile_min_term_at_its_exactness_limits(device):
    """The min term's fp16 operands at their extremes: x rows of all +127 / all
    -127 / alternating signs per 16-element half (half-sums +-2032, the largest
    magnitude the fp16 operand must hold exactly), every scale and min 63, every
    nibble 15, d = dmin = 1: the tile GEMM (and the M <= 16 GEMV) against the
    oracle's exact sums."""
    M, N, K = 40, 256, 1024
    nsb = K // 256
    d = np.ones((N, nsb), np.float16)
    sc = np.full((N, nsb, 8), 63, np.uint8)
    q = np.full((N, nsb, 8, 32), 15, np.uint8)
    q[1::2, :, :, ::3] = 0                      # some rows not all-15
    w = oq.make_blocks(d, d, sc, sc.copy(), q).reshape(N, nsb * oq.TYPE_SIZE)
    x = np.empty((M, K), np.int8)
    x[0::3] = 127
    x[1::3] = -127
    x[2::3] = np.where((np.arange(K) // 16) % 2 == 0, 127, -127)
    xs = np.ones(M, np.float32)
    ref = oq.gemv(x, xs, w, K)
    xt, xst, wd = (torch.from_numpy(a).to(device) for a in (x, xs, w))
    y = _C.gemm_q4k(xt, xst, wd, torch.float32)
    err = np.abs(_np(y).astype(np.float64) - ref)
    assert (err <= 1e-6 * np.abs(ref).max()).all(), f"tile: max err {err.max():.3e}"
    y16 = _C.gemm_decode_q4k(xt[:16].contiguous(), xst[:16].contiguous(), wd, torch.float32)
    err = np.abs(_np(y16).astype(np.float64) - ref[:16])
    assert (err <= 1e-6 * np.abs(ref).max()).all(), f"gemv: max err {err.max():.3e}"


def test_tile_matches_decode_and_large_m(device):
    """reference test_gemm_q4k.py:715-728: the tile path and the decode path agree
    (to fp16 output rounding) on the rows they share."""
    x, w, wd = _case(40, 256, 1024, seed=5, device=device)
    x_i8, xs = _C.quantize_i8_rowwise(x)
    y = _C.gemm_q4k(x_i8, xs, wd)
    ref = oq.gemv(_np(x_i8), _np(xs), w, 1024)
    assert_int8_quality(y, ref, min_cos=0.9999, max_rel_l1=1e-3, min_sqnr_db=40.0)
    y16 = _C.gemm_decode_q4k(x_i8[:16].contiguous(), xs[:16].contiguous(), wd)
    assert_close_abs(y16, _np(y[:16].float()), atol=2e-3 * float(y.abs().max()), rtol=2e-3,
                     what="decode vs tile")


def test_linear_q4k_routes_decode_and_is_deterministic(device, monkeypatch):
    x, w, wd = _case(1, 4096, 1024, seed=7, device=device)
    called = {}
    orig = _C.gemm_decode_q4k

    def spy(*a, **k):
        called["decode"] = True
        return orig(*a, **k)

    monkeypatch.setattr(_C, "gemm_decode_q4k", spy)
    y = superl8_amd.linear_q4k(x, wd)
    assert called.get("decode")
    monkeypatch.undo()
    for _ in range(3):
        assert torch.equal(superl8_amd.linear_q4k(x, wd), y)
    bias = torch.randn(4096, device=device, dtype=torch.float16)
    yb = superl8_amd.linear_q4k(x, wd, bias=bias)
    assert torch.equal(yb, (y.float() + bias.float()).half())


def test_rejects_bad_k(device):
    x_i8 = torch.randint(-127, 128, (4, 128), device=device, dtype=torch.int8)
    xs = torch.ones(4, device=device)
    blk = torch.zeros(8, 144, device=device, dtype=torch.uint8)
    with pytest.raises(RuntimeError):
        _C.gemm_q4k(x_i8, xs, blk, torch.float16)
    with pytest.raises(RuntimeError, match="M<=16"):
        _C.gemm_decode_q4k(torch.zeros(17, 256, device=device, dtype=torch.int8),
                           torch.ones(17, device=device), blk[:, :144].contiguous())


@pytest.mark.parametrize("M", [1, 4])
def test_gemv_per_row_scale_shaped_m1(device, M):
    """A per-row x_scale shaped [M, 1] at K = 1024 is the reference's per-row scale
    (numel == M), not per-256-block scales: same result as x_scale [M]."""
    N, K = 96, 1024
    x, w, wd = _case(M, N, K, seed=M + 5, device=device)
    x_i8, xs = _C.quantize_i8_rowwise(x)
    y_flat = _C.gemm_decode_q4k(x_i8, xs, wd, torch.float32)
    y_col = _C.gemm_decode_q4k(x_i8, xs.reshape(M, 1).contiguous(), wd, torch.float32)
    assert torch.equal(y_flat, y_col)
    ref = oq.gemv(_np(x_i8), _np(xs), w, K)
    err = np.abs(_np(y_col).astype(np.float64) - ref)
    assert (err <= 1e-5 * np.abs(ref) + 1e-5 * np.abs(ref).max()).all()
    with pytest.raises(RuntimeError, match=r"\[M\] \(per row\) or \[M, K/256\]"):
        _C.gemm_decode_q4k(x_i8, torch.ones(M, 3, device=device), wd, torch.float32)

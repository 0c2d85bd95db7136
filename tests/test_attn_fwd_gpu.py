"""GPU parity of the prefill attention (attn_int8_fwd) against the oracle.

* int32 Q.K^T from the kernel's MFMA tiles: bit-exact.
* kernel output on identical int8 inputs vs the oracle's float64 softmax/PV:
  within the fp16-P rounding of the PV MFMA (cos >= 0.9999, rel-L1 <= 3e-3).
* end to end (prologue + kernel) vs fp32 attention on the original fp16
  inputs: the reference's int8 gate (cos >= 0.999, rel-L1 <= 0.02, 20 dB).
"""
import math

import numpy as np
import pytest
import torch

import superl8_amd as sl8
from oracle import attention as oa
from oracle import quant as oqn
from superl8_amd import _C, quant
from tests.tolerances import assert_close_abs, assert_finite, assert_int8_quality

pytestmark = pytest.mark.gpu


def _np(x):
    return x.detach().cpu().numpy()


def _qkv(B, Hq, Hkv, M, N, D, device, dtype=torch.float16):
    q = torch.randn(B, Hq, M, D, device=device, dtype=dtype)
    k = torch.randn(B, Hkv, N, D, device=device, dtype=dtype)
    v = torch.randn(B, Hkv, N, D, device=device, dtype=dtype)
    return q, k, v


def _v_f32(v):
    if v.dtype == torch.bfloat16:
        return oqn.bf16_bits_to_f32(_np(v.view(torch.int16)).view(np.uint16))
    return _np(v.float())


def _fp32_oracle(q, k, v, causal=False):
    """reference tests/reference.py:26-54 (fp32 einsum attention, bottom-right causal)."""
    return oa.attention_fp64(_np(q.float()), _np(k.float()), _np(v.float()), causal)


QK_SHAPES = [  # B, Hq, Hkv, M, N, D: every head dim, ragged M/N, GQA
    (1, 2, 2, 128, 128, 64), (2, 4, 2, 257, 300, 64), (1, 4, 1, 1, 77, 128),
    (1, 2, 2, 333, 129, 128), (1, 8, 8, 64, 1, 64), (1, 4, 2, 200, 190, 32),
    (2, 6, 3, 130, 97, 72), (1, 4, 1, 65, 513, 80), (1, 4, 2, 300, 333, 256),
    (1, 8, 2, 1000, 1031, 128)]
NOT_STORED = -(2 ** 31)  # |int32 score| <= 256 * 127^2, so this is never a real score


def _check_scores(s, q_i8, k_i8, causal, heads=None):
    """Every stored score equals the exact integer Q.K^T, and (causal) every
    score the mask lets through was stored."""
    s, q_i8, k_i8 = _np(s), _np(q_i8), _np(k_i8)
    Hq, M, N = s.shape[1], s.shape[2], s.shape[3]
    gsz = Hq // k_i8.shape[1]
    for h in (range(Hq) if heads is None else heads):
        exact = oa.scores_i32(q_i8[:, h:h + 1], k_i8[:, h // gsz:h // gsz + 1])
        got = s[:, h:h + 1]
        if not causal:
            np.testing.assert_array_equal(got, exact, err_msg=f"head {h}")
            continue
        stored = got != NOT_STORED
        np.testing.assert_array_equal(got[stored], exact[stored], err_msg=f"head {h}")
        vis = np.broadcast_to(oa.valid_mask(M, N, True), got.shape)
        assert stored[vis].all(), f"head {h}: visible scores not computed"


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", QK_SHAPES)
def test_qk_scores_bit_exact(device, shape, causal):
    """int32 S from the production kernel (attn_fwd_wide_kernel's dump
    instantiation) against the exact integer product (reference
    attn_int8_fwd.cuh:127-138: dp4a int32 accumulation)."""
    B, Hq, Hkv, M, N, D = shape
    q = torch.randint(-127, 128, (B, Hq, M, D), device=device, dtype=torch.int8)
    k = torch.randint(-127, 128, (B, Hkv, N, D), device=device, dtype=torch.int8)
    s = _C.attn_int8_qk_scores(q, k, causal=causal, fill=NOT_STORED)
    _check_scores(s, q, k, causal)


def test_qk_scores_extreme_codes(device):
    """All codes +-127 (the largest |sum| = D * 127^2) at D = 256 and 128."""
    for D in (128, 256):
        q = torch.full((1, 2, 70, D), 127, device=device, dtype=torch.int8)
        k = torch.full((1, 1, 90, D), -127, device=device, dtype=torch.int8)
        q[0, 1, ::2] = -127
        s = _C.attn_int8_qk_scores(q, k)
        _check_scores(s, q, k, False)
        assert int(s.abs().max()) == D * 127 * 127


def test_qk_scores_config2_head_subset(device):
    """BASELINE config 2 (B1 Hq32 Hkv8 S4096 D128 causal) on 8 query heads (two
    KV heads), K quantised with smoothing as the path does: bit-exact."""
    torch.manual_seed(2)
    q = torch.randn(1, 8, 4096, 128, device=device, dtype=torch.float16)
    k = torch.randn(1, 2, 4096, 128, device=device, dtype=torch.float16)
    q_i8, _, k_i8, _, _ = quant.quantize_qk(q, k)
    s = _C.attn_int8_qk_scores(q_i8, k_i8, causal=True, fill=NOT_STORED)
    _check_scores(s, q_i8, k_i8, True, heads=(0, 3, 4, 7))


KERNEL_CASES = [
    # B, Hq, Hkv, M, N, D, causal, window
    (1, 2, 2, 128, 128, 64, False, -1),
    (1, 2, 2, 128, 128, 64, True, -1),
    (2, 4, 2, 257, 257, 64, True, -1),
    (1, 4, 1, 100, 333, 128, True, -1),     # rectangular causal, MQA
    (1, 2, 2, 333, 333, 128, False, -1),
    (1, 4, 2, 200, 260, 64, True, 50),      # sliding window
    (1, 2, 2, 64, 64, 128, False, 16),      # window without causal
    (1, 2, 1, 5, 9, 64, True, 0),           # window 0: every row fully masked
    (1, 2, 2, 300, 40, 64, True, -1),       # M > N: leading rows see nothing
    (1, 2, 1, 200, 200, 256, True, -1),     # head dim 256 (one wave per SIMD)
    (1, 2, 2, 70, 90, 256, False, 20),
    # head dims 32/72/80 (reference attn_int8_fwd.cu:138; zero-padded to 64/128)
    (2, 8, 2, 257, 257, 72, True, -1), (2, 8, 2, 257, 257, 80, False, -1),
    (1, 4, 1, 100, 333, 32, True, -1), (1, 2, 2, 130, 130, 32, False, 24),
    (1, 4, 2, 200, 260, 80, True, 50),
]


@pytest.mark.parametrize("case", KERNEL_CASES)
@pytest.mark.parametrize("vdt", [torch.float16, torch.bfloat16])
def test_kernel_matches_oracle(device, case, vdt):
    B, Hq, Hkv, M, N, D, causal, wl = case
    q, k, v = _qkv(B, Hq, Hkv, M, N, D, device)
    v = v.to(vdt)
    q_i8, qs, k_i8, ks, _ = quant.quantize_qk(q, k)
    qs, ks = qs.squeeze(-1).contiguous(), ks.squeeze(-1).contiguous()
    out, lse = _C.attn_int8_fwd_train(q_i8, qs, k_i8, ks, v, causal) if wl < 0 else (
        _C.attn_int8_fwd(q_i8, qs, k_i8, ks, v, causal, wl), None)
    assert out.dtype == vdt and out.shape == (B, Hq, M, D)
    ref, ref_lse = oa.attn_int8_fwd(_np(q_i8), _np(qs), _np(k_i8), _np(ks), _v_f32(v), causal, wl)
    assert_finite(out)
    tol = 1e-2 if vdt == torch.float16 else 4e-2
    assert_close_abs(out, ref, atol=tol, what="attn_int8_fwd vs oracle")
    if np.abs(ref).sum() > 0:
        assert_int8_quality(out, ref, min_cos=0.9999 if vdt == torch.float16 else 0.999,
                            max_rel_l1=3e-3 if vdt == torch.float16 else 1e-2, min_sqnr_db=40)
    else:
        assert not out.float().abs().sum().item()
    if lse is not None:
        finite = np.isfinite(ref_lse)
        np.testing.assert_array_equal(np.isfinite(_np(lse)), finite)
        # l sums the fp16/bf16-rounded P that enters the PV product (the oracle sums
        # fp32 P): |dLSE| up to the relative P rounding (2^-11 fp16, 2^-8 bf16),
        # undamped on rows with few keys
        lse_tol = 5e-4 if vdt == torch.float16 else 4e-3
        np.testing.assert_allclose(_np(lse)[finite], ref_lse[finite], rtol=0, atol=lse_tol)


SHAPES = [(1, 2, 128, 64), (2, 4, 512, 64), (2, 4, 257, 64), (1, 2, 333, 128),
          (1, 8, 2048, 64), (1, 8, 2048, 128), (2, 4, 257, 32), (1, 4, 513, 72), (1, 4, 300, 80)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_end_to_end_quality(device, shape, causal):
    """reference tests/test_attn_fwd.py:44-51."""
    b, h, m, d = shape
    q, k, v = _qkv(b, h, h, m, m, d, device)
    out = sl8.attn_int8_fwd(q, k, v, causal=causal)
    assert out.shape == q.shape and out.dtype == torch.float16
    assert_int8_quality(out, _fp32_oracle(q, k, v, causal), what=f"{shape} causal={causal}")


def test_gqa_rectangular_and_bf16(device):
    q, k, v = _qkv(1, 8, 2, 96, 300, 128, device)
    out = sl8.attn_int8_fwd(q, k, v, causal=True)
    assert_int8_quality(out, _fp32_oracle(q, k, v, True), what="gqa rectangular")
    qb, kb, vb = q.bfloat16(), k.bfloat16(), v.bfloat16()
    outb = sl8.attn_int8_fwd(qb, kb, vb, causal=True)
    assert outb.dtype == torch.bfloat16
    assert_int8_quality(outb, _fp32_oracle(qb, kb, vb, True), what="bf16")


def test_outlier_k_and_peaked_softmax(device):
    """reference tests/test_attn_fwd.py:55-104."""
    q, k, v = _qkv(2, 4, 4, 512, 512, 64, device)
    k = k.clone()
    k[..., 13] += 8.0
    assert_int8_quality(sl8.attn_int8_fwd(q, k, v), _fp32_oracle(q, k, v), what="outlier-K")
    q = torch.randn(1, 4, 256, 64, device=device, dtype=torch.float16)
    k = torch.randn(1, 4, 256, 64, device=device, dtype=torch.float16) * 0.1
    v = torch.randn(1, 4, 256, 64, device=device, dtype=torch.float16)
    k[:, :, 0] += 4.0
    k[:, :, 1] += 3.98
    assert_int8_quality(sl8.attn_int8_fwd(q, k, v), _fp32_oracle(q, k, v), what="near-tie")


def test_deterministic_and_rejects(device):
    q, k, v = _qkv(2, 4, 4, 512, 512, 64, device)
    r0 = sl8.attn_int8_fwd(q, k, v)
    for _ in range(3):
        assert torch.equal(sl8.attn_int8_fwd(q, k, v), r0)
    q, k, v = _qkv(1, 2, 2, 128, 128, 96, device)
    with pytest.raises(RuntimeError, match="32/64/72/80/128/256"):
        sl8.attn_int8_fwd(q, k, v)
    q8 = torch.zeros(1, 2, 8, 64, device=device, dtype=torch.int8)
    s = torch.ones(1, 2, 8, device=device)
    with pytest.raises(RuntimeError, match="float16|bfloat16"):
        _C.attn_int8_fwd(q8, s, q8, s, torch.zeros(1, 2, 8, 64, device=device))


@pytest.mark.parametrize("d", [72, 80])
def test_odd_head_dim_deterministic(device, d):
    """reference tests/test_odd_dims.py:30-36."""
    q, k, v = (torch.randn(1, 4, 200, d, device=device, dtype=torch.float16) for _ in range(3))
    r0 = sl8.attn_int8_fwd(q, k, v)
    assert r0.shape == q.shape
    for _ in range(3):
        assert torch.equal(sl8.attn_int8_fwd(q, k, v), r0)


@pytest.mark.parametrize("d", [32, 72, 80])
@pytest.mark.parametrize("causal", [False, True])
def test_odd_head_dim_gqa_quality(device, d, causal):
    """reference tests/test_odd_dims.py:14-27 (ragged M, GQA) against fp attention."""
    q, k, v = _qkv(2, 8, 2, 257, 257, d, device)
    out = sl8.attn_int8_fwd(q, k, v, causal=causal)
    assert out.shape == q.shape
    assert_int8_quality(out, _fp32_oracle(q, k, v, causal), what=f"odd-dim D={d} causal={causal}")


def test_accuracy_gate_and_rotate(device, monkeypatch):
    """Gate: an outlier-dominated Q row routes to full precision (reference ops.py:115-147);
    internal_accuracy_gate=False skips the detector; rotate=True keeps quality."""
    q, k, v = _qkv(1, 4, 4, 257, 257, 128, device)
    out = sl8.attn_int8_fwd(q, k, v, rotate=True, internal_accuracy_gate=False)
    assert_int8_quality(out, _fp32_oracle(q, k, v), what="rotate")
    q2 = q.clone()
    q2[0, 0, 5, 7] = 500.0
    called = {}
    orig = _C.attn_int8_fwd
    monkeypatch.setattr(_C, "attn_int8_fwd",
                        lambda *a, **kw: called.setdefault("x", (kw.get("gate_flag"), orig(*a, **kw))))
    out2 = sl8.attn_int8_fwd(q2, k, v)
    # the int8 kernel is either not launched or launched gated on the device
    # flag (then it exits at once and its output is discarded)
    assert "x" not in called or called["x"][0] is not None
    assert_int8_quality(out2, _fp32_oracle(q2, k, v), min_cos=0.9999, what="gate fallback")


def test_config2_shape_against_oracle(device):
    """BASELINE config 2 (B1 Hq32 Hkv8 S4096 D128 causal), every one of the 32
    query heads against the oracle (~1 s of numpy per head)."""
    torch.manual_seed(2)
    q, k, v = _qkv(1, 32, 8, 4096, 4096, 128, device)
    q_i8, qs, k_i8, ks, _ = quant.quantize_qk(q, k)
    qs, ks = qs.squeeze(-1).contiguous(), ks.squeeze(-1).contiguous()
    out = _C.attn_int8_fwd(q_i8, qs, k_i8, ks, v, True)
    for h in range(32):
        kvh = h // 4
        ref, _ = oa.attn_int8_fwd(_np(q_i8[:, h:h + 1]), _np(qs[:, h:h + 1]),
                                  _np(k_i8[:, kvh:kvh + 1]), _np(ks[:, kvh:kvh + 1]),
                                  _np(v[:, kvh:kvh + 1].float()), True)
        assert_close_abs(out[:, h:h + 1], ref, atol=1e-2, what=f"config2 head {h}")
        assert_int8_quality(out[:, h:h + 1], ref, min_cos=0.9999, max_rel_l1=3e-3, min_sqnr_db=40,
                            what=f"config2 head {h}")


@pytest.mark.parametrize("causal", [False, True])
def test_reference_point_restart(device, causal):
    """Logits of later key tiles exceed the first tile's maximum by far more than
    the kernel's fixed-reference headroom (2^15), which forces the second run of
    the pass with the row maximum; results must still match the oracle."""
    B, Hq, Hkv, M, N, D = 1, 2, 2, 192, 320, 128
    g = torch.Generator(device="cpu").manual_seed(7)
    q_i8 = torch.randint(-127, 128, (B, Hq, M, D), generator=g, dtype=torch.int8)
    k_i8 = torch.randint(-127, 128, (B, Hkv, N, D), generator=g, dtype=torch.int8)
    qs = torch.full((B, Hq, M), 1.0 / (127.0 * 127.0 * np.sqrt(D) / 3.0), dtype=torch.float32)
    ks = torch.full((B, Hkv, N), 12.0, dtype=torch.float32)
    ks[..., :64] = 1e-3  # the first tile is nearly flat
    v = torch.randn(B, Hkv, N, D, generator=g).to(torch.float16)
    out, lse = _C.attn_int8_fwd_train(q_i8.to(device), qs.to(device), k_i8.to(device),
                                      ks.to(device), v.to(device), causal)
    ref, ref_lse = oa.attn_int8_fwd(_np(q_i8), _np(qs), _np(k_i8), _np(ks), _v_f32(v), causal, -1)
    assert_finite(out)
    assert_close_abs(out, ref, atol=1e-2, what="restart path vs oracle")
    finite = np.isfinite(ref_lse)
    np.testing.assert_allclose(_np(lse)[finite], ref_lse[finite], rtol=0, atol=5e-4)


@pytest.mark.parametrize("qv,kv", [(127, 127), (-128, -128), (-128, 127)])
def test_seeded_accumulator_extreme_codes(device, qv, kv):
    """The D = 128 straight-line path reads the QK accumulator seeded with the
    bits of 1/(2 pi) as a float; it is exact for |acc| <= 2,292,099 and the
    largest int8 sums (128 * 128^2 = 2,097,152 for codes -128) stay inside. Rows
    of constant codes with a few flipped keys: every score is +-|acc|max or
    close to it, so a wrong binade or a lost seed shows in the softmax."""
    B, Hq, Hkv, M, N, D = 1, 2, 1, 256, 320, 128
    q = torch.full((B, Hq, M, D), qv, device=device, dtype=torch.int8)
    k = torch.full((B, Hkv, N, D), kv, device=device, dtype=torch.int8)
    k[:, :, 5::7, :40] = 0  # some keys with smaller |score|
    q[:, 1, :, 64:] = 1
    qs = torch.full((B, Hq, M), 2e-6, device=device)  # logits ~ +-4 log2 units
    ks = torch.rand(B, Hkv, N, device=device) + 0.5
    v = torch.randn(B, Hkv, N, D, device=device, dtype=torch.float16)
    for causal in (False, True):
        out = _C.attn_int8_fwd(q, qs, k, ks, v, causal)
        ref, _ = oa.attn_int8_fwd(_np(q), _np(qs), _np(k), _np(ks), _np(v.float()), causal)
        assert_close_abs(out, ref, atol=1e-2, what=f"codes {qv}/{kv} causal={causal}")
        s = _C.attn_int8_qk_scores(q, k)
        _check_scores(s, q, k, False)


def _waves_for(B, Hq, M, D, causal, cus=256):
    """The workgroup size the launcher picks (waves of 32 queries): the default
    (8 for D = 128, 4 for D = 64) halved while the grid is below the CU count."""
    wv = 8 if D == 128 else 4
    while wv > 2:
        nqb = -(-M // (32 * wv))
        if B * Hq * ((nqb + 1) // 2 if causal else nqb) >= cus:
            break
        wv //= 2
    return wv


# small grids run 2- or 4-wave workgroups: each wave count and dtype against the oracle
WAVE_CASES = [
    (1, 32, 8, 1024, 1024, 128, True),   # 2 waves
    (1, 32, 8, 2048, 2048, 128, True),   # 4 waves
    (1, 32, 8, 1024, 1024, 128, False),  # 4 waves
    (1, 32, 8, 1024, 1024, 64, True),    # 2 waves
    (2, 8, 8, 1000, 1000, 128, True),    # 2 waves, ragged last block
    (1, 32, 8, 300, 1000, 128, True),    # 2 waves, bottom-right causal offset
]


@pytest.mark.parametrize("vdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", WAVE_CASES, ids=lambda c: "B%dH%d_%dS%dx%dD%d%s" % (*c[:6], "c" if c[6] else ""))
def test_small_grid_wave_counts(device, case, vdt):
    """Output (fp16 and bf16 V) and LSE (the train entry) against the oracle."""
    B, Hq, Hkv, M, N, D, causal = case
    torch.manual_seed(M + D)
    if torch.cuda.get_device_properties(device).multi_processor_count == 256:
        assert _waves_for(B, Hq, M, D, causal) in (2, 4)
    q, k, v = _qkv(B, Hq, Hkv, M, N, D, device)
    v = v.to(vdt)
    q_i8, qs, k_i8, ks, _ = quant.quantize_qk(q, k)
    qs, ks = qs.squeeze(-1).contiguous(), ks.squeeze(-1).contiguous()
    out = _C.attn_int8_fwd(q_i8, qs, k_i8, ks, v, causal)
    out_t, lse = _C.attn_int8_fwd_train(q_i8, qs, k_i8, ks, v, causal)
    assert_finite(out)
    assert torch.equal(out, out_t)
    gsz = Hq // Hkv
    f16 = vdt == torch.float16
    for b, h in [(0, 0), (B - 1, Hq - 1), (B - 1, Hq // 2 + 1)]:
        kvh = h // gsz
        ref, ref_lse = oa.attn_int8_fwd(_np(q_i8[b:b + 1, h:h + 1]), _np(qs[b:b + 1, h:h + 1]),
                                        _np(k_i8[b:b + 1, kvh:kvh + 1]), _np(ks[b:b + 1, kvh:kvh + 1]),
                                        _v_f32(v[b:b + 1, kvh:kvh + 1]), causal)
        got = out[b:b + 1, h:h + 1]
        assert_close_abs(got, ref, atol=1e-2 if f16 else 4e-2, what=f"{case} head {(b, h)}")
        assert_int8_quality(got, ref, min_cos=0.9999 if f16 else 0.999,
                            max_rel_l1=3e-3 if f16 else 1e-2, min_sqnr_db=40, what=f"{case} head {(b, h)}")
        # tolerance as test_kernel_matches_oracle: the P rounding of the PV operand
        np.testing.assert_allclose(_np(lse[b:b + 1, h:h + 1]), ref_lse, rtol=0,
                                   atol=5e-4 if f16 else 4e-3)

"""Pins the CPU oracle (oracle/) before it is trusted as the GPU checker.

Each oracle function is checked against something other than its own
formula: known answers from the reference's tests, closed forms, brute-force
loops on tiny inputs, invariants, and an independent textbook formulation.
The plausible mistakes each test would catch are named in its docstring.
"""
import math

import numpy as np
import pytest

from oracle import attention as oa
from oracle import kquant as okq
from oracle import q4k as oq
from oracle import quant as oqn
from tests.tolerances import assert_int8_quality

RNG = np.random.default_rng(1234)


# ---------------------------------------------------------------- quantisation
def test_quant_zero_and_outlier_rows():
    """Reference test_quant_rowwise.py:75-86: zero row -> scale 1 and codes 0;
    a single outlier sets the scale and quantises to 127."""
    x = np.zeros((3, 128), np.float16)
    x[1, 40] = 50.0
    q, s = oqn.quantize_rows(x.astype(np.float32))
    assert s[0] == 1.0 and not q[0].any()
    assert s[1] == np.float32(np.float32(50.0) * np.float32(1 / np.float32(127)))
    assert q[1, 40] == 127 and np.count_nonzero(q[1]) == 1
    assert not q[2].any() and s[2] == 1.0


def test_quant_scale_is_reciprocal_multiply():
    """scale = amax * fp32(1/127) (quant_rowwise.cuh:33-38), not amax/127.
    Rows are chosen where the two differ, so a true-division oracle fails."""
    amax = np.arange(1, 30000, dtype=np.float32).astype(np.float16).astype(np.float32) / 64
    mul = (amax * oqn.INV127).astype(np.float32)
    div = (amax / np.float32(127)).astype(np.float32)
    differ = amax[mul != div][:64]
    assert differ.size > 10
    x = np.zeros((differ.size, 8), np.float32)
    x[:, 3] = differ
    _, s = oqn.quantize_rows(x)
    np.testing.assert_array_equal(s, (differ * oqn.INV127).astype(np.float32))
    assert (s != (differ / np.float32(127))).all()


def test_quant_rounding_brute_force():
    """Codes satisfy |x/s - q| <= 0.5 with ties to even, clamp at +-127 (never -128)."""
    x = (RNG.standard_normal((64, 96)) * 3).astype(np.float16).astype(np.float32)
    q, s = oqn.quantize_rows(x)
    quo = (x / s[:, None]).astype(np.float32).astype(np.float64)
    assert np.all(np.abs(quo - q) <= 0.5)
    tie = np.abs(quo - np.trunc(quo)) == 0.5
    assert np.all(q[tie] % 2 == 0)
    assert q.min() >= -127 and q.max() <= 127
    # explicit half-way case: s a power of two so (k + 0.5) * s divides exactly
    row = np.zeros((1, 8), np.float32)
    row[0, 0] = np.float32(127.0)  # amax 127
    s0 = oqn.quantize_rows(row)[1][0]
    ties = [np.float32(k + 0.5) * s0 for k in (2, 3, -2, -5)]
    if all(np.float32(t) / s0 == np.float32(k + 0.5) for t, k in zip(ties, (2, 3, -2, -5))):
        row[0, 1:5] = ties
        q1 = oqn.quantize_rows(row)[0][0]
        assert list(q1[1:5]) == [2, 4, -2, -4]


def test_quant_row_groups_pins():
    """Group quantiser: one row per group is the row quantiser; a group's scale is
    its largest row amax (brute force); codes use the group scale."""
    x = (RNG.standard_normal((2, 70, 24)) * RNG.random((2, 70, 1)) * 4).astype(np.float32)
    q1, s1 = oqn.quantize_row_groups(x, 1, 0.5)
    qr, sr = oqn.quantize_rows(x, 0.5)
    np.testing.assert_array_equal(q1, qr)
    np.testing.assert_array_equal(s1, sr)
    q, s = oqn.quantize_row_groups(x, 32)
    for b in range(2):
        for r0 in (0, 32, 64):
            blk = x[b, r0:r0 + 32]
            sc = np.float32(np.abs(blk).max()) * oqn.INV127
            assert (s[b, r0:r0 + 32] == sc).all()
            np.testing.assert_array_equal(
                q[b, r0:r0 + 32], np.clip(np.rint(blk / sc), -127, 127).astype(np.int8))
    assert s[0, 64:].shape == (6,)  # short last group


def test_k_mean_exact_and_order_free():
    """fp16 mean: exact sum, so equal to the float64 mean rounded once, and
    invariant under any key permutation (catches a plain fp32 running sum)."""
    k = (RNG.standard_normal((2, 3, 2000, 64)) * 4).astype(np.float16)
    m = oqn.k_mean(k, "f16")
    ref = k.astype(np.float64).mean(axis=-2, keepdims=True)
    np.testing.assert_array_equal(m, ref.astype(np.float32))
    perm = RNG.permutation(2000)
    np.testing.assert_array_equal(m, oqn.k_mean(k[:, :, perm], "f16"))
    const = np.full((1, 1, 777, 8), 0.3, np.float16)
    np.testing.assert_array_equal(oqn.k_mean(const, "f16"), np.float16(0.3).astype(np.float32))


def test_k_mean_bf16_and_smooth():
    bits = oqn.f32_to_bf16_bits(RNG.standard_normal((1, 2, 300, 16)).astype(np.float32))
    m = oqn.k_mean(bits, "bf16")
    ref = oqn.bf16_bits_to_f32(bits).astype(np.float64).mean(axis=-2, keepdims=True)
    assert np.abs(m - ref).max() <= np.spacing(np.abs(ref).astype(np.float32)).max()
    k = (RNG.standard_normal((1, 1, 50, 8))).astype(np.float16)
    ks, mean = oqn.smooth_k(k, "f16")
    for n, d in [(0, 0), (7, 3), (49, 7)]:
        want = float(np.float16(np.float32(k[0, 0, n, d]) - mean[0, 0, 0, d]))
        assert ks[0, 0, n, d] == want


def test_bf16_rounding_helpers():
    vals = np.array([1.0, 1.00390625, 1.01171875, -3.0e38, 1e-40], np.float32)
    bits = oqn.f32_to_bf16_bits(vals)
    # 1 + 2^-8 is a tie between 1 and 1+2^-7 -> even (1.0); 1+3*2^-8 -> 1+2^-6
    assert bits[0] == 0x3F80 and bits[1] == 0x3F80 and bits[2] == 0x3F82


def test_quantize_qk_fold():
    """q_scale = safe * fp32(softmax_scale*log2 e) (core.py:195)."""
    q = RNG.standard_normal((1, 2, 5, 64)).astype(np.float16)
    k = RNG.standard_normal((1, 2, 7, 64)).astype(np.float16)
    q_i8, qs, k_i8, ks, _ = oqn.quantize_qk(q, k)
    _, safe = oqn.quantize_rows(q.astype(np.float32))
    fold = np.float32(1.0 / math.sqrt(64) * math.log2(math.e))
    np.testing.assert_array_equal(qs, (safe * fold).astype(np.float32))


# ---------------------------------------------------------------- Q4_K
def _scale_min_literal(s, j):
    """get_scale_min_k4 as a per-byte scalar routine (llama.cpp convert.cu form)."""
    if j < 4:
        return s[j] & 63, s[j + 4] & 63
    return (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4), (s[j + 4] >> 4) | ((s[j] >> 6) << 4)


def test_q4k_scale_min_matches_literal_and_roundtrips():
    s12 = RNG.integers(0, 256, (500, 12), dtype=np.uint8)
    sc, mn = oq.scale_min_k4(s12)
    for r in range(0, 500, 37):
        for j in range(8):
            assert (sc[r, j], mn[r, j]) == _scale_min_literal([int(b) for b in s12[r]], j)
    a = np.arange(64, dtype=np.uint8)
    sc_all = np.stack(np.meshgrid(a, a, indexing="ij"), -1).reshape(-1, 2)  # all (sc,m) pairs
    sc8 = np.repeat(sc_all[:, :1], 8, 1)
    mn8 = np.repeat(sc_all[:, 1:], 8, 1)
    sc8[:, 3], mn8[:, 6] = sc_all[::-1, 0], sc_all[::-1, 1]
    back = oq.scale_min_k4(oq.pack_scale_min_k4(sc8, mn8))
    np.testing.assert_array_equal(back[0], sc8)
    np.testing.assert_array_equal(back[1], mn8)


def test_q4k_dequant_known_answer():
    """d=1, dmin=0.5, sc_j=j+1, m_j=2j, q[j][l]=(l+j)%16 -> w = (j+1)*q - j."""
    j = np.arange(8)
    q = (np.arange(32)[None, :] + j[:, None]) % 16
    blk = oq.make_blocks(np.array([1.0]), np.array([0.5]), (j + 1)[None], (2 * j)[None], q[None])
    w = oq.dequant(blk, 256)[0].reshape(8, 32)
    np.testing.assert_array_equal(w, ((j[:, None] + 1) * q - j[:, None]).astype(np.float32))


def test_q4k_nibble_positions():
    """Byte 32g+l: low nibble -> element 64g+l, high nibble -> element 64g+32+l
    (gemm_decode_dp4a.cuh:502-503). Catches swapped halves / interleave."""
    blk = oq.make_blocks(np.array([1.0]), np.array([0.0]), np.ones((1, 8), np.uint8),
                         np.zeros((1, 8), np.uint8), np.zeros((1, 8, 32), np.uint8))
    blk[0, 16 + 32 * 2 + 5] = 0x93  # g=2, l=5: low 3, high 9
    w = oq.dequant(blk, 256)[0]
    nz = np.nonzero(w)[0]
    assert list(nz) == [64 * 2 + 5, 64 * 2 + 32 + 5]
    assert w[133] == 3 and w[165] == 9


def test_q4k_gemv_matches_dequant_matmul():
    w = oq.random_weights(40, 512, seed=3)
    x = RNG.integers(-127, 128, (5, 512), dtype=np.int8)
    xs = RNG.random(5).astype(np.float32)
    y = oq.gemv(x, xs, w, 512)
    ref = (x.astype(np.float64) @ oq.dequant(w, 512).astype(np.float64).T) * xs[:, None]
    # dequant rounds d*sc*q - dmin*m to fp32 once; the oracle sums exactly
    np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-6)


def test_q4k_gemv_xblock_pins():
    """Per-256-block activation scales: equals the dequantised matmul with x
    scaled per block, and reduces to gemv() when each row's blocks share one scale."""
    w = oq.random_weights(24, 768, seed=5)
    x = RNG.integers(-127, 128, (3, 768), dtype=np.int8)
    xb = (RNG.random((3, 3)) + 0.1).astype(np.float32)
    y = oq.gemv_xblock(x, xb, w, 768)
    xf = x.astype(np.float64) * np.repeat(xb.astype(np.float64), 256, axis=1)
    ref = xf @ oq.dequant(w, 768).astype(np.float64).T
    np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-6)
    row = xb[:, :1]
    np.testing.assert_allclose(oq.gemv_xblock(x, np.repeat(row, 3, axis=1), w, 768),
                               oq.gemv(x, row[:, 0], w, 768), rtol=1e-12, atol=1e-9)
    # a wrong block-to-scale pairing (scales reversed) is caught
    assert np.abs(oq.gemv_xblock(x, xb[:, ::-1].copy(), w, 768) - ref).max() > 1e-3


# ---------------------------------------------------------------- Q5_K / Q6_K
def _q5k_dequant_literal(blk):
    """dequantize_row_q5_K as a scalar loop over one 176-byte block (llama.cpp
    ggml-quants.c form: pairs of sub-blocks, qh bit masks u1/u2 shifted by 2)."""
    d = float(np.frombuffer(blk[0:2].tobytes(), np.float16)[0])
    dmin = float(np.frombuffer(blk[2:4].tobytes(), np.float16)[0])
    s = [int(b) for b in blk[4:16]]
    qh, ql = blk[16:48], blk[48:176]
    y, u1, u2, is_ = [], 1, 2, 0
    for g in range(4):
        sc1, m1 = _scale_min_literal(s, is_)
        sc2, m2 = _scale_min_literal(s, is_ + 1)
        d1, mm1 = np.float32(d) * np.float32(sc1), np.float32(dmin) * np.float32(m1)
        d2, mm2 = np.float32(d) * np.float32(sc2), np.float32(dmin) * np.float32(m2)
        for l in range(32):
            y.append(d1 * np.float32((ql[32 * g + l] & 0xF) + (16 if qh[l] & u1 else 0)) - mm1)
        for l in range(32):
            y.append(d2 * np.float32((ql[32 * g + l] >> 4) + (16 if qh[l] & u2 else 0)) - mm2)
        is_ += 2
        u1 <<= 2
        u2 <<= 2
    return np.array(y, np.float32)


def _q6k_dequant_literal(blk):
    """dequantize_row_q6_K as a scalar loop over one 210-byte block (llama.cpp form:
    two halves of 128, four outputs per l, pointers advanced by 64/32/8)."""
    d = np.float32(np.frombuffer(blk[208:210].tobytes(), np.float16)[0])
    sc = blk[192:208].view(np.int8)
    y = np.zeros(256, np.float32)
    for n in range(2):
        ql, qh, s = blk[64 * n:64 * n + 64], blk[128 + 32 * n:160 + 32 * n], sc[8 * n:8 * n + 8]
        for l in range(32):
            is_ = l // 16
            q1 = int((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32
            q2 = int((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32
            q3 = int((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32
            q4 = int((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32
            for off, qq, si in ((0, q1, 0), (32, q2, 2), (64, q3, 4), (96, q4, 6)):
                y[128 * n + l + off] = (d * np.float32(s[is_ + si])) * np.float32(qq)
    return y


def test_q5k_dequant_matches_literal_loop():
    w = okq.q5k_random(6, 512, seed=1)
    deq = okq.q5k_dequant(w, 512)
    for r in range(6):
        for b in range(2):
            np.testing.assert_array_equal(
                deq[r, 256 * b:256 * b + 256], _q5k_dequant_literal(w[r, 176 * b:176 * b + 176]))


def test_q6k_dequant_matches_literal_loop():
    w = okq.q6k_random(6, 512, seed=2)
    deq = okq.q6k_dequant(w, 512)
    for r in range(6):
        for b in range(2):
            np.testing.assert_array_equal(
                deq[r, 256 * b:256 * b + 256], _q6k_dequant_literal(w[r, 210 * b:210 * b + 210]))


def test_kquant_bytes_roundtrip():
    w5 = okq.q5k_random(9, 768, seed=3)
    np.testing.assert_array_equal(okq.q5k_make(*okq.q5k_fields(w5, 768)).reshape(w5.shape), w5)
    w6 = okq.q6k_random(9, 768, seed=4)
    np.testing.assert_array_equal(okq.q6k_make(*okq.q6k_fields(w6, 768)).reshape(w6.shape), w6)


def test_q6k_code_positions():
    """One nonzero code per quadrant lands at e = 128g + 32qd + l with scale sc[e//16]."""
    for g, qd, l in [(0, 0, 3), (0, 1, 17), (1, 2, 31), (1, 3, 0)]:
        q = np.full((1, 256), 32, np.uint8)
        e = 128 * g + 32 * qd + l
        q[0, e] = 45
        sc = np.arange(1, 17, dtype=np.int8)[None]
        blk = okq.q6k_make(np.array([1.0]), sc, q)
        y = okq.q6k_dequant(blk, 256)[0]
        assert list(np.nonzero(y)[0]) == [e]
        assert y[e] == 13 * (e // 16 + 1)
        np.testing.assert_array_equal(y, _q6k_dequant_literal(blk[0]))


def test_kquant_encoders_error_ladder():
    """Reference tests/test_gemm_q4k.py:440-448,483-496: faithful reconstructions,
    6-bit tighter than 5-bit tighter than 4-bit."""
    w = (RNG.standard_normal((16, 1024)) * 0.1).astype(np.float32)
    _, d5 = okq.q5k_quantize(w)
    _, d6 = okq.q6k_quantize(w)

    def cos(a, b):
        return float((a * b).sum() / np.sqrt((a * a).sum() * (b * b).sum()))

    e5, e6 = np.abs(d5 - w).mean(), np.abs(d6 - w).mean()
    assert cos(d5, w) > 0.99 and cos(d6, w) > 0.99
    assert e6 < e5


def test_kquant_gemv_matches_dequant_matmul():
    x = RNG.integers(-127, 128, (5, 768), dtype=np.int8)
    xs = RNG.random(5).astype(np.float32)
    for gemv, deqf, w in ((okq.q5k_gemv, okq.q5k_dequant, okq.q5k_random(40, 768, seed=5)),
                          (okq.q6k_gemv, okq.q6k_dequant, okq.q6k_random(40, 768, seed=6))):
        y = gemv(x, xs, w, 768)
        dq = deqf(w, 768).astype(np.float64)
        ref = (x.astype(np.float64) @ dq.T) * xs[:, None]
        # the dequantised weights carry one or two fp32 roundings each (2^-23 relative)
        bound = (np.abs(x).astype(np.float64) @ np.abs(dq).T) * xs[:, None] * 2.0 ** -22
        assert (np.abs(y - ref) <= bound + 1e-12).all()


# ---------------------------------------------------------------- attention
def test_scores_brute_force_gqa():
    q = RNG.integers(-127, 128, (1, 4, 3, 8), dtype=np.int8)
    k = RNG.integers(-127, 128, (1, 2, 5, 8), dtype=np.int8)
    s = oa.scores_i32(q, k)
    for h in range(4):
        for i in range(3):
            for j in range(5):
                assert s[0, h, i, j] == sum(int(q[0, h, i, d]) * int(k[0, h // 2, j, d])
                                            for d in range(8))


def _case(B=1, Hq=4, Hkv=2, M=37, N=53, D=64, seed=0):
    r = np.random.default_rng(seed)
    q = r.standard_normal((B, Hq, M, D)).astype(np.float16)
    k = r.standard_normal((B, Hkv, N, D)).astype(np.float16)
    v = r.standard_normal((B, Hkv, N, D)).astype(np.float16)
    return q, k, v


@pytest.mark.parametrize("causal", [False, True])
def test_prefill_oracle_vs_textbook(causal):
    """Online/exp2 oracle == dense e-base softmax on dequantised operands
    (catches transposes, GQA head map, causal alignment M != N, log2e fold)."""
    q, k, v = _case()
    q_i8, qs, k_i8, ks, _ = oqn.quantize_qk(q, k)
    out, lse = oa.attn_int8_fwd(q_i8, qs, k_i8, ks, v.astype(np.float32), causal)
    qd = q_i8.astype(np.float64) * qs[..., None]
    kd = k_i8.astype(np.float64) * ks[..., None]
    ref = oa.attention_fp64(qd, kd, v.astype(np.float64), causal, scale=math.log(2))
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)
    # LSE in natural log of ln2-scaled logits
    s = np.matmul(qd, np.swapaxes(kd[:, oa.kv_head_index(4, 2)], -1, -2)) * math.log(2)
    if causal:
        s = np.where(oa.valid_mask(37, 53, True), s, -np.inf)
    mx = s.max(-1, keepdims=True)
    np.testing.assert_allclose(lse, (mx + np.log(np.exp(s - mx).sum(-1, keepdims=True)))[..., 0],
                               rtol=1e-5)


def test_prefill_oracle_quality_vs_true_attention():
    """The whole prologue + int8 attention meets the reference's int8 gate
    against fp64 attention on the original fp16 inputs (test_attn_fwd.py:44-51)."""
    q, k, v = _case(B=1, Hq=2, Hkv=2, M=128, N=128, D=64, seed=5)
    for causal in (False, True):
        q_i8, qs, k_i8, ks, _ = oqn.quantize_qk(q, k)
        out, _ = oa.attn_int8_fwd(q_i8, qs, k_i8, ks, v.astype(np.float32), causal)
        assert_int8_quality(out, oa.attention_fp64(q, k, v, causal))


def test_window_mask_brute_force():
    M, N, wl = 6, 9, 3
    ok = oa.valid_mask(M, N, True, wl)
    for i in range(M):
        for j in range(N):
            pos = i + N - M
            assert ok[i, j] == (j <= pos and j > pos - wl)
    empty = oa.valid_mask(4, 4, True, 0)
    assert not empty.any()  # window 0 masks everything -> rows output 0


def test_fully_masked_rows_output_zero():
    q, k, v = _case(M=4, N=4, Hq=2, Hkv=2)
    q_i8, qs, k_i8, ks, _ = oqn.quantize_qk(q, k)
    out, lse = oa.attn_int8_fwd(q_i8, qs, k_i8, ks, v.astype(np.float32), True, window_left=0)
    assert not out.any() and np.isneginf(lse).all()


@pytest.mark.parametrize("ns", [1, 3, 16, 64])
def test_decode_split_invariance(ns):
    """Split partials + LSE merge equal the unsplit softmax for any split count,
    including splits that are empty (ns=64 > N/…)."""
    q, k, v = _case(B=2, Hq=8, Hkv=2, M=1, N=50, D=64, seed=9)
    q_i8, qs, k_i8, ks, _ = oqn.quantize_qk(q, k)
    dec = oa.attn_int8_decode(q_i8[:, :, 0], qs[:, :, 0], k_i8, ks, v.astype(np.float32), ns)
    pre, _ = oa.attn_int8_fwd(q_i8, qs, k_i8, ks, v.astype(np.float32), False)
    np.testing.assert_allclose(dec, pre[:, :, 0], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("ns", [1, 5, 64])
def test_decode_kv8_equals_dequantised_v(ns):
    """int8-V decode: folding v_scale[d] into each split's partial commutes with the
    LSE merge, so it equals the fp decode on V = v_i8 * v_scale (scaled here, per KV
    head, independently of the oracle's head map); v_scale = 1 reduces to v_i8."""
    q, k, v = _case(B=2, Hq=8, Hkv=2, M=1, N=70, D=64, seed=13)
    q_i8, qs, k_i8, ks, _ = oqn.quantize_qk(q, k)
    v_i8, vs = oqn.quantize_v_perchannel(v)  # vs [B,Hkv,D]
    got = oa.attn_int8_decode_kv8(q_i8[:, :, 0], qs[:, :, 0], k_i8, ks, v_i8, vs, ns)
    deq = v_i8.astype(np.float64) * vs[:, :, None, :].astype(np.float64)
    ref = oa.attn_int8_decode(q_i8[:, :, 0], qs[:, :, 0], k_i8, ks, deq, ns)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    ones = np.ones_like(vs)
    got1 = oa.attn_int8_decode_kv8(q_i8[:, :, 0], qs[:, :, 0], k_i8, ks, v_i8, ones, ns)
    ref1 = oa.attn_int8_decode(q_i8[:, :, 0], qs[:, :, 0], k_i8, ks, v_i8.astype(np.float64), ns)
    np.testing.assert_allclose(got1, ref1, rtol=1e-12, atol=1e-12)
    # the dequantised cache is close to the fp16 one (per-channel int8 V)
    fp = oa.attn_int8_decode(q_i8[:, :, 0], qs[:, :, 0], k_i8, ks, v.astype(np.float64), ns)
    assert_int8_quality(got, fp, min_cos=0.998, max_rel_l1=0.03, min_sqnr_db=18)


def test_w8a8_oracle_close_to_fp16v():
    """Int8 PV (per-row and per-half P scales) stays within the reference's int8-PV
    bars of the fp16-V result (test_attn_fwd_w8a8.py:37)."""
    q, k, v = _case(B=1, Hq=4, Hkv=2, M=96, N=160, D=64, seed=11)
    q_i8, qs, k_i8, ks, _ = oqn.quantize_qk(q, k)
    v_i8, vs = oqn.quantize_v_perchannel(v)
    for causal in (False, True):
        ref, _ = oa.attn_int8_fwd(q_i8, qs, k_i8, ks, v.astype(np.float32), causal)
        for pw in (True, False):
            out = oa.attn_w8a8_fwd(q_i8, qs, k_i8, ks, v_i8, vs, causal, 160 - 96, pw)
            assert_int8_quality(out, ref, min_cos=0.998, max_rel_l1=0.03, min_sqnr_db=18)


def _w8_bf16_case():
    """Logits set exactly through k_scale (q codes 1, k codes 1, D = 128, q_scale =
    1/128): in every 32-key half one key sits at the half's max and 31 keys
    log2(127/101) below it, so 31 codes equal 101 and their bf16(101 * f)
    operands share one rounding error (101/127 is not a bf16 number)."""
    D, M, N = 128, 64, 128
    q = np.ones((1, 1, M, D), np.int8)
    k = np.ones((1, 1, N, D), np.int8)
    qs = np.full((1, 1, M), 1.0 / 128.0, np.float32)
    base = np.float32(-1.0)
    off = np.float32(np.log2(101.0 / 127.0))
    ks = np.full((1, 1, N), base + off, np.float32)
    ks[..., ::32] = base
    g = np.random.default_rng(3)
    v = g.integers(-127, 128, (1, 1, N, D), dtype=np.int8)
    vs = np.full((1, 1, D), 0.01, np.float32)
    return q, qs, k, ks, v, vs


def test_w8a8_bf16_model_bounds_and_sensitivity():
    """The kernel model (bf16 P operands, lazy reference point) against the
    reference-semantics oracle: within the bf16 bound on random data, and
    visibly apart on the correlated-rounding case, where a model without the
    bf16 rounding would agree with the oracle."""
    g = np.random.default_rng(9)
    B, H, M, N, D = 1, 2, 96, 200, 64
    q = g.integers(-127, 128, (B, H, M, D), dtype=np.int8)
    k = g.integers(-127, 128, (B, H, N, D), dtype=np.int8)
    v = g.integers(-127, 128, (B, H, N, D), dtype=np.int8)
    qs = np.full((B, H, M), 1.0 / 2000.0, np.float32)
    ks = (g.random((B, H, N)) * 0.5 + 0.5).astype(np.float32)
    vs = np.full((B, H, D), 0.01, np.float32)
    for causal in (False, True):
        diag = N - M if causal else 0
        ref = oa.attn_w8a8_fwd(q, qs, k, ks, v, vs, causal, diag, True)
        mod = oa.attn_w8a8_fwd_bf16pv_model(q, qs, k, ks, v, vs, causal, diag)
        assert_int8_quality(mod, ref, min_cos=0.99999, max_rel_l1=4e-3, min_sqnr_db=45)
        # a zero rescale headroom moves the reference point at every rising half:
        # the same softmax (other bf16 roundings), still within the bound
        mod0 = oa.attn_w8a8_fwd_bf16pv_model(q, qs, k, ks, v, vs, causal, diag, excess=0.0)
        assert_int8_quality(mod0, ref, min_cos=0.99999, max_rel_l1=4e-3, min_sqnr_db=45)
    q, qs, k, ks, v, vs = _w8_bf16_case()
    ref = oa.attn_w8a8_fwd(q, qs, k, ks, v, vs, False, 0, True)
    mod = oa.attn_w8a8_fwd_bf16pv_model(q, qs, k, ks, v, vs, False, 0)
    rel = np.abs(mod - ref).max() / np.abs(ref).max()
    assert rel > 1e-3, rel


def test_w8a8_p_requant_known_answer():
    """One query, 2 keys in one tile with p = (1, 1/3): p_scale = fp32(1/127),
    codes (127, rint(127/3)=42); output = (127*v0 + 42*v1)*ps*vs / (1 + 1/3)."""
    q_i8 = np.zeros((1, 1, 1, 4), np.int8)
    q_i8[..., 0] = 1
    k_i8 = np.zeros((1, 1, 2, 4), np.int8)
    k_i8[0, 0, 0, 0] = 2
    k_i8[0, 0, 1, 0] = 1
    l3 = np.float32(math.log2(3.0))
    qs = np.array([[[l3]]], np.float32)
    ks = np.array([[[1.0, 0.0]]], np.float32)
    # logits: key0 = 2*log2(3)... use ks to make key1 logit 0 and key0 log2(3)
    ks[0, 0, 0] = np.float32(0.5)
    v_i8 = np.array([[[[10, 0, 0, 0], [-20, 0, 0, 0]]]], np.int8)
    vs = np.ones((1, 1, 4), np.float32)
    out = oa.attn_w8a8_fwd(q_i8, qs, k_i8, ks, v_i8, vs, per_warp_quant=False)
    s0 = np.float32(np.float32(2.0) * l3) * np.float32(0.5)
    p1 = 2.0 ** (0.0 - float(s0))
    ps = np.float32(np.float32(1.0) * np.float32(1.0 / 127.0))
    inv = np.float32(1.0) / ps
    c1 = np.rint(np.float32(np.float32(p1) * inv))
    want = (127 * 10 + float(c1) * -20) * float(ps) / (1.0 + p1)
    assert abs(out[0, 0, 0, 0] - want) < 1e-9


# ---------------------------------------------------------------------------
# Paged decode and quantize-on-write (reference attn_paged_decode.cuh)
# ---------------------------------------------------------------------------
def _paged_case(B=2, Hq=8, Hkv=2, D=64, bs=16, lens=(50, 50), nblk=12, seed=21, perm=True):
    rng = np.random.default_rng(seed)
    maxb = max((n + bs - 1) // bs for n in lens)
    k_cache = rng.integers(-127, 128, (nblk, Hkv, bs, D)).astype(np.int8)
    v_cache = rng.integers(-127, 128, (nblk, Hkv, bs, D)).astype(np.int8)
    k_scale = (rng.random((nblk, Hkv, bs)) * 0.02 + 1e-3).astype(np.float32)
    v_scale = (rng.random((nblk, Hkv, bs)) * 0.02 + 1e-3).astype(np.float32)
    blocks = rng.permutation(nblk) if perm else np.arange(nblk)
    bt = np.zeros((B, maxb), np.int32)
    used = 0
    for b, n in enumerate(lens):
        nb = (n + bs - 1) // bs
        bt[b, :nb] = blocks[used:used + nb]
        used += nb
    q = rng.integers(-127, 128, (B, Hq, D)).astype(np.int8)
    qs = (rng.random((B, Hq)) * 0.01 + 1e-3).astype(np.float32)
    return q, qs, k_cache, k_scale, v_cache, v_scale, bt, np.array(lens, np.int32)


@pytest.mark.parametrize("ns", [1, 3, 16])
def test_paged_decode_equals_contiguous(ns):
    """Equal lengths: gathering through a permuted block table gives the contiguous
    decode of the gathered cache with the per-token V scale applied to V."""
    q, qs, kc, ksc, vc, vsc, bt, lens = _paged_case(lens=(50, 50))
    got = oa.attn_paged_decode(q, qs, kc, ksc, vc, vsc, bt, lens, 50, ns)
    bs = kc.shape[2]
    for b in range(2):
        blk = bt[b, np.arange(50) // bs]
        off = np.arange(50) % bs
        k = np.swapaxes(kc[blk, :, off], 0, 1)[None]          # [1,Hkv,50,D]
        ks = np.swapaxes(ksc[blk, :, off], 0, 1)[None]
        v = (np.swapaxes(vc[blk, :, off], 0, 1).astype(np.float64)
             * np.swapaxes(vsc[blk, :, off], 0, 1)[..., None])[None]
        ref = oa.attn_int8_decode(q[b:b + 1], qs[b:b + 1], k, ks, v, ns)
        np.testing.assert_allclose(got[b:b + 1], ref, rtol=1e-9, atol=1e-12)


def test_paged_decode_ragged_lengths_and_block_order():
    """Ragged lengths: each sequence sees exactly its own keys (one split = plain
    softmax over them), and the physical block order does not matter."""
    q, qs, kc, ksc, vc, vsc, bt, lens = _paged_case(lens=(7, 61), perm=False, seed=23)
    a = oa.attn_paged_decode(q, qs, kc, ksc, vc, vsc, bt, lens, 61, 1)
    for b, n in enumerate(lens):
        kb = oa.gather_paged(kc, bt, b, n)[None]
        ksb = oa.gather_paged(ksc, bt, b, n)[None]
        vb = (oa.gather_paged(vc, bt, b, n).astype(np.float64)
              * oa.gather_paged(vsc, bt, b, n)[..., None])[None]
        ref = oa.attn_int8_decode(q[b:b + 1], qs[b:b + 1], kb, ksb, vb, 1)
        np.testing.assert_allclose(a[b:b + 1], ref, rtol=1e-9, atol=1e-12)
    # move every block to another physical slot: same result
    nblk = kc.shape[0]
    perm = np.random.default_rng(5).permutation(nblk)
    kc2, ksc2, vc2, vsc2 = (np.empty_like(x) for x in (kc, ksc, vc, vsc))
    kc2[perm], ksc2[perm], vc2[perm], vsc2[perm] = kc, ksc, vc, vsc
    b2 = oa.attn_paged_decode(q, qs, kc2, ksc2, vc2, vsc2, perm[bt].astype(np.int32), lens, 61, 4)
    b1 = oa.attn_paged_decode(q, qs, kc, ksc, vc, vsc, bt, lens, 61, 4)
    np.testing.assert_allclose(b2, b1, rtol=0, atol=0)


def test_paged_split_heuristic():
    """reference attn_paged_decode.cu:20-31 on hand-evaluated cases."""
    assert oa.paged_choose_num_splits(0, 8) == 1
    assert oa.paged_choose_num_splits(32768, 512) == 128    # max(4, 128) within [1, 683]
    assert oa.paged_choose_num_splits(100, 8) == 3          # min(256, 3)
    assert oa.paged_choose_num_splits(4096, 1) == 86        # min(2048, ceil(4096/48))
    assert oa.paged_choose_num_splits(10 ** 6, 1) == 256


def test_kv_write_quantiser_known_answers():
    from fractions import Fraction

    x = np.zeros((3, 8), np.float32)
    x[1, 3] = -0.75
    rng = np.random.default_rng(3)
    x[2] = rng.standard_normal(8).astype(np.float32)
    q, s = oqn.quantize_row_div(x)
    assert s[0] == 1.0 and not q[0].any()
    assert s[1] == np.float32(np.float32(0.75) / np.float32(127)) and q[1, 3] == -127 and q[1].sum() == -127
    # codes = round-half-even of the correctly rounded fp32 quotient (exact rationals)
    for r in range(3):
        for c in range(8):
            quo = np.float32(Fraction(float(x[r, c])) / Fraction(float(s[r])))
            want = int(np.rint(np.clip(quo, -127, 127)))
            assert q[r, c] == want
    # the scale is amax / 127, not amax * fp32(1/127) as in quantize_rows: the two
    # differ by an ulp on some rows, so a swapped formula fails here
    xs = rng.standard_normal((4000, 64)).astype(np.float32)
    _, sd = oqn.quantize_row_div(xs)
    _, sm = oqn.quantize_rows(xs)
    amax = np.abs(xs).max(-1)
    np.testing.assert_array_equal(sd, (amax / np.float32(127)).astype(np.float32))
    assert (sd != sm.reshape(sd.shape)).any()


def test_kv_write_paged_places_rows():
    kc = np.zeros((4, 2, 8, 16), np.int8)
    vc = np.zeros_like(kc)
    ks = np.zeros((4, 2, 8), np.float32)
    vs = np.zeros_like(ks)
    rng = np.random.default_rng(8)
    kn = rng.standard_normal((3, 2, 16)).astype(np.float32)
    vn = rng.standard_normal((3, 2, 16)).astype(np.float32)
    slots = np.array([5, 8 * 3 + 7, 8], np.int32)
    oqn.kv_write_paged(kn, vn, slots, kc, ks, vc, vs)
    kq, kscl = oqn.quantize_row_div(kn)
    for b, slot in enumerate(slots):
        blk, off = divmod(int(slot), 8)
        np.testing.assert_array_equal(kc[blk, :, off], kq[b])
        np.testing.assert_array_equal(ks[blk, :, off], kscl[b])
    assert np.count_nonzero(ks) == 3 * 2


def test_q_outlier_gate_definition():
    """Lower median for even D (torch.median), the 1e-10 guard, the fp32 ratio."""
    q = np.array([[1, 2, 3, 40], [4, 3, 2, 1], [0, 0, 0, 0], [-5, 1, 1, 60]], np.float32)
    mx, md = oqn.q_outlier_stats(q)
    np.testing.assert_array_equal(mx, [40, 4, 0, 60])
    np.testing.assert_array_equal(md, [2, 2, 0, 1])  # sorted |q|[(4-1)//2] = index 1
    assert oqn.q_outlier_gate(q)                      # 40/2 = 20 > 12, 60/1 > 12
    assert not oqn.q_outlier_gate(q[1:3])             # 4/2 = 2; zero row: 0/1e-10 = 0
    row = np.full((1, 5), 1.0, np.float32)
    row[0, 0] = 12.0
    assert not oqn.q_outlier_gate(row)                # exactly 12 is not > 12
    row[0, 0] = np.nextafter(np.float32(12.0), np.float32(13.0))
    assert oqn.q_outlier_gate(row)
    # brute force on random rows: the k-th smallest by counting
    rng = np.random.default_rng(4)
    x = rng.standard_normal((50, 33)).astype(np.float32)
    _, md = oqn.q_outlier_stats(x)
    a = np.abs(x)
    for r in range(50):
        cnt_lt = (a[r] < md[r]).sum()
        cnt_le = (a[r] <= md[r]).sum()
        assert cnt_lt <= 16 < cnt_le


def test_seeded_accumulator_logit_bound():
    """The prefill's seeded-accumulator logit (oracle/attention.py:seeded_logits)
    against the exact rational qs * ks * acc - m: the only error beyond fp32
    rounding is the rounding of the constant rn(C0 * qs * 2^26), worth at most
    0.64 integer units of acc. Extremes (+-128^3, 0, +-1) and random accs over
    q/k scales across 12 decades. A dropped seed offset (f read as acc * 2^-26)
    or a wrong binade (2^-25 spacing) fails by orders of magnitude."""
    from fractions import Fraction

    rng = np.random.default_rng(11)
    acc = np.concatenate([[0, 1, -1, 2 ** 21, -(2 ** 21), 128 * 127 * 127, -128 * 127 * 127],
                          rng.integers(-(2 ** 21), 2 ** 21, 3000)])
    qs = (10.0 ** rng.uniform(-8, 2, acc.size)).astype(np.float32)
    ks = (10.0 ** rng.uniform(-4, 2, acc.size)).astype(np.float32)
    m = rng.uniform(-20, 20, acc.size).astype(np.float32)
    x = oa.seeded_logits(acc, qs, ks, m)
    for a, q, k, mm, xx in zip(acc, qs, ks, m, x):
        exact = Fraction(float(q)) * Fraction(float(k)) * int(a) - Fraction(float(mm))
        mag = abs(Fraction(float(q)) * Fraction(float(k)) * int(a)) + abs(Fraction(float(mm)))
        bound = Fraction(0.65) * Fraction(float(q)) * Fraction(float(k)) + mag * Fraction(2.0 ** -22)
        assert abs(Fraction(float(xx)) - exact) <= bound, (a, q, k, mm, xx, float(exact))
    # f is exact: the seeded bits minus the seed are acc itself
    f = (acc + oa.SEED_BITS).astype(np.uint32).view(np.float32).astype(np.float64)
    c0 = float(np.uint32(oa.SEED_BITS).view(np.float32))
    np.testing.assert_array_equal((f - c0) * 2.0 ** 26, acc.astype(np.float64))

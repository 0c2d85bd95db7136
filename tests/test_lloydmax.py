"""3-bit Lloyd-Max V store (K8V3): the oracle and the torch format helpers, on CPU.

How oracle/lloydmax.py is pinned:
  * codebook  - J. Max's 1960 table of the 8-level N(0,1) quantiser (4 digits),
                symmetry, and a Lloyd-Max fit on 2M Gaussian samples;
  * pack3 / unpack3 - hand-worked words (codes 0..7 -> 0xFAC688, the code
                that straddles bits 30..32), all-ones, round trips;
  * quantize  - brute-force nearest level, ties to the lower level;
  * dequant_fp16 - the double rounding fp32 then fp16 on a product where a
                single rounding gives a different fp16 value;
  * attn_paged_decode_k8v3 - an independent float64 softmax attention over
                the dequantised store, and split invariance.
Reference tests mirrored: tests/test_lloydmax.py, tests/test_lloydmax_contiguous.py,
tests/test_k8v3_paged_decode.py (the store builder's recipe).
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import lloydmax as olm
from superl8_amd.quant import lloydmax as lm

# Max (1960), table I, N = 8 output levels (positive half)
MAX_1960 = (0.2451, 0.7560, 1.3440, 2.1520)


def test_codebook_is_max_1960_table():
    cb = olm.gaussian_codebook(1).astype(np.float64)
    np.testing.assert_allclose(cb[4:], MAX_1960, atol=2e-4)
    np.testing.assert_array_equal(cb[:4], -cb[4:][::-1])
    for bs in (32, 64, 128):
        np.testing.assert_array_equal(olm.gaussian_codebook(bs),
                                      lm.gaussian_codebook(3, bs).numpy())
        np.testing.assert_allclose(olm.gaussian_codebook(bs) * math.sqrt(bs),
                                   olm.gaussian_codebook(1), rtol=1e-6)


def test_lloyd_max_fit_recovers_gaussian_levels():
    # a mirrored sample (the fit's shift direction is weakly determined by a
    # finite sample, so sampling noise would move all levels together)
    h = np.random.default_rng(0).standard_normal(1_000_000)
    x = torch.from_numpy(np.concatenate([h, -h]))
    c = lm.lloyd_max_fit(x, 8, iters=200, tol=1e-9).double().numpy()
    np.testing.assert_allclose(c[4:], MAX_1960, atol=3e-3)
    np.testing.assert_allclose(c[:4], -c[4:][::-1], atol=1e-6)
    # deterministic, and an empty input gives zeros
    assert torch.equal(lm.lloyd_max_fit(x[:1000], 8), lm.lloyd_max_fit(x[:1000], 8))
    assert torch.equal(lm.lloyd_max_fit(torch.zeros(0), 8), torch.zeros(8))


def test_pack_known_answers():
    codes = np.tile(np.arange(8, dtype=np.uint8), 4)[None]          # 32 codes, 3 words
    w = olm.pack3(codes).view(np.uint32)[0]
    # codes 0..7 fill bits 0..23 with 0xFAC688; code 8 (=0) bits 24..26,
    # code 9 (=1) bit 27, code 10 (=2 = 0b010) straddles: bit 31 set
    assert w[0] == 0x88FAC688
    one = np.zeros((1, 32), np.uint8)
    one[0, 10] = 7                                                   # bits 30, 31, 32
    assert list(olm.pack3(one).view(np.uint32)[0]) == [0xC0000000, 0x1, 0x0]
    one[0, 10] = 0
    one[0, 21] = 5                                                   # bits 63..65: 1 at 63, 0, 1 at 65
    assert list(olm.pack3(one).view(np.uint32)[0]) == [0, 0x80000000, 0x2]
    assert (olm.pack3(np.full((2, 128), 7, np.uint8)) == -1).all()
    for arr in (codes, one):
        t = lm.pack_indices_lowbit(torch.from_numpy(arr), 3).numpy()
        np.testing.assert_array_equal(t, olm.pack3(arr))


@pytest.mark.parametrize("d", [32, 128, 256])
def test_pack_round_trip(d):
    codes = np.random.default_rng(d).integers(0, 8, (5, 3, d)).astype(np.uint8)
    words = olm.pack3(codes)
    assert words.shape == (5, 3, 3 * d // 32) and words.dtype == np.int32
    np.testing.assert_array_equal(olm.unpack3(words, d), codes)
    tw = lm.pack_indices_lowbit(torch.from_numpy(codes), 3)
    np.testing.assert_array_equal(tw.numpy(), words)
    np.testing.assert_array_equal(lm.unpack_indices_lowbit(tw, 3, d).numpy(), codes)


def test_quantize_is_nearest_level_ties_low():
    cb = olm.gaussian_codebook(128)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((64, 256)).astype(np.float32)
    x[0, :128] = 0.0                                                 # zero block: norm 1, code 3
    codes, norms = olm.quantize(x, cb)
    assert norms[0, 0] == 1.0 and (codes[0, :128] == 3).all()
    unit = x.reshape(64, 2, 128) / norms[..., None]
    brute = np.abs(unit[..., None].astype(np.float64) - cb.astype(np.float64)).argmin(-1)
    # argmin picks the lower index on an exact tie, as bucketize does
    np.testing.assert_array_equal(codes.reshape(64, 2, 128), brute)
    tc, tn, tcb = lm.quantize_lloydmax(torch.from_numpy(x))
    np.testing.assert_array_equal(tcb.numpy(), cb)
    np.testing.assert_allclose(tn.numpy(), norms, rtol=1e-6)
    np.testing.assert_array_equal(tc.numpy(), codes)
    # a value on a decision boundary takes the lower code (bucketize, right=False)
    cbt = torch.tensor([-3.0, -2.0, -1.0, -0.5, 0.5, 1.0, 2.0, 3.0])
    on_mid = torch.tensor([[0.0, 0.75, -2.5, 0.7500001]])
    c, _, _ = lm.quantize_lloydmax(on_mid, block_size=4, codebook=cbt)
    u = (on_mid / on_mid.norm()).numpy().astype(np.float32)
    np.testing.assert_array_equal(c.numpy(), np.searchsorted(
        (0.5 * (cbt[1:] + cbt[:-1])).numpy(), u, side="left"))
    assert c[0, 0] == 3


def test_dequant_rounds_product_to_fp32_then_fp16():
    # (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24: fp32 rounds it to the fp16 midpoint
    # 1 + 2^-11 (tie -> even: 1.0); one rounding of the exact product gives 1 + 2^-10
    a = np.float32(1 + 2.0 ** -12)
    cb = np.array([a] * 8, np.float32)
    v = olm.dequant_fp16(np.zeros((1, 128), np.uint8), np.array([[a]], np.float32), cb)
    assert (v == 1.0).all()
    assert np.float16(float(a) * float(a)) == np.float16(1 + 2.0 ** -10)


def test_dequant_matches_torch_helper():
    x = torch.from_numpy(np.random.default_rng(2).standard_normal((7, 256)).astype(np.float32))
    codes, norm, cb = lm.quantize_lloydmax(x)
    want = lm.dequantize_lloydmax(codes, norm, cb).numpy()
    got = olm.dequant_fp16(codes.numpy(), norm.numpy(), cb.numpy())
    np.testing.assert_array_equal(got, want.astype(np.float16).astype(np.float32))
    # fake quant == quantise + dequantise, and a fitted codebook does not lose quality
    fq = lm.fake_quant_lloydmax(x)
    np.testing.assert_array_equal(fq.numpy(), want)
    e0 = ((lm.fake_quant_lloydmax(x) - x) ** 2).mean()
    e1 = ((lm.fake_quant_lloydmax(x, fit=True) - x) ** 2).mean()
    assert e1 <= e0 * 1.02
    rel = (((fq - x) ** 2).sum() / (x ** 2).sum()).item()
    assert rel < 0.04  # 3-bit Gaussian quantiser: distortion 0.0345 of the variance


def _k8v3_store(rng, lens, Hkv, D, bs, shuffle=True):
    B = len(lens)
    nbs = [(n + bs - 1) // bs for n in lens]
    nblk = sum(nbs) + 2
    perm = rng.permutation(nblk) if shuffle else np.arange(nblk)
    bt = np.zeros((B, max(max(nbs), 1)), np.int32)
    o = 0
    for b, nb in enumerate(nbs):
        bt[b, :nb] = perm[o:o + nb]
        o += nb
    kc = rng.integers(-127, 128, (nblk, Hkv, bs, D)).astype(np.int8)
    ks = (rng.random((nblk, Hkv, bs)) * 0.02 + 0.001).astype(np.float32)
    codes = rng.integers(0, 8, (nblk, Hkv, bs, D)).astype(np.uint8)
    vp = olm.pack3(codes)
    vn = (rng.random((nblk, Hkv, bs, D // 128)) * 20 + 1).astype(np.float32)
    return kc, ks, vp, vn, bt, np.array(lens, np.int32)


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 4, 2), (256, 8, 2)])
def test_k8v3_decode_oracle_is_softmax_attention(D, Hq, Hkv):
    rng = np.random.default_rng(D + Hq)
    lens, bs = [5, 33, 64], 16
    kc, ks, vp, vn, bt, ctx = _k8v3_store(rng, lens, Hkv, D, bs)
    cb = olm.gaussian_codebook(128)
    q = rng.integers(-127, 128, (3, Hq, D)).astype(np.int8)
    qs = (rng.random((3, Hq)) * 0.02 + 0.001).astype(np.float32)
    out = olm.attn_paged_decode_k8v3(q, qs, kc, ks, vp, vn, cb, bt, ctx, 64, 2)
    out4 = olm.attn_paged_decode_k8v3(q, qs, kc, ks, vp, vn, cb, bt, ctx, 64, 4)
    np.testing.assert_allclose(out, out4, rtol=1e-12, atol=1e-12)
    idx = oa.kv_head_index(Hq, Hkv)
    for b, n in enumerate(lens):
        pos = np.arange(n)
        blk, off = bt[b, pos // bs], pos % bs
        kf = kc[blk, :, off].astype(np.float64) * ks[blk, :, off][..., None]   # [n, Hkv, D]
        codes = np.stack([olm.unpack3(vp[blk[i], :, off[i]], D) for i in range(n)])
        vf = cb[codes] * np.repeat(vn[blk, :, off], 128, -1)               # fp32 products
        vf = vf.astype(np.float16).astype(np.float64)
        for h in range(Hq):
            s = (q[b, h].astype(np.float64) * qs[b, h]) @ kf[:, idx[h]].T      # exp2 domain
            p = np.exp2(s - s.max())
            ref = p @ vf[:, idx[h]] / p.sum()
            np.testing.assert_allclose(out[b, h], ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())

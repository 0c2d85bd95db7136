"""Q5_K and Q6_K super-block decode and GEMV (numpy restatement).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Q5_K, 176 bytes per 256 weights (reference csrc/include/gemm_q4k_dp4a.cuh:
200-209,250-275; tests/test_gemm_q4k.py:151-192; originally llama.cpp
block_q5_K / dequantize_row_q5_K):
  [0:2] d fp16, [2:4] dmin fp16, [4:16] the 12-byte 6-bit (sc, m) packing of
  Q4_K, [16:48] qh (bit j of qh[l] = 5th bit of element l of sub-block j),
  [48:176] qs with Q4_K's nibble interleave (byte 32g + l: low nibble =
  sub-block 2g, high nibble = sub-block 2g + 1).
  q = nibble | (qh bit << 4) in [0, 31];  w = fp32(d)*sc_j*q - fp32(dmin)*m_j.
Q6_K, 210 bytes per 256 weights (gemm_q4k_dp4a.cuh:351-360,404-445;
tests/test_gemm_q4k.py:195-237; llama.cpp block_q6_K / dequantize_row_q6_K):
  [0:128] ql, [128:192] qh, [192:208] 16 signed int8 scales, [208:210] d fp16.
  Element e = 128*g + 32*qd + l (g in 0..1, qd in 0..3, l in 0..31):
  nibble = ql[64g + l + 32*(qd & 1)] (low nibble for qd < 2, high otherwise),
  high 2 bits = (qh[32g + l] >> 2qd) & 3; q = nibble | high << 4 in [0, 63];
  w = fp32(d) * sc[e // 16] * (q - 32).
GEMV: y[m, n] = x_scale[m] * sum over sub-blocks of the scaled integer dot
products (plus the Q5_K min term), evaluated in float64 from exact integer sums.
"""
from __future__ import annotations

import numpy as np

from .q4k import QK_K, pack_scale_min_k4, scale_min_k4

Q5K_BYTES = 176
Q6K_BYTES = 210


# ---------------------------------------------------------------- Q5_K
def q5k_fields(w: np.ndarray, K: int):
    """bytes [N, K/256*176] -> (d, dmin fp32 [N,nsb], sc, mn [N,nsb,8], q [N,nsb,8,32] in 0..31)."""
    N = w.shape[0]
    b = w.reshape(N, K // QK_K, Q5K_BYTES)
    d = b[..., 0:2].copy().view(np.float16).astype(np.float32)[..., 0]
    dmin = b[..., 2:4].copy().view(np.float16).astype(np.float32)[..., 0]
    sc, mn = scale_min_k4(b[..., 4:16])
    qh = b[..., 16:48]                                   # [N,nsb,32]
    qs = b[..., 48:176].reshape(N, K // QK_K, 4, 32)
    q = np.empty((N, K // QK_K, 8, 32), np.uint8)
    q[..., 0::2, :] = qs & 0xF
    q[..., 1::2, :] = qs >> 4
    for j in range(8):
        q[..., j, :] |= ((qh >> j) & 1) << 4
    return d, dmin, sc, mn, q


def q5k_make(d, dmin, sc, mn, q) -> np.ndarray:
    """Fields -> bytes [..., 176] (q [..., 8, 32] in 0..31)."""
    lead = d.shape
    blk = np.zeros(lead + (Q5K_BYTES,), np.uint8)
    blk[..., 0:2] = np.ascontiguousarray(d.astype(np.float16)).view(np.uint8).reshape(lead + (2,))
    blk[..., 2:4] = np.ascontiguousarray(dmin.astype(np.float16)).view(np.uint8).reshape(lead + (2,))
    blk[..., 4:16] = pack_scale_min_k4(sc, mn)
    q = q.astype(np.uint8)
    qh = np.zeros(lead + (32,), np.uint8)
    for j in range(8):
        qh |= ((q[..., j, :] >> 4) & 1) << j
    blk[..., 16:48] = qh
    lo = q & 0xF
    blk[..., 48:176] = (lo[..., 0::2, :] | (lo[..., 1::2, :] << 4)).reshape(lead + (128,))
    return blk


def q5k_random(N: int, K: int, seed: int) -> np.ndarray:
    """Synthetic Q5_K bytes [N, K/256*176]: d, dmin = fp16(|N(0,1)|*1e-2), sc/m in [0,63], q in [0,31]."""
    rng = np.random.default_rng(seed)
    nsb = K // QK_K
    d = (np.abs(rng.standard_normal((N, nsb))) * 1e-2).astype(np.float16)
    dmin = (np.abs(rng.standard_normal((N, nsb))) * 1e-2).astype(np.float16)
    sc = rng.integers(0, 64, (N, nsb, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, (N, nsb, 8), dtype=np.uint8)
    q = rng.integers(0, 32, (N, nsb, 8, 32), dtype=np.uint8)
    return q5k_make(d, dmin, sc, mn, q).reshape(N, nsb * Q5K_BYTES)


def q5k_dequant(w: np.ndarray, K: int) -> np.ndarray:
    """fp32 [N,K]: fp32(d)*sc*q - fp32(dmin)*m (reference tests/test_gemm_q4k.py:188-190)."""
    d, dmin, sc, mn, q = q5k_fields(w, K)
    dsc = (d[..., None] * sc.astype(np.float32)).astype(np.float32)
    dm = (dmin[..., None] * mn.astype(np.float32)).astype(np.float32)
    return (dsc[..., None] * q.astype(np.float32) - dm[..., None]).astype(np.float32).reshape(w.shape[0], K)


def q5k_gemv(x_i8: np.ndarray, x_scale: np.ndarray, w: np.ndarray, K: int) -> np.ndarray:
    """y [M,N] float64: x_scale[m] * sum_j (d*sc_j*<x_j,q_j> - dmin*m_j*sum(x_j))."""
    d, dmin, sc, mn, q = q5k_fields(w, K)
    nsb = K // QK_K
    xs = x_i8.astype(np.float64).reshape(x_i8.shape[0], nsb, 8, 32)
    S = np.einsum("mbjk,nbjk->mnbj", xs, q.astype(np.float64))
    X = xs.sum(-1)
    t = (d[None, :, :, None].astype(np.float64) * sc[None].astype(np.float64) * S
         - dmin[None, :, :, None].astype(np.float64) * mn[None].astype(np.float64) * X[:, None])
    return t.sum(axis=(2, 3)) * x_scale.astype(np.float64)[:, None]


# ---------------------------------------------------------------- Q6_K
def q6k_fields(w: np.ndarray, K: int):
    """bytes [N, K/256*210] -> (d fp32 [N,nsb], sc int8 [N,nsb,16], q [N,nsb,256] in 0..63, natural order)."""
    N = w.shape[0]
    nsb = K // QK_K
    b = w.reshape(N, nsb, Q6K_BYTES)
    ql = b[..., 0:128].reshape(N, nsb, 2, 64)
    qh = b[..., 128:192].reshape(N, nsb, 2, 32)
    sc = b[..., 192:208].copy().view(np.int8)
    d = b[..., 208:210].copy().view(np.float16).astype(np.float32)[..., 0]
    q = np.empty((N, nsb, 2, 4, 32), np.uint8)
    for qd in range(4):
        src = ql[..., 32 * (qd & 1):32 * (qd & 1) + 32]
        nib = (src & 0xF) if qd < 2 else (src >> 4)
        q[..., qd, :] = nib | (((qh >> (2 * qd)) & 3) << 4)
    return d, sc, q.reshape(N, nsb, 256)


def q6k_make(d, sc, q) -> np.ndarray:
    """Fields -> bytes [..., 210] (sc int8 [...,16], q [...,256] in 0..63, natural order)."""
    lead = d.shape
    qc = q.astype(np.uint8).reshape(lead + (2, 4, 32))
    ql = np.zeros(lead + (2, 64), np.uint8)
    ql[..., 0:32] = (qc[..., 0, :] & 0xF) | ((qc[..., 2, :] & 0xF) << 4)
    ql[..., 32:64] = (qc[..., 1, :] & 0xF) | ((qc[..., 3, :] & 0xF) << 4)
    qh = np.zeros(lead + (2, 32), np.uint8)
    for qd in range(4):
        qh |= ((qc[..., qd, :] >> 4) & 3) << (2 * qd)
    blk = np.zeros(lead + (Q6K_BYTES,), np.uint8)
    blk[..., 0:128] = ql.reshape(lead + (128,))
    blk[..., 128:192] = qh.reshape(lead + (64,))
    blk[..., 192:208] = np.ascontiguousarray(sc.astype(np.int8)).view(np.uint8)
    blk[..., 208:210] = np.ascontiguousarray(d.astype(np.float16)).view(np.uint8).reshape(lead + (2,))
    return blk


def q6k_random(N: int, K: int, seed: int) -> np.ndarray:
    """Synthetic Q6_K bytes [N, K/256*210]: d = fp16(|N(0,1)|*1e-3), sc uniform int8, q in [0,63]."""
    rng = np.random.default_rng(seed)
    nsb = K // QK_K
    d = (np.abs(rng.standard_normal((N, nsb))) * 1e-3).astype(np.float16)
    sc = rng.integers(-128, 128, (N, nsb, 16)).astype(np.int8)
    q = rng.integers(0, 64, (N, nsb, 256), dtype=np.uint8)
    return q6k_make(d, sc, q).reshape(N, nsb * Q6K_BYTES)


def q6k_dequant(w: np.ndarray, K: int) -> np.ndarray:
    """fp32 [N,K]: (fp32(d)*sc) * (q - 32) (reference tests/test_gemm_q4k.py:218-221)."""
    d, sc, q = q6k_fields(w, K)
    rs = (d[..., None] * sc.astype(np.float32)).astype(np.float32)           # [N,nsb,16]
    qq = (q.astype(np.float32) - 32.0).reshape(q.shape[:-1] + (16, 16))
    return (rs[..., None] * qq).astype(np.float32).reshape(w.shape[0], K)


def q6k_gemv(x_i8: np.ndarray, x_scale: np.ndarray, w: np.ndarray, K: int) -> np.ndarray:
    """y [M,N] float64: x_scale[m] * sum_i d*sc_i*<x_i, q_i - 32> over 16-element sub-blocks."""
    d, sc, q = q6k_fields(w, K)
    N, nsb = d.shape
    xs = x_i8.astype(np.float64).reshape(x_i8.shape[0], nsb, 16, 16)
    qq = (q.astype(np.float64) - 32.0).reshape(N, nsb, 16, 16)
    S = np.einsum("mbik,nbik->mnbi", xs, qq)
    t = d[None, :, :, None].astype(np.float64) * sc[None].astype(np.float64) * S
    return t.sum(axis=(2, 3)) * x_scale.astype(np.float64)[:, None]


# ------------------------------------------- encoders of the reference tests
def q5k_quantize(w: np.ndarray):
    """fp32 [N,K] -> (bytes, deq): the encoder of reference tests/test_gemm_q4k.py:151-192."""
    N, K = w.shape
    nsb = K // QK_K
    x = w.astype(np.float32).reshape(N, nsb, 8, 32)
    xmax = x.max(axis=-1)
    xmin = np.maximum(0.0, -x.min(axis=-1))
    scale = (xmax + xmin) / 31.0
    scale = np.where(scale == 0, 1.0, scale)
    q = np.clip(np.rint((x + xmin[..., None]) / scale[..., None]), 0, 31).astype(np.uint8)
    d = scale.max(axis=-1) / 63.0
    dmin = xmin.max(axis=-1) / 63.0
    d = np.where(d == 0, 1.0, d)
    dmin = np.where(dmin == 0, 1.0, dmin)
    sc = np.clip(np.rint(scale / d[..., None]), 0, 63).astype(np.uint8)
    mn = np.clip(np.rint(xmin / dmin[..., None]), 0, 63).astype(np.uint8)
    blk = q5k_make(d.astype(np.float16), dmin.astype(np.float16), sc, mn, q)
    blk = blk.reshape(N, nsb * Q5K_BYTES)
    return blk, q5k_dequant(blk, K)


def q6k_quantize(w: np.ndarray):
    """fp32 [N,K] -> (bytes, deq): the encoder of reference tests/test_gemm_q4k.py:195-237."""
    N, K = w.shape
    nsb = K // QK_K
    x = w.astype(np.float32).reshape(N, nsb, 16, 16)
    a = np.abs(x).max(axis=-1)
    scale_f = np.where(a == 0, 1.0, a / 32.0)
    d = scale_f.max(axis=-1) / 127.0
    d = np.where(d == 0, 1.0, d)
    sc = np.clip(np.rint(scale_f / d[..., None]), -128, 127).astype(np.int8)
    d16 = d.astype(np.float16)
    rs = d16.astype(np.float32)[..., None] * sc.astype(np.float32)
    rs_safe = np.where(rs == 0, 1.0, rs)
    q = np.clip(np.rint(x / rs_safe[..., None]) + 32, 0, 63).astype(np.uint8).reshape(N, nsb, 256)
    blk = q6k_make(d16, sc, q).reshape(N, nsb * Q6K_BYTES)
    return blk, q6k_dequant(blk, K)

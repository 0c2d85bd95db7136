"""Q4_K super-block decode and GEMV (numpy restatement).

Block layout, 144 bytes per 256 weights (reference
csrc/include/gemm_q4k_dp4a.cuh:35-51, csrc/include/gemm_decode_dp4a.cuh:450-537,
tests/test_gemm_q4k.py:52-76,132-148; originally llama.cpp ggml-common.h
block_q4_K and get_scale_min_k4):
  [0:2] d fp16, [2:4] dmin fp16, [4:16] 12 bytes of packed 6-bit (sc, m) for
  8 sub-blocks, [16:144] 128 bytes of nibbles: byte 32*g + l holds element l
  of sub-block 2g (low nibble) and of sub-block 2g+1 (high nibble).
  w = fp32(d) * sc_j * q - fp32(dmin) * m_j   (exact in fp32).
GEMV: y[m,n] = x_scale[m] * sum_j (d*sc_j*<x_j,q_j> - dmin*m_j*sum(x_j)).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
from __future__ import annotations

import numpy as np

QK_K = 256
TYPE_SIZE = 144


def scale_min_k4(s12: np.ndarray):
    """get_scale_min_k4 over the last axis (12 bytes) -> (sc [...,8], m [...,8]) uint8."""
    s = s12.astype(np.uint16)
    sc = np.empty(s.shape[:-1] + (8,), np.uint16)
    mn = np.empty(s.shape[:-1] + (8,), np.uint16)
    sc[..., :4] = s[..., 0:4] & 63
    mn[..., :4] = s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 0xF) | ((s[..., 0:4] >> 6) << 4)
    mn[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    return sc.astype(np.uint8), mn.astype(np.uint8)


def pack_scale_min_k4(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Inverse of scale_min_k4: 8 six-bit scales and mins -> 12 bytes."""
    sc = sc.astype(np.uint16)
    mn = mn.astype(np.uint16)
    out = np.zeros(sc.shape[:-1] + (12,), np.uint16)
    out[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    out[..., 4:8] = (mn[..., 0:4] & 63) | ((mn[..., 4:8] >> 4) << 6)
    out[..., 8:12] = (sc[..., 4:8] & 0xF) | ((mn[..., 4:8] & 0xF) << 4)
    return out.astype(np.uint8)


def nibbles(qs: np.ndarray) -> np.ndarray:
    """128 qs bytes [...,128] -> codes [..., 8 sub-blocks, 32]."""
    g = qs.reshape(qs.shape[:-1] + (4, 32))
    q = np.empty(qs.shape[:-1] + (8, 32), np.uint8)
    q[..., 0::2, :] = g & 0xF
    q[..., 1::2, :] = g >> 4
    return q


def make_blocks(d: np.ndarray, dmin: np.ndarray, sc: np.ndarray, mn: np.ndarray,
                q: np.ndarray) -> np.ndarray:
    """Assemble blocks from fields: d, dmin fp16 [...], sc, mn [...,8], q [...,8,32] -> uint8 [...,144]."""
    lead = d.shape
    blk = np.zeros(lead + (TYPE_SIZE,), np.uint8)
    blk[..., 0:2] = np.ascontiguousarray(d.astype(np.float16)).view(np.uint8).reshape(lead + (2,))
    blk[..., 2:4] = np.ascontiguousarray(dmin.astype(np.float16)).view(np.uint8).reshape(lead + (2,))
    blk[..., 4:16] = pack_scale_min_k4(sc, mn)
    q = q.astype(np.uint8)
    qs = (q[..., 0::2, :] & 0xF) | ((q[..., 1::2, :] & 0xF) << 4)  # [...,4,32]
    blk[..., 16:144] = qs.reshape(lead + (128,))
    return blk


def random_weights(N: int, K: int, seed: int) -> np.ndarray:
    """Config-4 synthetic Q4_K bytes: d, dmin = fp16(|N(0,1)|*1e-2), sc/m uniform
    [0,63], nibbles uniform [0,15]. Returns uint8 [N, K/256*144]."""
    rng = np.random.default_rng(seed)
    nsb = K // QK_K
    d = (np.abs(rng.standard_normal((N, nsb))) * 1e-2).astype(np.float16)
    dmin = (np.abs(rng.standard_normal((N, nsb))) * 1e-2).astype(np.float16)
    sc = rng.integers(0, 64, (N, nsb, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, (N, nsb, 8), dtype=np.uint8)
    q = rng.integers(0, 16, (N, nsb, 8, 32), dtype=np.uint8)
    return make_blocks(d, dmin, sc, mn, q).reshape(N, nsb * TYPE_SIZE)


def fields(w: np.ndarray, K: int):
    """Split bytes [N, K/256*144] into (d fp32, dmin fp32 [N,nsb], sc, mn [N,nsb,8], q [N,nsb,8,32])."""
    N = w.shape[0]
    b = w.reshape(N, K // QK_K, TYPE_SIZE)
    d = b[..., 0:2].copy().view(np.float16).astype(np.float32)[..., 0]
    dmin = b[..., 2:4].copy().view(np.float16).astype(np.float32)[..., 0]
    sc, mn = scale_min_k4(b[..., 4:16])
    return d, dmin, sc, mn, nibbles(b[..., 16:144])


def dequant(w: np.ndarray, K: int) -> np.ndarray:
    """fp32 [N,K]: fp32(d)*sc*q - fp32(dmin)*m, two fp32 roundings as the kernels do."""
    d, dmin, sc, mn, q = fields(w, K)
    dsc = (d[..., None] * sc.astype(np.float32)).astype(np.float32)
    dm = (dmin[..., None] * mn.astype(np.float32)).astype(np.float32)
    out = (dsc[..., None] * q.astype(np.float32) - dm[..., None]).astype(np.float32)
    return out.reshape(w.shape[0], K)


def gemv(x_i8: np.ndarray, x_scale: np.ndarray, w: np.ndarray, K: int) -> np.ndarray:
    """y [M,N] in float64: x_scale[m] * sum_j(d*sc_j*S_j - dmin*m_j*X_j), integer sums exact."""
    d, dmin, sc, mn, q = fields(w, K)
    N, nsb = d.shape
    xs = x_i8.astype(np.float64).reshape(x_i8.shape[0], nsb, 8, 32)
    S = np.einsum("mbjk,nbjk->mnbj", xs, q.astype(np.float64))      # exact integer sums
    X = xs.sum(-1)                                                   # [M,nsb,8]
    t = (d[None, :, :, None].astype(np.float64) * sc[None].astype(np.float64) * S
         - dmin[None, :, :, None].astype(np.float64) * mn[None].astype(np.float64) * X[:, None])
    return t.sum(axis=(2, 3)) * x_scale.astype(np.float64)[:, None]


def gemv_xblock(x_i8: np.ndarray, x_scale_blk: np.ndarray, w: np.ndarray, K: int) -> np.ndarray:
    """y [M,N] float64 with one activation scale per 256-element block (x_scale_blk
    [M, K/256]): sum_b x_scale_blk[m,b] * sum_{j in b}(d*sc_j*S_j - dmin*m_j*X_j).
    Not in the reference (it has one scale per row, gemm_decode_dp4a.cu:398); the
    per-block form of BASELINE config 4. Equals gemv() when every block of a row
    carries the row's scale."""
    d, dmin, sc, mn, q = fields(w, K)
    N, nsb = d.shape
    xs = x_i8.astype(np.float64).reshape(x_i8.shape[0], nsb, 8, 32)
    S = np.einsum("mbjk,nbjk->mnbj", xs, q.astype(np.float64))
    X = xs.sum(-1)
    t = (d[None, :, :, None].astype(np.float64) * sc[None].astype(np.float64) * S
         - dmin[None, :, :, None].astype(np.float64) * mn[None].astype(np.float64) * X[:, None])
    return (t.sum(axis=3) * x_scale_blk.astype(np.float64)[:, None, :]).sum(axis=2)


"""Per-row int8 quantisation, K mean and quantize_qk (numpy restatement).

Reference: csrc/include/quant_rowwise.cuh:33-91 (scale = amax * fp32(1/127),
zero row -> 1, q = clamp(rint(x / scale), +-127) with correctly rounded fp32
division), superl8/quant/core.py:29-44,70-95 (K mean / smoothing),
core.py:164-196 (quantize_qk: fold softmax_scale*log2(e) into the Q scale),
superl8/quant/core.py:113-145 (outlier gate: any row with
max|q| / (median|q| + 1e-10) > ratio in fp32, median = the lower middle element),
csrc/include/attn_paged_decode.cuh:55-115 (quantize-on-write of one token per
paged row: scale = amax / 127 as an fp32 division, zero row -> 1, code =
rint(clamp(x / scale, +-127))).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
from __future__ import annotations

import math

import numpy as np

LOG2E = math.log2(math.e)
INV127 = np.float32(1.0) / np.float32(127.0)  # fp32(1/127), correctly rounded


# ---- bf16 helpers (bf16 carried as uint16 bit patterns) ----
def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round-to-nearest-even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def to_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_bits_to_f32(x)
    return x.astype(np.float32)


def round_to(x32: np.ndarray, dtype: str) -> np.ndarray:
    """Round fp32 values to the storage dtype, returned as fp32 values."""
    if dtype == "f16":
        return x32.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x32))
    return x32.astype(np.float32)


def quantize_rows(xf: np.ndarray, scale_mul: float = 1.0):
    """Per-row (last axis) symmetric int8 of fp32 values.

    Returns (q int8, scale fp32[...]) with scale = safe * fp32(scale_mul).
    Reference quant_rowwise.cuh:70-91 and core.py:195.
    """
    xf = np.asarray(xf, dtype=np.float32)
    amax = np.abs(xf).max(axis=-1) if xf.shape[-1] else np.zeros(xf.shape[:-1], np.float32)
    s = (amax.astype(np.float32) * INV127).astype(np.float32)
    safe = np.where(s == 0, np.float32(1.0), s).astype(np.float32)
    with np.errstate(invalid="ignore"):
        r = np.rint(xf / safe[..., None])  # fp32 division is correctly rounded in numpy
    q = np.clip(r, -127, 127).astype(np.int8)
    return q, (safe * np.float32(scale_mul)).astype(np.float32)


def quantize_row_groups(xf: np.ndarray, rows: int, scale_mul: float = 1.0):
    """One scale per `rows` consecutive rows (axis -2; the last group may be short)
    of fp32 values xf[..., N, D]: the row-wise formula with the group's amax.
    Returns (q int8 like xf, scale fp32 [..., N], each row holding its group's)."""
    xf = np.asarray(xf, dtype=np.float32)
    N = xf.shape[-2]
    q = np.empty(xf.shape, np.int8)
    sc = np.empty(xf.shape[:-1], np.float32)
    for r0 in range(0, N, rows):
        blk = xf[..., r0:r0 + rows, :]
        flat = blk.reshape(blk.shape[:-2] + (-1,))
        qq, ss = quantize_rows(flat, scale_mul)
        q[..., r0:r0 + rows, :] = qq.reshape(blk.shape)
        sc[..., r0:r0 + rows] = ss[..., None]
    return q, sc


def quantize_qk_per_wave(q: np.ndarray, k: np.ndarray, softmax_scale: float | None = None,
                         q_rows: int = 32, k_rows: int = 64, dtype: str = "f16"):
    """quantize_qk with per-tile scales (Q per q_rows queries, smoothed K per k_rows keys)."""
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    k_s, mean = smooth_k(k, dtype)
    q_i8, q_scale = quantize_row_groups(to_f32(q, dtype), q_rows, softmax_scale * LOG2E)
    k_i8, k_scale = quantize_row_groups(k_s, k_rows)
    return q_i8, q_scale, k_i8, k_scale, mean


def k_mean(k: np.ndarray, dtype: str = "f16") -> np.ndarray:
    """fp32 per-channel mean over axis -2 of k[..., N, D] (reference core.py:29-44).

    fp16: exact int64 sum of x * 2^24 (order independent), mean =
    fp32(double(sum) * 2^-24 / N). bf16/f32: fp64 running sum in row order,
    mean = fp32(sum / N). This is the order the GPU kernel uses.
    """
    N = k.shape[-2]
    if dtype == "f16":
        s = (k.astype(np.float64) * 2.0 ** 24).astype(np.int64).sum(axis=-2, keepdims=True)
        return ((s.astype(np.float64) * 2.0 ** -24) / N).astype(np.float32)
    kf = to_f32(k, dtype).astype(np.float64)
    s = np.zeros(kf.shape[:-2] + (1, kf.shape[-1]), np.float64)
    for n in range(N):
        s += kf[..., n:n + 1, :]
    return (s / N).astype(np.float32)


def smooth_k(k: np.ndarray, dtype: str = "f16"):
    """k_s = dtype(k - mean) (fp32 subtract, RN to dtype). Returns (k_s as fp32 values, mean)."""
    mean = k_mean(k, dtype)
    return round_to(to_f32(k, dtype) - mean, dtype), mean


def quantize_qk(q: np.ndarray, k: np.ndarray, softmax_scale: float | None = None,
                dtype: str = "f16"):
    """(q_i8, q_scale folded [..., M], k_i8, k_scale [..., N], k_mean). Reference core.py:164-196."""
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    k_s, mean = smooth_k(k, dtype)
    q_i8, q_scale = quantize_rows(to_f32(q, dtype), softmax_scale * LOG2E)
    k_i8, k_scale = quantize_rows(k_s)
    return q_i8, q_scale, k_i8, k_scale, mean


def quantize_v_perchannel(v: np.ndarray, dtype: str = "f16"):
    """Per-channel (over keys) int8 of V: scale = amax_n * fp32(1/127) -> (v_i8, v_scale [..., D]).
    Reference core.py:98-110 (on the GPU torch evaluates amax/127 as a reciprocal multiply)."""
    vf = to_f32(v, dtype)
    q, s = quantize_rows(np.swapaxes(vf, -1, -2))
    return np.swapaxes(q, -1, -2).copy(), s


def quantize_row_div(x: np.ndarray):
    """Per-row int8 with an IEEE-division scale (reference attn_paged_decode.cuh:74-110):
    scale = fp32(amax) / 127 (fp32), 1 for an all-zero row; code = rint(clamp(x / scale,
    -127, 127)). Rows are the last axis; returns (int8 codes, fp32 scales [...])."""
    xf = np.asarray(x, dtype=np.float32)
    amax = np.abs(xf).max(-1)
    scale = np.where(amax > 0, (amax / np.float32(127.0)).astype(np.float32), np.float32(1.0))
    scale = scale.astype(np.float32)
    y = (xf / scale[..., None]).astype(np.float32)
    q = np.rint(np.clip(y, -127.0, 127.0)).astype(np.int8)
    return q, scale


def kv_write_paged(k_new, v_new, slot_mapping, k_cache, k_scale, v_cache, v_scale):
    """Quantise one new token per (batch, KV head) and store it at the flat slot
    block * block_size + offset (reference attn_paged_decode.cuh:55-115); caches are
    updated in place: k_cache/v_cache int8 [num_blocks, Hkv, block_size, D],
    k_scale/v_scale fp32 [num_blocks, Hkv, block_size]; k_new/v_new [B, Hkv, D]."""
    bs = k_cache.shape[2]
    kq, ks = quantize_row_div(k_new)
    vq, vs = quantize_row_div(v_new)
    for b, slot in enumerate(np.asarray(slot_mapping).tolist()):
        blk, off = divmod(int(slot), bs)
        k_cache[blk, :, off] = kq[b]
        v_cache[blk, :, off] = vq[b]
        k_scale[blk, :, off] = ks[b]
        v_scale[blk, :, off] = vs[b]


def q_outlier_stats(q: np.ndarray):
    """Per-row max|q| and lower median |q| (the ((D-1)//2)-th smallest, torch.median's
    choice for even D) of the last axis, fp32 (reference quant/core.py:139-141)."""
    a = np.abs(np.asarray(q, dtype=np.float32))
    srt = np.sort(a, axis=-1)
    return a.max(-1), srt[..., (a.shape[-1] - 1) // 2]


def q_outlier_gate(q: np.ndarray, ratio_threshold: float = 12.0) -> bool:
    """True when any row has max / (median + 1e-10) > ratio_threshold, evaluated in
    fp32 (reference quant/core.py:113-145)."""
    mx, md = q_outlier_stats(q)
    ratio = (mx / (md + np.float32(1e-10))).astype(np.float32)
    return bool((ratio > np.float32(ratio_threshold)).any())

"""3-bit Lloyd-Max V store of the K8V3 paged decode (numpy restatement).

Reference restated:
  superl8/quant/lloydmax.py:41-65 (fixed codebook: the 8 N(0,1) Lloyd-Max
      levels times block_size^-1/2, formed in double precision, stored fp32)
  superl8/quant/lloydmax.py:118-145 (block L2 norm, zero norm -> 1, code =
      torch.bucketize of x / norm against the level midpoints: a value equal
      to a midpoint takes the lower code)
  superl8/quant/lloydmax.py:196-219 (3-bit codes packed LSB-first into int32
      words: code i at bits 3i..3i+2 of the row's stream)
  csrc/include/attn_paged_decode.cuh:214-236 (the kernel's value:
      fp16_rn(fp32(codebook[code] * norm[d / 128])), the product rounded to
      fp32 first, then to fp16)
  csrc/include/attn_paged_decode.cuh:134-257 (the K8V3 paged split kernel:
      the paged int8-K decode with that V and no V scale)

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
from __future__ import annotations

import numpy as np

from . import attention as oa

STDNORMAL_LM8 = (-2.152135, -1.343909, -0.756096, -0.245098,
                 0.245098, 0.756096, 1.343909, 2.152135)


def gaussian_codebook(block_size: int = 128) -> np.ndarray:
    """lloydmax.py:56-65: level * block_size**-0.5 in double, stored fp32."""
    sigma = block_size ** -0.5
    return np.array([c * sigma for c in STDNORMAL_LM8], dtype=np.float32)


def quantize(x: np.ndarray, codebook: np.ndarray, block_size: int = 128):
    """lloydmax.py:118-145 over the last axis: -> (codes uint8, norms fp32 [..., D/bs]).
    Norms are summed in float64 and rounded to fp32 (the reference sums in fp32:
    norms may differ in the last bit; codes use these norms)."""
    xf = x.astype(np.float32)
    d = xf.shape[-1]
    xb = xf.reshape(*xf.shape[:-1], d // block_size, block_size)
    norm = np.sqrt((xb.astype(np.float64) ** 2).sum(-1)).astype(np.float32)
    norm = np.where(norm == 0, np.float32(1.0), norm)
    unit = xb / norm[..., None]
    bounds = (np.float32(0.5) * (codebook[1:] + codebook[:-1])).astype(np.float32)
    codes = np.searchsorted(bounds, unit, side="left").astype(np.uint8)
    return codes.reshape(xf.shape), norm


def pack3(codes: np.ndarray) -> np.ndarray:
    """lloydmax.py:203-212: codes [..., D] (0..7) -> int32 words [..., 3D/32]."""
    d = codes.shape[-1]
    assert (3 * d) % 32 == 0
    c = codes.reshape(-1, d).astype(np.uint64)
    words = np.zeros((c.shape[0], 3 * d // 32), dtype=np.uint64)
    for i in range(d):
        for bit in range(3):
            pos = 3 * i + bit
            words[:, pos // 32] |= ((c[:, i] >> np.uint64(bit)) & np.uint64(1)) << np.uint64(pos % 32)
    return words.astype(np.uint32).view(np.int32).reshape(*codes.shape[:-1], 3 * d // 32)


def unpack3(words: np.ndarray, d: int) -> np.ndarray:
    """lloydmax.py:215-219 (and the kernel's extraction, attn_paged_decode.cuh:226-233)."""
    w = words.reshape(-1, words.shape[-1]).view(np.uint32).astype(np.uint64)
    codes = np.zeros((w.shape[0], d), dtype=np.uint8)
    for i in range(d):
        pos = 3 * i
        lo = (w[:, pos // 32] >> np.uint64(pos % 32))
        if pos % 32 > 29:
            lo = lo | (w[:, pos // 32 + 1] << np.uint64(32 - pos % 32))
        codes[:, i] = (lo & np.uint64(7)).astype(np.uint8)
    return codes.reshape(*words.shape[:-1], d)


def dequant_fp16(codes: np.ndarray, norms: np.ndarray, codebook: np.ndarray) -> np.ndarray:
    """attn_paged_decode.cuh:234: fp16_rn(fp32(codebook[code] * norm[d // 128])) as float32."""
    d = codes.shape[-1]
    nrm = np.repeat(norms.astype(np.float32), 128, axis=-1)[..., :d]
    prod = codebook.astype(np.float32)[codes.astype(np.int64)] * nrm  # fp32 product
    return prod.astype(np.float32).astype(np.float16).astype(np.float32)


def attn_paged_decode_k8v3(q_i8, q_scale, k_cache, k_scale, v_packed, v_norm, codebook,
                           block_table, context_lens, max_context_len, num_splits):
    """attn_paged_decode.cuh:134-257 (LowbitV): the paged decode with V rows
    dequantised as above and no per-token V scale. Returns [B,Hq,D] float64."""
    D = k_cache.shape[-1]
    v = dequant_fp16(unpack3(v_packed, D), v_norm, codebook)
    ones = np.ones(k_scale.shape, dtype=np.float32)
    return oa.attn_paged_decode(q_i8, q_scale, k_cache, k_scale, v, ones, block_table,
                                context_lens, max_context_len, num_splits)

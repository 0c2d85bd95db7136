"""Quantisation prologue of the int8 attention path, on the gfx950 kernels.

Restates superl8/quant/core.py of the reference with the same functions,
arguments and return shapes. The numerics contract (reference
core.py:47-62,70-110,164-196 and csrc/include/quant_rowwise.cuh:33-91):

  * per-row symmetric int8: scale = amax * fp32(1/127), 1 for a zero row;
    q = clamp(rint(x / scale), -127, 127) with IEEE division;
  * K-smoothing: k_s = dtype(k - mean_n(k)) with an fp32 per-channel mean;
  * quantize_qk folds softmax_scale * log2(e) into the Q scale (fp32 multiply)
    so the attention kernels work in the exp2 domain.

The key mean is computed order-independently (exact integer sum for fp16 keys),
where the reference sums 1024-key chunks in torch's reduction order; softmax
is invariant to the shift, so attention outputs are unaffected.

These functions run only on GPU tensors; there is no CPU implementation in the
product (the CPU restatement used to check it lives in the test oracle).
"""
from __future__ import annotations

import math

import torch

from .. import _C

LOG2E = math.log2(math.e)
Q_MAX = 127.0


def _need_gpu(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"superl8: {what} runs on the GPU kernels only; got a {t.device} tensor")


def quantize_int8_rowwise(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-row RTN int8. Returns (q int8 [..., d], scale fp32 [..., 1])."""
    _need_gpu(x, "quantize_int8_rowwise")
    shape = x.shape
    q, scale = _C.quantize_i8_rowwise(x.reshape(-1, shape[-1]))
    return q.reshape(shape), scale.reshape(*shape[:-1], 1)


def dequantize_int8_rowwise(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """Inverse of quantize_int8_rowwise (fp32 out)."""
    return q.float() * scale


def smooth_k(k: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Subtract K's per-channel mean over keys. Returns (k_smoothed [..., n, d], k_mean [..., 1, d])."""
    _need_gpu(k, "smooth_k")
    k_mean = _C.k_mean(k)
    k_s = torch.empty_like(k)
    torch.sub(k, k_mean, out=k_s)  # fp32 subtract, rounded to k's dtype
    return k_s, k_mean


def quantize_v_perchannel(v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-channel int8 for V (scale over keys). Returns (v_int8, v_scale [..., 1, d])."""
    _need_gpu(v, "quantize_v_perchannel")
    q, scale = _C.quantize_v_perchannel(v)
    return q, scale


def quantize_v_rowwise(v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-token int8 for V (scale per key)."""
    return quantize_int8_rowwise(v)


def detect_q_outlier_domination(q: torch.Tensor, *, ratio_threshold: float = 12.0) -> bool:
    """True when any Q row has max|q| / median|q| > ratio_threshold (reference core.py:113-145).

    One gate kernel (max and exact lower median per row, flag by atomic OR)
    decides on the GPU for head dims up to 256 (every dim the kernels accept);
    wider rows use torch ops.
    Skipped (False) while the current stream is capturing a graph, because the
    decision needs a device-to-host read.
    """
    try:
        if torch.cuda.is_current_stream_capturing():
            return False
    except Exception:
        pass
    if q.is_cuda and 1 <= q.shape[-1] <= _C._GATE_MAX_D:
        flag, _ = _C.q_outlier_gate(q, ratio_threshold)
        return bool(flag.item())
    q_abs = q.float().abs()
    row_max = q_abs.amax(dim=-1)
    row_med = q_abs.median(dim=-1).values
    return bool(((row_max / (row_med + 1e-10)) > ratio_threshold).any())


def _fused_ok(q: torch.Tensor, k: torch.Tensor) -> bool:
    """Shapes the fused fp16 prologue (sl8_quantize_qk) serves."""
    return (q.dtype == torch.float16 and k.dtype == torch.float16 and q.dim() == 4
            and k.dim() == 4 and q.shape[-1] == k.shape[-1] and q.shape[-1] in (64, 128, 256)
            and q.shape[0] == k.shape[0] and q.numel() > 0 and k.numel() > 0
            and k.shape[-2] < (1 << 23))


def quantize_qk_gated(q: torch.Tensor, k: torch.Tensor, *, softmax_scale: float | None = None,
                      rotate: bool = False, ratio_threshold: float = 12.0, defer: bool = False):
    """The attention prologue with the outlier gate (reference ops.py:115-150).

    Returns (fired, quantize_qk's five outputs or None). fired is
    detect_q_outlier_domination(q); when it holds the quantised tensors are
    not needed (the caller routes to full precision). For fp16 Q/K without
    rotation the gate is decided inside the fused prologue (one flag read);
    otherwise it is evaluated first and quantize_qk runs only when it passes.
    Under graph capture the gate is skipped (False), as in
    detect_q_outlier_domination. With defer=True the fused path returns the
    device flag (int32 [1]) in place of fired, unread, with the quantised
    tensors: the caller reads it later (the other paths still return a bool).
    """
    _need_gpu(q, "quantize_qk")
    try:
        capturing = torch.cuda.is_current_stream_capturing()
    except Exception:
        capturing = False
    if not rotate and not capturing and _fused_ok(q, k):
        s = (1.0 / math.sqrt(q.shape[-1])) if softmax_scale is None else softmax_scale
        q_i8, q_scale, k_i8, k_scale, k_mean, flag = _C.quantize_qk_fused(
            q, k, s * LOG2E, ratio_threshold)
        if defer:
            return flag, (q_i8, q_scale.unsqueeze(-1), k_i8, k_scale.unsqueeze(-1), k_mean)
        if bool(flag.item()):
            return True, None
        return False, (q_i8, q_scale.unsqueeze(-1), k_i8, k_scale.unsqueeze(-1), k_mean)
    if detect_q_outlier_domination(q, ratio_threshold=ratio_threshold):
        return True, None
    return False, quantize_qk(q, k, softmax_scale=softmax_scale, rotate=rotate)


def quantize_qk(q: torch.Tensor, k: torch.Tensor, *, softmax_scale: float | None = None,
                rotate: bool = False):
    """Quantise Q and smoothed K for the int8 QK^T.

    Returns (q_int8, q_scale[..., m, 1] folded with softmax_scale*log2(e),
    k_int8, k_scale[..., n, 1], k_mean[..., 1, d]). fp16 Q/K without rotation
    take the fused prologue (three launches); otherwise the K mean and the
    smooth-and-quantise of each side are separate kernels (the smoothed K is
    never written either way).
    """
    _need_gpu(q, "quantize_qk")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    if not rotate and _fused_ok(q, k):
        q_i8, q_scale, k_i8, k_scale, k_mean, _ = _C.quantize_qk_fused(q, k, softmax_scale * LOG2E)
        return q_i8, q_scale.unsqueeze(-1), k_i8, k_scale.unsqueeze(-1), k_mean
    if rotate:
        from .rotation import rotate_last

        k_s, k_mean = smooth_k(k)
        q = rotate_last(q)
        k_src, mean = rotate_last(k_s), None
    else:
        k_mean = _C.k_mean(k)
        k_src, mean = k, k_mean
    q_i8, q_scale = _C.quantize_rows_centered(q, None, softmax_scale * LOG2E)
    k_i8, k_scale = _C.quantize_rows_centered(k_src, mean, 1.0)
    return q_i8, q_scale.unsqueeze(-1), k_i8, k_scale.unsqueeze(-1), k_mean


def quantize_qk_per_wave(q: torch.Tensor, k: torch.Tensor, *, softmax_scale: float | None = None,
                         q_rows: int = 32, k_rows: int = 64):
    """quantize_qk with one scale per tile of rows instead of per row: Q per
    `q_rows` queries (one wavefront's query tile of the prefill kernels, 32) and
    the smoothed K per `k_rows` keys (one key tile, 64) -- the per-wavefront
    scheme of BASELINE config 5 (the reference quantises Q/K per row,
    core.py:164-196). Same outputs as quantize_qk; every row carries its tile's
    scale, so the attention kernels run unchanged."""
    _need_gpu(q, "quantize_qk_per_wave")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    k_mean = _C.k_mean(k)
    q_i8, q_scale = _C.quantize_row_groups(q, q_rows, None, softmax_scale * LOG2E)
    k_i8, k_scale = _C.quantize_row_groups(k, k_rows, k_mean, 1.0)
    return q_i8, q_scale.unsqueeze(-1), k_i8, k_scale.unsqueeze(-1), k_mean


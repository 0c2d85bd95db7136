"""`superl8._C` operator surface, served by libsuperl8_hip.so through its C ABI.

Each function keeps the name, positional/keyword signature, output
allocation and argument checks of the reference pybind11 binding it replaces
(reference csrc/fni8_api.cpp). Outputs and scratch are allocated here with
torch (the caching allocator); the kernels are enqueued on torch's current
stream of the input's device. Error messages keep the reference's key
phrases, and every failure raises RuntimeError.

There is no CPU implementation: a non-GPU tensor is rejected, exactly like the
reference's "must be CUDA tensors" checks.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from ._lib import call, dtype_code, stream_of

# reference csrc/kernel/attn_int8_fwd.cu:138, attn_w8a8_fwd.cu:113, attn_decode.cu:195
_HEAD_DIMS_FWD = (32, 64, 72, 80, 128, 256)
_HEAD_DIMS_W8A8 = (32, 64, 128, 256)
_HEAD_DIMS_DECODE = (32, 64, 128, 256)


def _dims_msg(dims) -> str:
    return "/".join(str(d) for d in dims)
DEC_MAX_SPLITS = 256
DEC_MAX_M = 16
Q4K_TYPE_SIZE = 144
Q5K_TYPE_SIZE = 176
Q6K_TYPE_SIZE = 210


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(f"fni8: {msg}")


def _on_gpu(*ts: torch.Tensor) -> None:
    _check(all(t.is_cuda for t in ts), "all inputs (incl. scales) must be CUDA tensors")
    dev = ts[0].device
    _check(all(t.device == dev for t in ts), "all inputs must be on the same device")


def _contig(*ts: torch.Tensor) -> None:
    _check(all(t.is_contiguous() for t in ts), "inputs must be contiguous")


# ---------------------------------------------------------------------------
# quantisation (reference csrc/kernel/quant_rowwise.cu:84-121)
# ---------------------------------------------------------------------------
def quantize_i8_rowwise(x: torch.Tensor):
    """x[M,K] fp16/bf16/fp32 -> (q int8 [M,K], scale fp32 [M])."""
    _check(x.is_cuda, "quantize_i8_rowwise expects a CUDA tensor")
    _check(x.dim() == 2, f"expect x[M,K], got dim={x.dim()}")
    _check(x.dtype in (torch.float16, torch.bfloat16, torch.float32),
           "quantize_i8_rowwise input must be float16/bfloat16/float32")
    x = x.contiguous()
    M, K = x.shape
    q = torch.empty((M, K), device=x.device, dtype=torch.int8)
    scale = torch.empty((M,), device=x.device, dtype=torch.float32)
    if M and K:
        with torch.cuda.device(x.device):
            call("sl8_quantize_i8_rowwise", x.data_ptr(), dtype_code(x.dtype), M, K,
                 q.data_ptr(), scale.data_ptr(), stream_of(x))
    return q, scale


def k_mean(k: torch.Tensor) -> torch.Tensor:
    """fp32 mean over the key axis of k[..., N, D] -> [..., 1, D] (order-independent)."""
    _check(k.is_cuda, "k_mean expects a CUDA tensor")
    _check(k.dtype in (torch.float16, torch.bfloat16, torch.float32),
           "k_mean input must be float16/bfloat16/float32")
    k = k.contiguous()
    *lead, N, D = k.shape
    G = math.prod(lead)
    mean = torch.empty((*lead, 1, D), device=k.device, dtype=torch.float32)
    if G and D:
        ws_bytes = _lib.load().sl8_k_mean_workspace(G, D)
        ws = torch.empty((max(ws_bytes, 8),), device=k.device, dtype=torch.uint8)
        with torch.cuda.device(k.device):
            call("sl8_k_mean", k.data_ptr(), dtype_code(k.dtype), G, N, D, mean.data_ptr(),
                 ws.data_ptr(), ws_bytes, stream_of(k))
    return mean


def quantize_rows_centered(x: torch.Tensor, mean: torch.Tensor | None, scale_mul: float = 1.0):
    """Fused smooth + per-row int8 of x[..., N, D]: rows of group g have
    mean[g] subtracted (rounded back to x's dtype) before quantising; the
    returned scale [..., N] is multiplied by fp32(scale_mul)."""
    _check(x.is_cuda, "quantize expects a CUDA tensor")
    _check(x.dtype in (torch.float16, torch.bfloat16, torch.float32),
           "quantize input must be float16/bfloat16/float32")
    x = x.contiguous()
    *lead, N, D = x.shape
    G = math.prod(lead)
    if mean is not None:
        mean = mean.to(torch.float32).contiguous()
        _check(mean.numel() == G * D, "mean shape mismatch")
    q = torch.empty(x.shape, device=x.device, dtype=torch.int8)
    scale = torch.empty((*lead, N), device=x.device, dtype=torch.float32)
    if G and N and D:
        with torch.cuda.device(x.device):
            call("sl8_quantize_i8_rows_centered", x.data_ptr(), dtype_code(x.dtype), G, N, D,
                 None if mean is None else mean.data_ptr(), float(scale_mul), q.data_ptr(),
                 scale.data_ptr(), stream_of(x))
    return q, scale


def quantize_row_groups(x: torch.Tensor, rows_per_group: int, mean: torch.Tensor | None = None,
                        scale_mul: float = 1.0):
    """int8 of x[..., N, D] with one scale per `rows_per_group` consecutive rows
    (groups restart at every leading index; mean as quantize_rows_centered).
    Returns (q int8 like x, scale fp32 [..., N]: each row holds its group's scale)."""
    _check(x.is_cuda, "quantize expects a CUDA tensor")
    _check(x.dtype in (torch.float16, torch.bfloat16, torch.float32),
           "quantize input must be float16/bfloat16/float32")
    _check(rows_per_group >= 1, "rows_per_group must be >= 1")
    x = x.contiguous()
    *lead, N, D = x.shape
    G = math.prod(lead)
    if mean is not None:
        mean = mean.to(torch.float32).contiguous()
        _check(mean.numel() == G * D, "mean shape mismatch")
    q = torch.empty(x.shape, device=x.device, dtype=torch.int8)
    scale = torch.empty((*lead, N), device=x.device, dtype=torch.float32)
    if G and N and D:
        with torch.cuda.device(x.device):
            call("sl8_quantize_i8_row_groups", x.data_ptr(), dtype_code(x.dtype), G, N, D,
                 int(rows_per_group), None if mean is None else mean.data_ptr(),
                 float(scale_mul), q.data_ptr(), scale.data_ptr(), stream_of(x))
    return q, scale


def quantize_qk_fused(q: torch.Tensor, k: torch.Tensor, q_scale_mul: float,
                      gate_ratio: float = 0.0):
    """Fused fp16 prologue: q [B,Hq,M,D], k [B,Hkv,N,D] -> (q_i8, q_scale [B,Hq,M],
    k_i8, k_scale [B,Hkv,N], k_mean fp32 [B,Hkv,1,D], flag int32 [1] or None).

    K is smoothed by its exact per-channel mean, q_scale carries q_scale_mul;
    with gate_ratio > 0, flag = 1 when some Q row has max/(median+1e-10) above it."""
    _on_gpu(q, k)
    _check(q.dtype == torch.float16 and k.dtype == torch.float16,
           "fused prologue expects float16 q and k")
    _check(q.dim() == 4 and k.dim() == 4 and q.shape[-1] == k.shape[-1],
           "fused prologue expects q[B,Hq,M,D], k[B,Hkv,N,D]")
    q, k = q.contiguous(), k.contiguous()
    B, Hq, M, D = q.shape
    _, Hkv, N, _ = k.shape
    qrows, G = B * Hq * M, B * Hkv
    q_i8 = torch.empty(q.shape, device=q.device, dtype=torch.int8)
    q_scale = torch.empty((B, Hq, M), device=q.device, dtype=torch.float32)
    k_i8 = torch.empty(k.shape, device=k.device, dtype=torch.int8)
    k_scale = torch.empty((B, Hkv, N), device=k.device, dtype=torch.float32)
    k_mean = torch.empty((B, Hkv, 1, D), device=k.device, dtype=torch.float32)
    flag = torch.empty((1,), device=q.device, dtype=torch.int32) if gate_ratio > 0 else None
    ws_bytes = _lib.load().sl8_quantize_qk_workspace(qrows, G, N, D)
    ws = torch.empty((max(ws_bytes, 8),), device=q.device, dtype=torch.uint8)
    with torch.cuda.device(q.device):
        call("sl8_quantize_qk", q.data_ptr(), k.data_ptr(), dtype_code(q.dtype), qrows, G, N, D,
             float(q_scale_mul), float(gate_ratio), q_i8.data_ptr(), q_scale.data_ptr(),
             k_i8.data_ptr(), k_scale.data_ptr(), k_mean.data_ptr(),
             None if flag is None else flag.data_ptr(), ws.data_ptr(), ws_bytes, stream_of(q))
    return q_i8, q_scale, k_i8, k_scale, k_mean, flag


_GATE_MAX_D = 256


def q_outlier_gate(q: torch.Tensor, ratio: float = 12.0, *, stats: bool = False):
    """On-device outlier gate over the rows of q[..., D] (D up to 256).

    Returns (flag int32 [1], stats fp32 [rows, 2] or None): flag is 1 when some
    row has max|q| / (median|q| + 1e-10) > ratio (fp32, median = lower middle
    element, as torch.median); stats holds each row's (max, median)."""
    _check(q.is_cuda, "q_outlier_gate expects a CUDA tensor")
    _check(q.dtype in (torch.float16, torch.bfloat16, torch.float32),
           "q_outlier_gate input must be float16/bfloat16/float32")
    D = q.shape[-1]
    _check(1 <= D <= _GATE_MAX_D, f"q_outlier_gate supports head dims 1..{_GATE_MAX_D}, got {D}")
    q = q.contiguous()
    rows = q.numel() // D
    flag = torch.zeros((1,), device=q.device, dtype=torch.int32)
    st = torch.empty((rows, 2), device=q.device, dtype=torch.float32) if stats else None
    if rows:
        with torch.cuda.device(q.device):
            call("sl8_q_outlier_gate", q.data_ptr(), dtype_code(q.dtype), rows, D, float(ratio),
                 flag.data_ptr(), None if st is None else st.data_ptr(), stream_of(q))
    return flag, st


def quantize_v_perchannel(v: torch.Tensor):
    """Per-channel int8 of v[..., N, D] over N -> (q int8 [..., N, D], scale fp32 [..., 1, D])."""
    _check(v.is_cuda, "quantize_v_perchannel expects a CUDA tensor")
    _check(v.dtype in (torch.float16, torch.bfloat16, torch.float32),
           "quantize_v_perchannel input must be float16/bfloat16/float32")
    v = v.contiguous()
    *lead, N, D = v.shape
    G = math.prod(lead)
    q = torch.empty(v.shape, device=v.device, dtype=torch.int8)
    scale = torch.empty((*lead, 1, D), device=v.device, dtype=torch.float32)
    if G and D:
        with torch.cuda.device(v.device):
            call("sl8_quantize_i8_cols", v.data_ptr(), dtype_code(v.dtype), G, N, D, q.data_ptr(),
                 scale.data_ptr(), stream_of(v))
    return q, scale


# ---------------------------------------------------------------------------
# prefill attention (reference csrc/kernel/attn_int8_fwd.cu:101-200)
# ---------------------------------------------------------------------------
def _fwd_checks(q, q_scale, k, k_scale, v):
    _on_gpu(q, q_scale, k, k_scale, v)
    _check(q.dtype == torch.int8 and k.dtype == torch.int8, "q/k must be int8")
    _check(q_scale.dtype == torch.float32 and k_scale.dtype == torch.float32,
           "scales must be float32")
    _check(q.dim() == 4 and k.dim() == 4 and v.dim() == 4, "expect [B,H,S,D]")
    _contig(q, q_scale, k, k_scale, v)
    _check(q.data_ptr() % 4 == 0 and k.data_ptr() % 4 == 0,
           "q/k must be 4-byte aligned for int32 loads")
    B, H, M, D = q.shape
    N, Hkv = k.shape[2], k.shape[1]
    _check(k.shape[0] == B and v.shape[0] == B and v.shape[1] == Hkv, "batch/head mismatch")
    _check(Hkv > 0 and H % Hkv == 0, "H_q must be divisible by H_kv (GQA)")
    _check(k.shape[3] == D and v.shape[3] == D and v.shape[2] == N, "K/V shape mismatch")
    return B, H, Hkv, M, N, D


def _attn_fwd(q, q_scale, k, k_scale, v, causal, window_left, want_lse, gate_flag=None):
    B, H, Hkv, M, N, D = _fwd_checks(q, q_scale, k, k_scale, v)
    _check(v.dtype in (torch.float16, torch.bfloat16), "v must be float16 or bfloat16")
    _check(q_scale.numel() == B * H * M and k_scale.numel() == B * Hkv * N, "scale shape mismatch")
    _check(D in _HEAD_DIMS_FWD, f"head dim must be {_dims_msg(_HEAD_DIMS_FWD)}, got {D}")
    out = torch.empty((B, H, M, D), device=v.device, dtype=v.dtype)
    lse = torch.empty((B, H, M) if want_lse else (0,), device=q.device, dtype=torch.float32)
    if M == 0 or B == 0 or H == 0:
        return out, lse
    ws_bytes = _lib.load().sl8_attn_int8_fwd_workspace(B, H, Hkv, M, N, D)
    ws = torch.empty((ws_bytes,), device=q.device, dtype=torch.uint8) if ws_bytes else None
    args = (q.data_ptr(), q_scale.data_ptr(), k.data_ptr(), k_scale.data_ptr(), v.data_ptr(),
            dtype_code(v.dtype), out.data_ptr(), lse.data_ptr() if want_lse else None,
            B, H, Hkv, M, N, D, int(bool(causal)), int(window_left),
            ws.data_ptr() if ws is not None else None, ws_bytes)
    with torch.cuda.device(q.device):
        if gate_flag is None:
            call("sl8_attn_int8_fwd", *args, stream_of(q))
        else:
            _check(gate_flag.is_cuda and gate_flag.dtype == torch.int32 and gate_flag.numel() >= 1,
                   "gate_flag must be a CUDA int32 tensor")
            call("sl8_attn_int8_fwd_gated", *args, gate_flag.data_ptr(), stream_of(q))
    return out, lse


def attn_int8_fwd(q, q_scale, k, k_scale, v, causal=False, window_left=-1, *, gate_flag=None):
    """q int8 [B,Hq,M,D], q_scale fp32 [B,Hq,M] (folded), k int8 [B,Hkv,N,D],
    k_scale fp32 [B,Hkv,N], v fp16/bf16 [B,Hkv,N,D] -> out [B,Hq,M,D] (v's dtype).

    gate_flag (this build only): a CUDA int32 tensor written earlier on the
    stream; when it holds a nonzero value the kernel exits at once and the
    output is left unwritten (the caller discards it)."""
    return _attn_fwd(q, q_scale, k, k_scale, v, causal, window_left, False, gate_flag)[0]


def attn_int8_fwd_train(q, q_scale, k, k_scale, v, causal=False):
    """Same forward, also returns the natural-log LSE fp32 [B,Hq,M]."""
    return _attn_fwd(q, q_scale, k, k_scale, v, causal, -1, True)


def attn_int8_qk_scores(q, k, causal=False, fill=0):
    """int32 Q.K^T [B,Hq,M,N] from the production prefill kernel's own MFMA tiles
    (its score-dump instantiation; test hook). causal=True runs the causal
    kernel, which only computes key tiles a wave can see: entries it does not
    store keep `fill`."""
    _on_gpu(q, k)
    _check(q.dtype == torch.int8 and k.dtype == torch.int8, "q/k must be int8")
    _contig(q, k)
    B, H, M, D = q.shape
    Hkv, N = k.shape[1], k.shape[2]
    _check(Hkv > 0 and H % Hkv == 0 and k.shape[3] == D and k.shape[0] == B, "q/k shape mismatch")
    _check(D in _HEAD_DIMS_FWD, f"head dim must be {_dims_msg(_HEAD_DIMS_FWD)}, got {D}")
    s = torch.full((B, H, M, N), fill, device=q.device, dtype=torch.int32)
    if s.numel():
        ws_bytes = _lib.load().sl8_attn_int8_fwd_workspace(B, H, Hkv, M, N, D)
        ws = torch.empty((ws_bytes,), device=q.device, dtype=torch.uint8) if ws_bytes else None
        with torch.cuda.device(q.device):
            call("sl8_attn_int8_qk_scores", q.data_ptr(), k.data_ptr(), s.data_ptr(), B, H, Hkv,
                 M, N, D, int(bool(causal)), ws.data_ptr() if ws is not None else None, ws_bytes,
                 stream_of(q))
    return s


# ---------------------------------------------------------------------------
# W8A8 prefill (reference csrc/kernel/attn_w8a8_fwd.cu:76-165)
# ---------------------------------------------------------------------------
def attn_w8a8_fwd(q, q_scale, k, k_scale, v, v_scale, causal=False, causal_diag=0,
                  per_warp_quant=True, *, exact_pv=False):
    """int8 QK^T + int8 PV; v int8 [B,Hkv,N,D], v_scale fp32 [B,Hkv,D] -> fp16 out.

    exact_pv (keyword of this build only; per_warp_quant=True): the reference's
    per-warp arithmetic exactly -- an int32 P.V per 32-key half scaled in fp32 --
    instead of the default bf16-P MFMA pipeline, at about twice the time."""
    _on_gpu(v_scale)
    B, H, Hkv, M, N, D = _fwd_checks(q, q_scale, k, k_scale, v)
    _check(v.dtype == torch.int8, "q/k/v must be int8")
    _check(v_scale.dtype == torch.float32, "scales must be float32")
    _contig(v_scale)
    _check(q_scale.numel() == B * H * M and k_scale.numel() == B * Hkv * N
           and v_scale.numel() == B * Hkv * D, "scale shape mismatch")
    _check(D in _HEAD_DIMS_W8A8, f"head dim must be {_dims_msg(_HEAD_DIMS_W8A8)}, got {D}")
    out = torch.empty((B, H, M, D), device=q.device, dtype=torch.float16)
    if M == 0 or B == 0 or H == 0:
        return out
    ws_bytes = _lib.load().sl8_attn_w8a8_fwd_workspace(B, H, Hkv, M, N, D)
    ws = torch.empty((max(ws_bytes, 1),), device=q.device, dtype=torch.uint8)
    with torch.cuda.device(q.device):
        call("sl8_attn_w8a8_fwd", q.data_ptr(), q_scale.data_ptr(), k.data_ptr(),
             k_scale.data_ptr(), v.data_ptr(), v_scale.data_ptr(), out.data_ptr(), B, H, Hkv, M,
             N, D, int(bool(causal)), int(causal_diag),
             (2 if exact_pv else 1) if per_warp_quant else 0,
             ws.data_ptr(), ws_bytes, stream_of(q))
    return out


# ---------------------------------------------------------------------------
# split-KV decode (reference csrc/kernel/attn_decode.cu:163-240)
# ---------------------------------------------------------------------------
def choose_n_splits(n_len: int, batch: int, h_kv: int) -> int:
    return int(_lib.load().sl8_choose_num_splits(n_len, batch, h_kv))


def attn_int8_decode(q, q_scale, k, k_scale, v, num_splits=-1):
    """q int8 [B,Hq,1,D], q_scale fp32 [B,Hq,1], k int8 [B,Hkv,N,D], k_scale fp32
    [B,Hkv,N], v fp16 [B,Hkv,N,D] -> fp16 [B,Hq,1,D].

    k_scale may also be fp16 (a cache with half-size per-token scales, BASELINE
    config 3): the kernels widen it to fp32 exactly and compute as before."""
    _on_gpu(q, q_scale, k, k_scale, v)
    _check(q.dtype == torch.int8 and k.dtype == torch.int8, "decode: q/k must be int8")
    _check(q_scale.dtype == torch.float32 and k_scale.dtype in (torch.float32, torch.float16),
           "decode: scales must be float32")
    _check(v.dtype == torch.float16, "decode: v must be float16")
    _check(q.dim() == 4 and k.dim() == 4 and v.dim() == 4, "decode: expect [B,H,S,D]")
    _check(q.shape[2] == 1, "decode: query length M must be 1 (decode)")
    _contig(q, q_scale, k, k_scale, v)
    B, H, _, D = q.shape
    Hkv, N = k.shape[1], k.shape[2]
    _check(k.shape[0] == B and v.shape[0] == B and v.shape[1] == Hkv, "decode: batch/head mismatch")
    _check(Hkv > 0 and H % Hkv == 0, "decode: H_q must be divisible by H_kv (GQA)")
    _check(k.shape[3] == D and v.shape[3] == D and v.shape[2] == N, "decode: K/V shape mismatch")
    _check(q_scale.numel() == B * H and k_scale.numel() == B * Hkv * N,
           "decode: scale shape mismatch")
    _check(D in _HEAD_DIMS_DECODE, f"decode: head dim must be {_dims_msg(_HEAD_DIMS_DECODE)}, got {D}")
    num_splits = int(num_splits)
    _check(num_splits != 0, f"decode: num_splits=0 is invalid; use -1 for auto or 1..{DEC_MAX_SPLITS}")
    out = torch.empty((B, H, 1, D), device=v.device, dtype=torch.float16)
    if B == 0 or H == 0:
        return out
    if N == 0:
        return out.zero_()
    ns = choose_n_splits(N, B, Hkv) if num_splits < 0 else num_splits
    _check(1 <= ns <= DEC_MAX_SPLITS, f"decode: num_splits must be 1..{DEC_MAX_SPLITS}, got {ns}")
    ws_bytes = _lib.load().sl8_attn_int8_decode_workspace(B, H, D, ns)
    ws = torch.empty((ws_bytes,), device=q.device, dtype=torch.uint8)
    fn = "sl8_attn_int8_decode_ks16" if k_scale.dtype == torch.float16 else "sl8_attn_int8_decode"
    with torch.cuda.device(q.device):
        call(fn, q.data_ptr(), q_scale.data_ptr(), k.data_ptr(),
             k_scale.data_ptr(), v.data_ptr(), out.data_ptr(), B, H, Hkv, N, D, ns,
             ws.data_ptr(), ws_bytes, stream_of(q))
    return out


def attn_int8_decode_kv8(q, q_scale, k, k_scale, v, v_scale, num_splits=-1):
    """Decode over an int8 K/V cache (reference csrc/kernel/attn_decode.cu:245-320):
    q int8 [B,Hq,1,D], q_scale fp32 [B,Hq,1], k int8 [B,Hkv,N,D], k_scale fp32 [B,Hkv,N],
    v int8 [B,Hkv,N,D], v_scale fp32 [B,Hkv,D] (per channel) -> fp16 [B,Hq,1,D]."""
    _on_gpu(q, q_scale, k, k_scale, v, v_scale)
    _check(q.dtype == torch.int8 and k.dtype == torch.int8 and v.dtype == torch.int8,
           "decode_kv8: q/k/v must be int8")
    _check(q_scale.dtype == torch.float32 and k_scale.dtype == torch.float32 and
           v_scale.dtype == torch.float32, "decode_kv8: scales must be float32")
    _check(q.dim() == 4 and k.dim() == 4 and v.dim() == 4, "decode_kv8: expect [B,H,S,D]")
    _check(q.shape[2] == 1, "decode_kv8: query length M must be 1 (decode)")
    _contig(q, q_scale, k, k_scale, v, v_scale)
    B, H, _, D = q.shape
    Hkv, N = k.shape[1], k.shape[2]
    _check(k.shape[0] == B and v.shape[0] == B and v.shape[1] == Hkv,
           "decode_kv8: batch/head mismatch")
    _check(Hkv > 0 and H % Hkv == 0, "decode_kv8: H_q must be divisible by H_kv (GQA)")
    _check(k.shape[3] == D and v.shape[3] == D and v.shape[2] == N, "decode_kv8: K/V shape mismatch")
    _check(q_scale.numel() == B * H and k_scale.numel() == B * Hkv * N and
           v_scale.numel() == B * Hkv * D, "decode_kv8: scale shape mismatch")
    _check(D in _HEAD_DIMS_DECODE, f"decode_kv8: head dim must be {_dims_msg(_HEAD_DIMS_DECODE)}, got {D}")
    num_splits = int(num_splits)
    _check(num_splits != 0,
           f"decode_kv8: num_splits=0 is invalid; use -1 for auto or 1..{DEC_MAX_SPLITS}")
    out = torch.empty((B, H, 1, D), device=q.device, dtype=torch.float16)
    if B == 0 or H == 0:
        return out
    if N == 0:
        return out.zero_()
    ns = choose_n_splits(N, B, Hkv) if num_splits < 0 else num_splits
    _check(1 <= ns <= DEC_MAX_SPLITS, f"decode_kv8: num_splits must be 1..{DEC_MAX_SPLITS}, got {ns}")
    ws_bytes = _lib.load().sl8_attn_int8_decode_workspace(B, H, D, ns)
    ws = torch.empty((ws_bytes,), device=q.device, dtype=torch.uint8)
    with torch.cuda.device(q.device):
        call("sl8_attn_int8_decode_kv8", q.data_ptr(), q_scale.data_ptr(), k.data_ptr(),
             k_scale.data_ptr(), v.data_ptr(), v_scale.data_ptr(), out.data_ptr(), B, H, Hkv, N,
             D, ns, ws.data_ptr(), ws_bytes, stream_of(q))
    return out


def paged_choose_n_splits(n_len_max, bhq):
    """Auto split count of the paged decode (reference attn_paged_decode.cu:14-31)."""
    return int(_lib.load().sl8_paged_choose_num_splits(int(n_len_max), int(bhq)))


def attn_paged_decode(q, q_scale, k_cache, k_scale, v_cache, v_scale, block_table, context_lens,
                      block_size, max_context_len, num_splits=-1):
    """Paged-KV decode (reference csrc/kernel/attn_paged_decode.cu:107-240): q int8
    [B,Hq,1,D], q_scale fp32 [B,Hq,1], k_cache/v_cache int8 [num_blocks,Hkv,bs,D],
    k_scale/v_scale fp32 [num_blocks,Hkv,bs], block_table int32 [B,max_blocks],
    context_lens int32 [B] -> fp16 [B,Hq,1,D]."""
    _on_gpu(q, q_scale, k_cache, k_scale, v_cache, v_scale, block_table, context_lens)
    _check(q.dtype == torch.int8 and k_cache.dtype == torch.int8 and v_cache.dtype == torch.int8,
           "paged_decode: q/k_cache/v_cache must be int8")
    _check(q_scale.dtype == torch.float32 and k_scale.dtype == torch.float32 and
           v_scale.dtype == torch.float32, "paged_decode: scales must be float32")
    _check(block_table.dtype == torch.int32 and context_lens.dtype == torch.int32,
           "paged_decode: block_table/context_lens must be int32")
    _check(q.dim() == 4 and q.shape[2] == 1, "paged_decode: q must be [B,H_q,1,D]")
    _check(k_cache.dim() == 4 and v_cache.dim() == 4,
           "paged_decode: k_cache/v_cache must be [num_blocks,H_kv,block_size,D]")
    _contig(q, q_scale, k_cache, k_scale, v_cache, v_scale, block_table, context_lens)
    B, H, _, D = q.shape
    nblk, Hkv, bs = k_cache.shape[0], k_cache.shape[1], k_cache.shape[2]
    _check(bs == block_size, "paged_decode: block_size mismatch vs k_cache.size(2)")
    _check(k_cache.shape[3] == D and v_cache.shape == k_cache.shape,
           "paged_decode: k_cache/v_cache shape mismatch")
    _check(Hkv > 0 and H % Hkv == 0, "paged_decode: H_q must be divisible by H_kv (GQA)")
    _check(k_cache.numel() == k_scale.numel() * D and v_cache.numel() == v_scale.numel() * D,
           "paged_decode: scale shape mismatch vs cache")
    _check(q_scale.numel() == B * H, "paged_decode: q_scale shape mismatch")
    _check(block_table.dim() == 2 and block_table.shape[0] == B,
           "paged_decode: block_table must be [B, max_blocks_per_seq]")
    _check(context_lens.dim() == 1 and context_lens.shape[0] == B,
           "paged_decode: context_lens must be [B]")
    _check(D in _HEAD_DIMS_DECODE, f"paged_decode: head dim must be {_dims_msg(_HEAD_DIMS_DECODE)}, got {D}")
    maxb = block_table.shape[1]
    _check(0 <= max_context_len <= maxb * bs,
           "paged_decode: max_context_len exceeds block_table capacity")
    num_splits = int(num_splits)
    _check(num_splits != 0,
           f"paged_decode: num_splits=0 is invalid; use -1 for auto or 1..{DEC_MAX_SPLITS}")
    out = torch.empty((B, H, 1, D), device=q.device, dtype=torch.float16)
    if B == 0 or H == 0:
        return out
    ns = paged_choose_n_splits(max_context_len, B * H) if num_splits < 0 else num_splits
    _check(1 <= ns <= DEC_MAX_SPLITS, f"paged_decode: num_splits must be 1..{DEC_MAX_SPLITS}, got {ns}")
    ws_bytes = _lib.load().sl8_attn_int8_decode_workspace(B, H, D, ns)
    ws = torch.empty((ws_bytes,), device=q.device, dtype=torch.uint8)
    with torch.cuda.device(q.device):
        call("sl8_attn_paged_decode", q.data_ptr(), q_scale.data_ptr(), k_cache.data_ptr(),
             k_scale.data_ptr(), v_cache.data_ptr(), v_scale.data_ptr(), block_table.data_ptr(),
             context_lens.data_ptr(), out.data_ptr(), B, H, Hkv, D, nblk, bs, maxb,
             int(max_context_len), ns, ws.data_ptr(), ws_bytes, stream_of(q))
    return out


def attn_paged_decode_k8v3(q, q_scale, k_cache, k_scale, v_packed, v_norm, v_codebook,
                           block_table, context_lens, block_size, max_context_len,
                           num_splits=-1):
    """Paged decode over a K8V3 store (reference csrc/kernel/attn_paged_decode.cu:229-330):
    K as attn_paged_decode; V as 3-bit Lloyd-Max codes v_packed int32
    [num_blocks,Hkv,bs,3D/32], per-128-channel norms v_norm fp32 [num_blocks,Hkv,bs,D/128]
    and a codebook fp32 [8]; D 128 or 256 -> fp16 [B,Hq,1,D]."""
    tag = "paged_decode_k8v3"
    _on_gpu(q, q_scale, k_cache, k_scale, v_packed, v_norm, v_codebook, block_table,
            context_lens)
    _check(q.dtype == torch.int8 and k_cache.dtype == torch.int8, f"{tag}: q/k_cache must be int8")
    _check(v_packed.dtype == torch.int32, f"{tag}: v_packed must be int32")
    _check(q_scale.dtype == torch.float32 and k_scale.dtype == torch.float32 and
           v_norm.dtype == torch.float32 and v_codebook.dtype == torch.float32,
           f"{tag}: scales/norms/codebook must be float32")
    _check(block_table.dtype == torch.int32 and context_lens.dtype == torch.int32,
           f"{tag}: block_table/context_lens must be int32")
    _check(q.dim() == 4 and q.shape[2] == 1, f"{tag}: q must be [B,H_q,1,D]")
    _check(k_cache.dim() == 4 and v_packed.dim() == 4 and v_norm.dim() == 4,
           f"{tag}: caches must be [num_blocks,H_kv,block_size,...]")
    _contig(q, q_scale, k_cache, k_scale, v_packed, v_norm, v_codebook, block_table, context_lens)
    B, H, _, D = q.shape
    nblk, Hkv, bs = k_cache.shape[0], k_cache.shape[1], k_cache.shape[2]
    _check(bs == block_size, f"{tag}: block_size mismatch vs k_cache.size(2)")
    _check(k_cache.shape[3] == D and tuple(v_packed.shape[:3]) == (nblk, Hkv, bs) and
           tuple(v_norm.shape[:3]) == (nblk, Hkv, bs),
           f"{tag}: k_cache/v_packed/v_norm shape mismatch")
    _check(Hkv > 0 and H % Hkv == 0, f"{tag}: H_q must be divisible by H_kv (GQA)")
    _check(D in (128, 256), f"{tag}: lloydmax3 requires head dim 128 or 256, got {D}")
    _check(k_cache.numel() == k_scale.numel() * D, f"{tag}: k_scale shape mismatch vs k_cache")
    _check(v_packed.shape[3] == D * 3 // 32,
           f"{tag}: v_packed last dim must be D*3/32, got {v_packed.shape[3]}")
    _check(v_norm.shape[3] == D // 128, f"{tag}: v_norm last dim must be D/128, got {v_norm.shape[3]}")
    _check(v_codebook.dim() == 1 and v_codebook.numel() == 8, f"{tag}: v_codebook must be [8] fp32")
    _check(q_scale.numel() == B * H, f"{tag}: q_scale shape mismatch")
    _check(block_table.dim() == 2 and block_table.shape[0] == B,
           f"{tag}: block_table must be [B, max_blocks_per_seq]")
    _check(context_lens.dim() == 1 and context_lens.shape[0] == B, f"{tag}: context_lens must be [B]")
    maxb = block_table.shape[1]
    _check(0 <= max_context_len <= maxb * bs, f"{tag}: max_context_len exceeds block_table capacity")
    num_splits = int(num_splits)
    _check(num_splits != 0,
           f"{tag}: num_splits=0 is invalid; use -1 for auto or 1..{DEC_MAX_SPLITS}")
    out = torch.empty((B, H, 1, D), device=q.device, dtype=torch.float16)
    if B == 0 or H == 0:
        return out
    ns = paged_choose_n_splits(max_context_len, B * H) if num_splits < 0 else num_splits
    _check(1 <= ns <= DEC_MAX_SPLITS, f"{tag}: num_splits must be 1..{DEC_MAX_SPLITS}, got {ns}")
    ws_bytes = _lib.load().sl8_attn_int8_decode_workspace(B, H, D, ns)
    ws = torch.empty((ws_bytes,), device=q.device, dtype=torch.uint8)
    with torch.cuda.device(q.device):
        call("sl8_attn_paged_decode_k8v3", q.data_ptr(), q_scale.data_ptr(), k_cache.data_ptr(),
             k_scale.data_ptr(), v_packed.data_ptr(), v_norm.data_ptr(), v_codebook.data_ptr(),
             block_table.data_ptr(), context_lens.data_ptr(), out.data_ptr(), B, H, Hkv, D, nblk,
             bs, maxb, int(max_context_len), ns, ws.data_ptr(), ws_bytes, stream_of(q))
    return out


def kv_write_paged(k_new, v_new, slot_mapping, k_cache, k_scale, v_cache, v_scale):
    """Quantize-on-write of one new token per (batch, KV head) into the paged int8
    cache, in place (reference csrc/kernel/attn_paged_decode.cu:360-421)."""
    _on_gpu(k_new, v_new, slot_mapping, k_cache, k_scale, v_cache, v_scale)
    _check(k_new.dtype == torch.float16 and v_new.dtype == torch.float16,
           "kv_write_paged: k_new/v_new must be float16")
    _check(slot_mapping.dtype == torch.int32, "kv_write_paged: slot_mapping must be int32")
    _check(k_cache.dtype == torch.int8 and v_cache.dtype == torch.int8,
           "kv_write_paged: k_cache/v_cache must be int8")
    _check(k_new.dim() == 3 and v_new.dim() == 3, "kv_write_paged: k_new/v_new must be [B,H_kv,D]")
    _contig(k_new, v_new, slot_mapping, k_cache, v_cache)
    B, Hkv, D = k_new.shape
    _check(tuple(v_new.shape) == (B, Hkv, D), "kv_write_paged: k_new/v_new shape mismatch")
    _check(slot_mapping.dim() == 1 and slot_mapping.shape[0] == B,
           "kv_write_paged: slot_mapping must be [B]")
    _check(k_cache.dim() == 4 and k_cache.shape[1] == Hkv and k_cache.shape[3] == D,
           "kv_write_paged: k_cache must be [num_blocks,H_kv,block_size,D]")
    _check(v_cache.shape == k_cache.shape, "kv_write_paged: v_cache shape must match k_cache")
    _check(k_scale.is_contiguous() and v_scale.is_contiguous(),
           "kv_write_paged: k_scale/v_scale must be contiguous")
    _check(k_scale.dtype == torch.float32 and v_scale.dtype == torch.float32,
           "kv_write_paged: k_scale/v_scale must be float32")
    _check(k_scale.numel() == k_cache.numel() // D and v_scale.numel() == v_cache.numel() // D,
           "kv_write_paged: scale shape mismatch vs cache")
    _check(D in _HEAD_DIMS_DECODE, f"kv_write_paged: head dim must be {_dims_msg(_HEAD_DIMS_DECODE)}, got {D}")
    if B == 0:
        return
    with torch.cuda.device(k_new.device):
        call("sl8_kv_write_paged", k_new.data_ptr(), v_new.data_ptr(), slot_mapping.data_ptr(),
             k_cache.data_ptr(), k_scale.data_ptr(), v_cache.data_ptr(), v_scale.data_ptr(),
             B, Hkv, D, k_cache.shape[0], k_cache.shape[2], stream_of(k_new))


# ---------------------------------------------------------------------------
# Q4_K (reference csrc/kernel/gemm_dp4a.cu:146-193, gemm_decode_dp4a.cu:375-436)
# ---------------------------------------------------------------------------
def _q4k_checks(x, x_scale, w, out_dtype, tag, type_size=Q4K_TYPE_SIZE, x_block_ok=False):
    _on_gpu(x, x_scale, w)
    _check(x.dtype == torch.int8, "x must be int8")
    _check(w.dtype == torch.uint8, f"w must be uint8 (native {tag} bytes)")
    _check(x_scale.dtype == torch.float32, "x_scale must be float32")
    _check(x.dim() == 2 and w.dim() == 2, f"expect x[M,K] and w[N,(K/256)*{type_size}]")
    _contig(x, x_scale, w)
    _check(out_dtype in (torch.float16, torch.bfloat16, torch.float32),
           f"out_dtype must be float16 or bfloat16, got {out_dtype}")
    M, K = x.shape
    N = w.shape[0]
    _check(K % 256 == 0, f"{tag} contraction dim K must be %256==0, got {K}")
    _check(w.shape[1] == (K // 256) * type_size,
           f"{tag} weight must be [N, (K/256)*{type_size}], got [{N},{w.shape[1]}] for K={K}")
    if x_block_ok:
        _check(x_scale.numel() == M or tuple(x_scale.shape) == (M, K // 256),
               f"x_scale must be [M] (per row) or [M, K/256] (per 256-block), got "
               f"{list(x_scale.shape)} for M={M}, K={K}")
    else:
        _check(x_scale.numel() == M, f"x_scale must be [M] (per row), got {list(x_scale.shape)}")
    return M, N, K


def _q4k(sym, x, x_scale, w, out_dtype, tag="Q4_K", type_size=Q4K_TYPE_SIZE):
    M, N, K = _q4k_checks(x, x_scale, w, out_dtype, tag, type_size)
    out = torch.empty((M, N), device=x.device, dtype=out_dtype)
    if M and N:
        with torch.cuda.device(x.device):
            call(sym, x.data_ptr(), x_scale.data_ptr(), w.data_ptr(), out.data_ptr(),
                 dtype_code(out_dtype), M, N, K, stream_of(x))
    return out


def gemm_q4k(x, x_scale, w, out_dtype=torch.float16):
    """x int8 [M,K], x_scale fp32 [M], w uint8 [N,(K/256)*144] -> [M,N] out_dtype."""
    return _q4k("sl8_gemm_q4k", x, x_scale, w, out_dtype)


def gemm_decode_q4k(x, x_scale, w, out_dtype=torch.float16):
    """Decode-shape (M <= 16) Q4_K GEMV; same math as gemm_q4k.

    x_scale [M] is the reference's per-row activation scale; x_scale [M, K/256]
    (one scale per 256-element block, from quantize_i8_blockwise) scales each
    super-block's integer sums instead (BASELINE config 4's activation format)."""
    _check(x.dim() == 2 and x.shape[0] <= DEC_MAX_M,
           f"gemm_decode_q4k supports M<={DEC_MAX_M}, got M={x.shape[0] if x.dim() else 0}"
           " -- use the tile gemm_q4k for prefill")
    M, N, K = _q4k_checks(x, x_scale, w, out_dtype, "Q4_K", Q4K_TYPE_SIZE, x_block_ok=True)
    # per-256-block scales only when the shape says so; any other x_scale with
    # M elements (e.g. [M, 1]) is the reference's per-row scale
    if x_scale.dim() == 2 and tuple(x_scale.shape) == (M, K // 256) and K // 256 > 1:
        out = torch.empty((M, N), device=x.device, dtype=out_dtype)
        if M and N:
            with torch.cuda.device(x.device):
                call("sl8_gemm_decode_q4k_xblock", x.data_ptr(), x_scale.data_ptr(), w.data_ptr(),
                     out.data_ptr(), dtype_code(out_dtype), M, N, K, stream_of(x))
        return out
    return _q4k("sl8_gemm_decode_q4k", x, x_scale.reshape(-1), w, out_dtype)


def quantize_i8_blockwise(x: torch.Tensor, block: int = 256):
    """x [M, K] -> (int8 [M, K], fp32 scale [M, K/block]): the row-wise quantiser
    applied to every `block`-element slice of each row."""
    _check(x.dim() == 2 and block > 0 and x.shape[1] % block == 0,
           f"quantize_i8_blockwise expects x[M,K] with K % {block} == 0")
    M, K = x.shape
    q, s = quantize_i8_rowwise(x.contiguous().reshape(M * (K // block), block))
    return q.reshape(M, K), s.reshape(M, K // block)


def gemm_q5k(x, x_scale, w, out_dtype=torch.float16):
    """x int8 [M,K], x_scale fp32 [M], w uint8 [N,(K/256)*176] (native Q5_K) -> [M,N]."""
    return _q4k("sl8_gemm_q5k", x, x_scale, w, out_dtype, "Q5_K", Q5K_TYPE_SIZE)


def gemm_q6k(x, x_scale, w, out_dtype=torch.float16):
    """x int8 [M,K], x_scale fp32 [M], w uint8 [N,(K/256)*210] (native Q6_K) -> [M,N]."""
    return _q4k("sl8_gemm_q6k", x, x_scale, w, out_dtype, "Q6_K", Q6K_TYPE_SIZE)


def gemm_decode_q5k(x, x_scale, w, out_dtype=torch.float16):
    """Decode-shape (M <= 16) Q5_K GEMV; same math as gemm_q5k."""
    _check(x.dim() == 2 and x.shape[0] <= DEC_MAX_M,
           f"gemm_decode_q5k supports M<={DEC_MAX_M}, got M={x.shape[0] if x.dim() else 0}"
           " -- use the tile gemm_q5k for prefill")
    return _q4k("sl8_gemm_decode_q5k", x, x_scale, w, out_dtype, "Q5_K", Q5K_TYPE_SIZE)


def gemm_decode_q6k(x, x_scale, w, out_dtype=torch.float16):
    """Decode-shape (M <= 16) Q6_K GEMV; same math as gemm_q6k."""
    _check(x.dim() == 2 and x.shape[0] <= DEC_MAX_M,
           f"gemm_decode_q6k supports M<={DEC_MAX_M}, got M={x.shape[0] if x.dim() else 0}"
           " -- use the tile gemm_q6k for prefill")
    return _q4k("sl8_gemm_decode_q6k", x, x_scale, w, out_dtype, "Q6_K", Q6K_TYPE_SIZE)


def _dequant_kq(sym, w, K, tag, type_size):
    _on_gpu(w)
    _check(w.dtype == torch.uint8 and w.dim() == 2, f"w must be uint8 [N,(K/256)*{type_size}]")
    _check(K % 256 == 0 and w.shape[1] == (K // 256) * type_size, f"{tag} weight/K mismatch")
    w = w.contiguous()
    out = torch.empty((w.shape[0], K), device=w.device, dtype=torch.float32)
    if out.numel():
        with torch.cuda.device(w.device):
            call(sym, w.data_ptr(), out.data_ptr(), w.shape[0], K, stream_of(w))
    return out


def dequant_q5k(w: torch.Tensor, K: int) -> torch.Tensor:
    """Native Q5_K bytes [N,(K/256)*176] -> fp32 [N,K] (d*sc*q - dmin*m, fp32)."""
    return _dequant_kq("sl8_dequant_q5k", w, K, "Q5_K", Q5K_TYPE_SIZE)


def dequant_q6k(w: torch.Tensor, K: int) -> torch.Tensor:
    """Native Q6_K bytes [N,(K/256)*210] -> fp32 [N,K] ((d*sc)*(q-32), fp32)."""
    return _dequant_kq("sl8_dequant_q6k", w, K, "Q6_K", Q6K_TYPE_SIZE)


def dequant_q4k(w: torch.Tensor, K: int) -> torch.Tensor:
    """Native Q4_K bytes [N,(K/256)*144] -> fp32 [N,K] (exact)."""
    _on_gpu(w)
    _check(w.dtype == torch.uint8 and w.dim() == 2, "w must be uint8 [N,(K/256)*144]")
    _check(K % 256 == 0 and w.shape[1] == (K // 256) * Q4K_TYPE_SIZE, "Q4_K weight/K mismatch")
    w = w.contiguous()
    out = torch.empty((w.shape[0], K), device=w.device, dtype=torch.float32)
    if out.numel():
        with torch.cuda.device(w.device):
            call("sl8_dequant_q4k", w.data_ptr(), out.data_ptr(), w.shape[0], K, stream_of(w))
    return out

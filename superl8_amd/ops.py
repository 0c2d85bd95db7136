"""Public operators of the hot path, drop-in for superl8/ops.py of the reference.

Same names, keyword arguments, routing and error behaviour as the reference
wrappers (reference superl8/ops.py:70-175 attn_int8_fwd, :230-267
attn_int8_decode, :531-584 quantize_kv_cache, :671-727 attn_decode_cached,
:730-849 quantize_kv_write_paged / attn_paged_decode_cached,
:975-991 quantize_i8_rowwise, :1254-1347 linear_q4k / linear_q5k / linear_q6k / _linear_kquant),
dispatching to the gfx950 kernels through `_C`.
"""
from __future__ import annotations

import math

import torch

from . import _C

# Decode-shape M cap for the k-quant linear (reference ops.py:1289).
_KQUANT_DECODE_MAX_M = 16


def attn_int8_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool = False,
                  scale: float | None = None, int8_pv: bool = False, rotate: bool = False,
                  window_left: int = -1, per_warp_quant: bool = True,
                  internal_accuracy_gate: bool = True) -> torch.Tensor:
    """INT8-QK^T FlashAttention-2 prefill (MFMA), fp16/bf16 PV; ``int8_pv`` = full W8A8.

    q, k, v: fp16/bf16 [B, H, S, D]. Q/K are quantised per row (K smoothed) in
    the prologue; causal attention is bottom-right aligned; ``window_left>=0``
    adds a left window (fp16-PV path only). With ``internal_accuracy_gate``,
    a Q row whose max/median magnitude ratio exceeds 12 sends the whole call
    to full-precision attention (reference ops.py:115-147).
    """
    from . import quant

    if internal_accuracy_gate:
        fired, qk = quant.quantize_qk_gated(q, k, softmax_scale=scale, rotate=rotate,
                                            defer=not int8_pv)
    else:
        fired, qk = False, quant.quantize_qk(q, k, softmax_scale=scale, rotate=rotate)
    if isinstance(fired, torch.Tensor):
        # gate decided on the device: its flag is copied to pinned host memory
        # right after the prologue, the attention is launched behind the copy
        # (it exits at once if the gate fired), and the host waits only for the
        # copy -- not for the attention, so the next call's prologue is queued
        # while this attention runs (a plain .item() after the launch would
        # wait for the attention and leave the GPU idle during the next enqueue)
        q_i8, q_scale, k_i8, k_scale, _k_mean = qk
        flag_host = torch.empty(1, dtype=torch.int32, pin_memory=True)
        flag_host.copy_(fired, non_blocking=True)
        flag_ready = torch.cuda.Event()
        flag_ready.record(torch.cuda.current_stream(q.device))
        out = _C.attn_int8_fwd(q_i8, q_scale.squeeze(-1).contiguous(), k_i8,
                               k_scale.squeeze(-1).contiguous(), v.contiguous(), causal,
                               window_left, gate_flag=fired)
        flag_ready.synchronize()
        if int(flag_host[0]) == 0:
            return out
        fired = True
    if fired:
        import torch.nn.functional as F

        s = (1.0 / math.sqrt(q.shape[-1])) if scale is None else scale
        attn_mask = None
        if causal and q.shape[-2] != k.shape[-2]:
            m, n = q.shape[-2], k.shape[-2]
            attn_mask = torch.ones(m, n, device=q.device, dtype=torch.bool).tril(n - m)
        if window_left >= 0:
            m, n = q.shape[-2], k.shape[-2]
            i = torch.arange(m, device=q.device)[:, None] + (n - m)
            j = torch.arange(n, device=q.device)[None, :]
            attn_mask = (j <= i) & (j > i - window_left)
        return F.scaled_dot_product_attention(
            q, k, v.to(q.dtype) if v.dtype != q.dtype else v, attn_mask=attn_mask,
            is_causal=causal and attn_mask is None, scale=s,
            enable_gqa=q.shape[1] != k.shape[1]).to(v.dtype)

    q_i8, q_scale, k_i8, k_scale, _k_mean = qk
    q_scale = q_scale.squeeze(-1).contiguous()
    k_scale = k_scale.squeeze(-1).contiguous()
    if int8_pv:
        if window_left >= 0:
            raise ValueError("window_left is only supported on the fp16-PV path (int8_pv=False)")
        v_i8, v_scale = quant.quantize_v_perchannel(v)
        return _C.attn_w8a8_fwd(q_i8, q_scale, k_i8, k_scale, v_i8,
                                v_scale.squeeze(-2).contiguous(), causal,
                                causal_diag=k.shape[-2] - q.shape[-2] if causal else 0,
                                per_warp_quant=per_warp_quant)
    return _C.attn_int8_fwd(q_i8, q_scale, k_i8, k_scale, v.contiguous(), causal, window_left)


def attn_int8_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                     scale: float | None = None, rotate: bool = False,
                     num_splits: int | None = None) -> torch.Tensor:
    """Split-KV decode: q fp16 [B, Hq, 1, D] against k, v fp16 [B, Hkv, N, D]."""
    from .quant import quantize_qk

    if q.shape[-2] != 1:
        raise AssertionError(f"decode expects M=1, got M={q.shape[-2]}")
    q_i8, q_scale, k_i8, k_scale, _k_mean = quantize_qk(q, k, softmax_scale=scale, rotate=rotate)
    q_scale = q_scale.reshape(q.shape[0], q.shape[1], 1).contiguous()
    k_scale = k_scale.squeeze(-1).contiguous()
    ns = -1 if num_splits is None else int(num_splits)
    return _C.attn_int8_decode(q_i8, q_scale, k_i8, k_scale, v.contiguous(), ns)


def quantize_kv_cache(k: torch.Tensor, v: torch.Tensor, *, rotate: bool = False,
                      v_quant: str = "per_channel"):
    """Quantise a K/V cache once for persistent int8 storage (reference ops.py:531-584):
    K smoothed (+ optional Hadamard rotation) then per-row int8; V per-channel int8
    (v_scale [B,Hkv,D]) or, with v_quant="per_token", per-key int8 (v_scale [B,Hkv,N]).
    Returns (k_i8, k_scale [B,Hkv,N], v_i8, v_scale)."""
    from .quant import quantize_int8_rowwise, quantize_v_perchannel, quantize_v_rowwise, smooth_k

    if v_quant not in ("per_channel", "per_token"):
        raise ValueError(f"v_quant must be 'per_channel' or 'per_token', got {v_quant!r}")
    k_s, _k_mean = smooth_k(k)
    if rotate:
        from .quant.rotation import rotate_last

        k_s = rotate_last(k_s)
    k_i8, k_scale = quantize_int8_rowwise(k_s)
    if v_quant == "per_channel":
        v_i8, v_scale = quantize_v_perchannel(v)
        v_scale = v_scale.squeeze(-2)
    else:
        v_i8, v_scale = quantize_v_rowwise(v)
        v_scale = v_scale.squeeze(-1)
    return k_i8.contiguous(), k_scale.squeeze(-1).contiguous(), v_i8.contiguous(), v_scale.contiguous()


def attn_decode_cached(q: torch.Tensor, k_i8: torch.Tensor, k_scale: torch.Tensor,
                       v_i8: torch.Tensor, v_scale: torch.Tensor, *, scale: float | None = None,
                       rotate: bool = False, num_splits: int | None = None) -> torch.Tensor:
    """Decode (M=1) against a pre-quantised int8 K/V cache from quantize_kv_cache
    (reference ops.py:671-727): only q is quantised per call. q fp16 [B,Hq,1,D] ->
    fp16 [B,Hq,1,D]; `rotate` must match the flag the cache was built with."""
    from .quant import LOG2E
    from .quant.rotation import rotate_last

    if q.shape[-2] != 1:
        raise AssertionError(f"decode expects M=1, got M={q.shape[-2]}")
    if v_scale.shape[-1] == k_i8.shape[2]:
        raise RuntimeError(
            "attn_decode_cached received a per-token V scale [B,H,N]; the contiguous int8-V "
            "decode kernel (attn_int8_decode_kv8) supports per-channel V scales [B,H,D] only")
    softmax_scale = (1.0 / (q.shape[-1] ** 0.5)) if scale is None else scale
    if rotate:
        q = rotate_last(q)
    q_shape = q.shape
    q_i8, q_scale = quantize_i8_rowwise(q.reshape(-1, q_shape[-1]).contiguous())
    q_i8 = q_i8.reshape(q_shape)
    q_scale = (q_scale.float() * (softmax_scale * LOG2E)).reshape(q_shape[0], q_shape[1], 1).contiguous()
    ns = -1 if num_splits is None else int(num_splits)
    return _C.attn_int8_decode_kv8(q_i8.contiguous(), q_scale, k_i8.contiguous(),
                                   k_scale.contiguous(), v_i8.contiguous(), v_scale.contiguous(), ns)


def quantize_kv_write_paged(k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
                            k_scale: torch.Tensor, v_cache: torch.Tensor, v_scale: torch.Tensor,
                            slot_mapping: torch.Tensor, *, rotate: bool = True) -> None:
    """Quantise-on-write of one new token per sequence into the paged int8 KV pool,
    in place (reference ops.py:730-775): per-token scales for K and V; `rotate`
    applies the Hadamard rotation to K (the smoothing usable one token at a time)."""
    from .quant.rotation import rotate_last

    if rotate:
        k_new = rotate_last(k_new)
    _C.kv_write_paged(k_new.contiguous(), v_new.contiguous(), slot_mapping.contiguous(),
                      k_cache, k_scale, v_cache, v_scale)


def attn_paged_decode_cached(q: torch.Tensor, k_cache: torch.Tensor, k_scale: torch.Tensor,
                             v_cache: torch.Tensor, v_scale: torch.Tensor,
                             block_table: torch.Tensor, context_lens: torch.Tensor,
                             block_size: int, *, max_context_len: int | None = None,
                             scale: float | None = None, rotate: bool = True,
                             num_splits: int | None = None) -> torch.Tensor:
    """Decode (M=1) against a paged int8 KV cache (reference ops.py:778-849): one
    launch for a batch of mixed-length sequences. `rotate` must match the flag the
    cache was written with; max_context_len defaults to max(context_lens) (a host sync)."""
    from .quant import LOG2E
    from .quant.rotation import rotate_last

    if q.shape[-2] != 1:
        raise AssertionError(f"paged decode expects M=1, got M={q.shape[-2]}")
    if max_context_len is None:
        max_context_len = int(context_lens.max().item())
    softmax_scale = (1.0 / (q.shape[-1] ** 0.5)) if scale is None else scale
    if rotate:
        q = rotate_last(q)
    q_shape = q.shape
    q_i8, q_scale = quantize_i8_rowwise(q.reshape(-1, q_shape[-1]).contiguous())
    q_i8 = q_i8.reshape(q_shape)
    q_scale = (q_scale.float() * (softmax_scale * LOG2E)).reshape(q_shape[0], q_shape[1], 1).contiguous()
    ns = -1 if num_splits is None else int(num_splits)
    return _C.attn_paged_decode(q_i8.contiguous(), q_scale, k_cache.contiguous(),
                                k_scale.contiguous(), v_cache.contiguous(), v_scale.contiguous(),
                                block_table.contiguous(), context_lens.contiguous(),
                                int(block_size), int(max_context_len), ns)


def attn_paged_decode_k8v3(q: torch.Tensor, k_cache: torch.Tensor, k_scale: torch.Tensor,
                           v_packed: torch.Tensor, v_norm: torch.Tensor, v_codebook: torch.Tensor,
                           block_table: torch.Tensor, context_lens: torch.Tensor,
                           block_size: int, *, max_context_len: int | None = None,
                           scale: float | None = None, rotate: bool = True,
                           num_splits: int | None = None) -> torch.Tensor:
    """Decode (M=1) against a paged K8V3 store (reference ops.py:852-915): int8 K
    (rotated when `rotate`, per-token fp32 scale) and 3-bit Lloyd-Max V (packed
    codes int32 [num_blocks,Hkv,bs,3D/32], norms fp32 [num_blocks,Hkv,bs,D/128],
    codebook fp32 [8]) read inside one paged split-KV launch; D 128 or 256.
    Returns fp16 [B,Hq,1,D]."""
    from .quant import LOG2E
    from .quant.rotation import rotate_last

    if q.shape[-2] != 1:
        raise AssertionError(f"paged decode expects M=1, got M={q.shape[-2]}")
    if max_context_len is None:
        max_context_len = int(context_lens.max().item())
    softmax_scale = (1.0 / (q.shape[-1] ** 0.5)) if scale is None else scale
    if rotate:
        q = rotate_last(q)
    q_shape = q.shape
    q_i8, q_scale = quantize_i8_rowwise(q.reshape(-1, q_shape[-1]).contiguous())
    q_i8 = q_i8.reshape(q_shape)
    q_scale = (q_scale.float() * (softmax_scale * LOG2E)).reshape(q_shape[0], q_shape[1], 1).contiguous()
    ns = -1 if num_splits is None else int(num_splits)
    return _C.attn_paged_decode_k8v3(q_i8.contiguous(), q_scale, k_cache.contiguous(),
                                     k_scale.contiguous(), v_packed.contiguous(),
                                     v_norm.contiguous(), v_codebook.contiguous(),
                                     block_table.contiguous(), context_lens.contiguous(),
                                     int(block_size), int(max_context_len), ns)


def quantize_kv_write_paged_k8v3(k_new: torch.Tensor, v_new: torch.Tensor,
                                 k_cache: torch.Tensor, k_scale: torch.Tensor,
                                 v_packed: torch.Tensor, v_norm: torch.Tensor,
                                 slot_mapping: torch.Tensor, *, rotate: bool = True,
                                 codebook: torch.Tensor | None = None) -> torch.Tensor:
    """Write one new token per (batch, KV head) into a paged K8V3 store, in place:
    K rotated (when `rotate`) and quantised per row to int8; V quantised to 3-bit
    Lloyd-Max codes over 128-channel blocks (`codebook`, default the fixed
    Gaussian one) and packed. k_new, v_new fp16 [B,Hkv,D]; slot_mapping int32 [B]
    (flat slot = block * block_size + offset). Returns the codebook used, the
    `v_codebook` argument of attn_paged_decode_k8v3. (The reference store is
    written the same way by its serving code, reference
    tests/test_k8v3_paged_decode.py:32-83.)"""
    from .quant.lloydmax import pack_indices_lowbit, quantize_lloydmax
    from .quant.rotation import rotate_last

    B, Hkv, D = k_new.shape
    bs = k_cache.shape[2]
    if rotate:
        k_new = rotate_last(k_new)
    k_i8, k_sc = quantize_i8_rowwise(k_new.reshape(-1, D).contiguous())
    codes, norms, cb = quantize_lloydmax(v_new, bits=3, block_size=128, codebook=codebook)
    packed = pack_indices_lowbit(codes, 3)
    slots = slot_mapping.long()
    rows = ((slots // bs)[:, None] * Hkv + torch.arange(Hkv, device=slots.device)) * bs + \
        (slots % bs)[:, None]
    rows = rows.reshape(-1)
    k_cache.view(-1, D)[rows] = k_i8
    k_scale.view(-1)[rows] = k_sc
    v_packed.view(-1, v_packed.shape[-1])[rows] = packed.reshape(-1, packed.shape[-1])
    v_norm.view(-1, v_norm.shape[-1])[rows] = norms.reshape(-1, norms.shape[-1])
    return cb


def quantize_kv_cache_3bit(k: torch.Tensor, v: torch.Tensor, *, rotate: bool = True,
                           fit: bool = True, block_size: int = 128) -> dict:
    """3-bit Lloyd-Max storage codec of a whole K/V cache (reference ops.py:590-655):
    K smoothed (+ rotated), both packed with a codebook fitted to the
    unit-normalised blocks (`fit`) or the fixed Gaussian one."""
    from .quant import smooth_k
    from .quant.lloydmax import (lloyd_max_fit, lloydmax_bits_levels, pack_indices_lowbit,
                                 quantize_lloydmax)
    from .quant.rotation import rotate_last

    k_s, k_mean = smooth_k(k)
    if rotate:
        k_s = rotate_last(k_s)

    def enc(x):
        cb = None
        if fit:
            xb = x.float().reshape(*x.shape[:-1], x.shape[-1] // block_size, block_size)
            norm = torch.sqrt((xb * xb).sum(-1, keepdim=True))
            cb = lloyd_max_fit(xb / torch.where(norm == 0, torch.ones_like(norm), norm),
                               lloydmax_bits_levels(3))
        codes, norm, codebook = quantize_lloydmax(x, bits=3, block_size=block_size, codebook=cb)
        return pack_indices_lowbit(codes, 3).contiguous(), norm.contiguous(), codebook

    k_packed, k_norm, k_cb = enc(k_s)
    v_packed, v_norm, v_cb = enc(v)
    return {"k_packed": k_packed, "k_norm": k_norm, "k_codebook": k_cb, "v_packed": v_packed,
            "v_norm": v_norm, "v_codebook": v_cb, "k_mean": k_mean, "rotate": rotate,
            "block_size": block_size, "bits": 3}


def dequantize_kv_cache_3bit(packed: dict, d: int):
    """Inverse of quantize_kv_cache_3bit -> (k, v) fp16, K still smoothed and
    rotated (reference ops.py:658-668)."""
    from .quant.lloydmax import dequantize_lloydmax, unpack_indices_lowbit

    bs = packed["block_size"]
    k = dequantize_lloydmax(unpack_indices_lowbit(packed["k_packed"], 3, d), packed["k_norm"],
                            packed["k_codebook"], block_size=bs)
    v = dequantize_lloydmax(unpack_indices_lowbit(packed["v_packed"], 3, d), packed["v_norm"],
                            packed["v_codebook"], block_size=bs)
    return k.half(), v.half()


def quantize_i8_rowwise(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Fused per-row symmetric int8: x[M,K] -> (q int8 [M,K], scale fp32 [M])."""
    return _C.quantize_i8_rowwise(x)


def linear_q4k(x: torch.Tensor, w_bytes: torch.Tensor, *, bias: torch.Tensor | None = None,
               out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """GGUF Q4_K linear on native 144-byte super-blocks: x [..., K] -> [..., N]."""
    return _linear_kquant(x, w_bytes, bias, out_dtype, _C.gemm_q4k,
                          getattr(_C, "gemm_decode_q4k", None))


def linear_q5k(x: torch.Tensor, w_bytes: torch.Tensor, *, bias: torch.Tensor | None = None,
               out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """GGUF Q5_K linear on native 176-byte super-blocks (reference ops.py:1328-1336)."""
    return _linear_kquant(x, w_bytes, bias, out_dtype, _C.gemm_q5k,
                          getattr(_C, "gemm_decode_q5k", None))


def linear_q6k(x: torch.Tensor, w_bytes: torch.Tensor, *, bias: torch.Tensor | None = None,
               out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """GGUF Q6_K linear on native 210-byte super-blocks (reference ops.py:1339-1347)."""
    return _linear_kquant(x, w_bytes, bias, out_dtype, _C.gemm_q6k,
                          getattr(_C, "gemm_decode_q6k", None))


_FUSED_KQUANT_OPS = {"q4_k": linear_q4k, "q5_k": linear_q5k, "q6_k": linear_q6k}


def linear(x: torch.Tensor, qt, *, bias: torch.Tensor | None = None,
           out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """Scheme-dispatched linear over a ``superl8_amd.format.QTensor`` (reference
    ops.py:2088-2150, the ``gguf_kquant`` arm): native Q4_K / Q5_K / Q6_K bytes run
    on the fused kernels; any other scheme or type tag raises ValueError."""
    if qt.scheme == "gguf_kquant":
        op = _FUSED_KQUANT_OPS.get(qt.codebook)
        if op is not None:
            return op(x, qt.data, bias=bias, out_dtype=out_dtype)
        raise ValueError(f"superl8.linear: gguf_kquant type {qt.codebook!r} has no fused kernel")
    raise ValueError(f"superl8.linear: unsupported weight scheme {qt.scheme!r}")


def _linear_kquant(x, w_bytes, bias, out_dtype, tile_op, decode_op):
    *lead, K = x.shape
    x2 = x.reshape(-1, K).contiguous()
    w_bytes = w_bytes.contiguous()
    x_i8, x_scale = quantize_i8_rowwise(x2)
    M = x2.shape[0]
    if decode_op is not None and x2.is_cuda and 0 < M <= _KQUANT_DECODE_MAX_M:
        y = decode_op(x_i8, x_scale, w_bytes, out_dtype)
    else:
        y = tile_op(x_i8, x_scale, w_bytes, out_dtype)
    if bias is not None:
        y = (y.float() + bias.float()).to(y.dtype)
    return y.reshape(*lead, y.shape[-1])

"""INT8 attention: prefill, W8A8 prefill and split-KV decode (numpy restatement).

Reference kernels restated:
  csrc/include/attn_int8_fwd.cuh:72-208  (GQA head map, bottom-right causal,
      window, exp2-domain logits acc*q_scale*k_scale, online softmax, O/l,
      l == 0 -> 0, LSE = m*ln2 + ln l)
  csrc/include/attn_w8a8_fwd.cuh:96-224  (64-key tiles, P re-quantised per row
      or per 32-key half: p_scale = max(pmax*(1/127), 2e-38), int8 PV,
      dequant p_scale * v_scale[d])
  csrc/include/attn_decode.cuh:47-132,430-466 (split s owns keys
      [s*per, min(N,(s+1)*per)), per = ceil(N/ns); partial (O, m, l);
      empty split -> m = -1e30; LSE merge)
  csrc/include/attn_paged_decode.cuh:126-262 (paged cache addressed by a
      per-sequence block table and context length, splits sized on the
      launch's max context length, per-token V scale inside the key sum)
  csrc/kernel/attn_paged_decode.cu:14-31 (its split-count heuristic)
  csrc/include/attn_decode.cuh:141-224 (int8 V cache: O accumulates
      p * v_i8 and each split's partial O is multiplied by the per-channel
      v_scale[d] of its KV head before the merge)

Softmax and PV are evaluated in float64 here (the reference keeps fp32 state);
the kernels are checked against this within stated tolerances, while the
int32 Q.K^T scores are checked bit-exactly.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
from __future__ import annotations

import math

import numpy as np

LN2 = math.log(2.0)
DEC_NEG_INF = -1e30


def kv_head_index(Hq: int, Hkv: int) -> np.ndarray:
    """Query head h reads K/V head h // (Hq/Hkv) (reference attn_int8_fwd.cuh:72)."""
    return np.arange(Hq) // (Hq // Hkv)


def scores_i32(q_i8: np.ndarray, k_i8: np.ndarray) -> np.ndarray:
    """Exact int32 Q.K^T [B,Hq,M,N] (float64 products of int8 are exact)."""
    kk = k_i8[:, kv_head_index(q_i8.shape[1], k_i8.shape[1])]
    s = np.matmul(q_i8.astype(np.float64), np.swapaxes(kk.astype(np.float64), -1, -2))
    return s.astype(np.int64).astype(np.int32)


def logits(acc: np.ndarray, q_scale: np.ndarray, k_scale: np.ndarray, Hq: int) -> np.ndarray:
    """fp32 exp2-domain logits ((float)acc * qs) * ks, as the reference evaluates them."""
    ks = k_scale[:, kv_head_index(Hq, k_scale.shape[1])]
    t = (acc.astype(np.float32) * q_scale[..., :, None].astype(np.float32)).astype(np.float32)
    return (t * ks[..., None, :].astype(np.float32)).astype(np.float32)


SEED_BITS = 0x3E22F983  # the float 1/(2 pi) rounded to fp32


def seeded_logits(acc: np.ndarray, q_scale: np.ndarray, k_scale: np.ndarray,
                  m: np.ndarray | float = 0.0) -> np.ndarray:
    """The D <= 128 prefill kernel's exp2 argument from a seeded accumulator
    (this build's formulation; the reference computes ((float)acc * qs) * ks,
    attn_int8_fwd.cuh:141-150): the int8 MFMA starts from the bits of
    C0 = fp32(1/(2 pi)), so its int32 result read as a float is
    f = C0 + acc * 2^-26 exactly (|acc| <= 2^21); then
        w = fma(f, qs * 2^26, -rn(C0 * qs * 2^26)),   x = fma(w, ks, -m)
    with single fp32 roundings (evaluated here in float64, which holds the
    products exactly, then rounded once to fp32; the sums of a 48-bit product
    and a float are exact in float64 when their exponents are close, which the
    tests' bound allows for). acc int [..], q_scale/k_scale broadcastable fp32."""
    acc = np.asarray(acc, np.int64)
    assert np.all(np.abs(acc) <= 1 << 21), "seeded accumulator range is |acc| <= 2^21"
    f = (acc + SEED_BITS).astype(np.uint32).view(np.float32).astype(np.float64)
    qs26 = (np.asarray(q_scale, np.float32) * np.float32(2.0 ** 26)).astype(np.float32)
    c0 = np.uint32(SEED_BITS).view(np.float32)
    cq = (-(c0 * qs26)).astype(np.float32)
    w = (f * qs26.astype(np.float64) + cq.astype(np.float64)).astype(np.float32)
    x = (w.astype(np.float64) * np.asarray(k_scale, np.float32).astype(np.float64)
         - np.float64(np.float32(m))).astype(np.float32)
    return x


def valid_mask(M: int, N: int, causal: bool, window_left: int = -1,
               causal_diag: int | None = None) -> np.ndarray:
    """[M,N] bool. Query i sits at key position i + (N - M) when causal."""
    diag = (N - M if causal_diag is None else causal_diag) if causal else 0
    i = np.arange(M)[:, None] + diag
    j = np.arange(N)[None, :]
    ok = np.ones((M, N), bool)
    if causal:
        ok &= j <= i
    if window_left >= 0:
        ok &= j > i - window_left
    return ok


def attn_int8_fwd(q_i8, q_scale, k_i8, k_scale, v, causal=False, window_left=-1):
    """Prefill output [B,Hq,M,D] float64 and natural-log LSE [B,Hq,M].

    v: fp32 values of the fp16/bf16 V [B,Hkv,N,D].
    """
    B, Hq, M, D = q_i8.shape
    N = k_i8.shape[2]
    s = logits(scores_i32(q_i8, k_i8), q_scale, k_scale, Hq).astype(np.float64)
    ok = valid_mask(M, N, causal, window_left)
    s = np.where(ok, s, -np.inf)
    m = s.max(axis=-1, keepdims=True) if N else np.full((B, Hq, M, 1), -np.inf)
    live = np.isfinite(m)
    p = np.where(live, np.exp2(s - np.where(live, m, 0.0)), 0.0)
    l = p.sum(-1, keepdims=True)
    vv = v[:, kv_head_index(Hq, v.shape[1])].astype(np.float64)
    o = np.matmul(p, vv)
    out = np.where(l > 0, o / np.where(l > 0, l, 1.0), 0.0)
    with np.errstate(divide="ignore"):
        lse = np.where(l[..., 0] > 0, m[..., 0] * LN2 + np.log(np.where(l[..., 0] > 0, l[..., 0], 1.0)),
                       -np.inf)
    return out, lse


def attn_w8a8_fwd(q_i8, q_scale, k_i8, k_scale, v_i8, v_scale, causal=False, causal_diag=0,
                  per_warp_quant=True, block_n=64):
    """W8A8 prefill with the reference's in-loop P requantisation, float64 state otherwise."""
    B, Hq, M, D = q_i8.shape
    N = k_i8.shape[2]
    kvh = kv_head_index(Hq, k_i8.shape[1])
    s_all = logits(scores_i32(q_i8, k_i8), q_scale, k_scale, Hq)
    ok = valid_mask(M, N, causal, -1, causal_diag if causal else 0)
    s_all = np.where(ok, s_all, np.float32(-np.inf))
    vq = v_i8[:, kvh].astype(np.float64)            # [B,Hq,N,D]
    vs = v_scale[:, kvh].astype(np.float64)         # [B,Hq,D]
    o = np.zeros((B, Hq, M, D))
    m_i = np.full((B, Hq, M), -np.inf)
    l_i = np.zeros((B, Hq, M))
    half = block_n // 2
    for n0 in range(0, N, block_n):
        s = s_all[..., n0:n0 + block_n]
        nb = s.shape[-1]
        tmax = s.max(-1).astype(np.float64)
        m_new = np.maximum(m_i, tmax)
        alive = np.isfinite(m_new)
        with np.errstate(invalid="ignore"):
            p = np.where(np.isfinite(s) & alive[..., None],
                         np.exp2(s.astype(np.float64) - np.where(alive, m_new, 0)[..., None]), 0.0)
        p32 = p.astype(np.float32)
        acc = np.zeros((B, Hq, M, D))
        for h0 in range(0, nb, half if per_warp_quant else block_n):
            h1 = min(nb, h0 + (half if per_warp_quant else block_n))
            pm = p32[..., h0:h1].max(-1)
            ps = np.maximum((pm * np.float32(1.0 / 127.0)).astype(np.float32), np.float32(2e-38))
            inv = (np.float32(1.0) / ps).astype(np.float32)
            pq = np.rint((p32[..., h0:h1] * inv[..., None]).astype(np.float32))
            acc += np.matmul(pq.astype(np.float64), vq[..., n0 + h0:n0 + h1, :]) * ps[..., None]
        with np.errstate(invalid="ignore"):
            resc = np.where(np.isfinite(m_i) & alive, np.exp2(m_i - np.where(alive, m_new, 0)), 1.0)
        o = o * resc[..., None] + np.where(alive[..., None], acc * vs[:, :, None, :], 0.0)
        l_i = l_i * resc + p.sum(-1)
        m_i = np.maximum(m_i, m_new)
    return np.where(l_i[..., None] > 0, o / np.where(l_i > 0, l_i, 1.0)[..., None], 0.0)


LOG2_127_F32 = np.float32(6.988684686772166)


def _bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 values rounded to bf16 (round to nearest even), returned as float64."""
    from .quant import bf16_bits_to_f32, f32_to_bf16_bits
    return bf16_bits_to_f32(f32_to_bf16_bits(x.astype(np.float32))).astype(np.float64)


def attn_w8a8_fwd_bf16pv_model(q_i8, q_scale, k_i8, k_scale, v_i8, v_scale, causal=False,
                               causal_diag=0, excess=100.0):
    """The per-warp W8A8 arithmetic of this build's kernel (not the reference's):
    per 32-key half h the codes are rint(2^(t*qs - (tmax_h - log2 127))) as in the
    reference, but each code enters the PV product as bf16(code * f_h) with
    f_h = 2^(tmax_h - m) / 127 against the int8 V codes, where m is the row's
    reference point: set by its first visible half's max and raised to a half's
    max (O and l rescaled) only when that max exceeds m by more than `excess`.
    The row sum adds the unrounded 2^(t*qs - (tmax_h - log2 127)) * f_h.
    Logits, codes and factors follow the kernel's fp32 evaluation; sums are
    float64. Used to bound the bf16 operand rounding: see
    tests/test_w8a8_gpu.py."""
    B, Hq, M, D = q_i8.shape
    N = k_i8.shape[2]
    kvh = kv_head_index(Hq, k_i8.shape[1])
    acc = scores_i32(q_i8, k_i8).astype(np.float32)
    ks = k_scale[:, kvh].astype(np.float32)
    t = (acc * ks[..., None, :]).astype(np.float32)              # [B,Hq,M,N]
    ok = valid_mask(M, N, causal, -1, causal_diag if causal else 0)
    t = np.where(ok, t, np.float32(-np.inf))
    qs = q_scale.astype(np.float32)[..., None]                   # [B,Hq,M,1]
    vq = v_i8[:, kvh].astype(np.float64)
    vs = v_scale[:, kvh].astype(np.float64)
    o = np.zeros((B, Hq, M, D))
    l = np.zeros((B, Hq, M))
    m = np.full((B, Hq, M), -np.inf, np.float32)
    for h0 in range(0, N, 32):
        x = t[..., h0:h0 + 32]
        tm = (x.max(-1) * qs[..., 0]).astype(np.float32)           # [B,Hq,M]
        live = np.isfinite(tm)
        first = live & ~np.isfinite(m)
        m = np.where(first, tm, m)
        up = live & ~first & (tm > m + np.float32(excess))
        if up.any():
            f = np.where(up, np.exp2(m.astype(np.float64) - tm), 1.0)
            o *= f[..., None]
            l *= f
            m = np.where(up, tm, m)
        sub = np.where(live, (tm - LOG2_127_F32).astype(np.float32), np.float32(0))
        with np.errstate(invalid="ignore"):
            z = (x.astype(np.float64) * qs.astype(np.float64) - sub[..., None]).astype(np.float32)
            y = np.where(np.isfinite(z), np.exp2(z.astype(np.float64)).astype(np.float32),
                         np.float32(0))
            fac = np.where(live, (np.exp2((tm - m).astype(np.float64)).astype(np.float32)
                                  * np.float32(1.0 / 127.0)).astype(np.float32), np.float32(0))
        code = np.rint(y).astype(np.float32)
        pe = _bf16_round((code * fac[..., None]).astype(np.float32))
        o += np.matmul(pe, vq[..., h0:h0 + 32, :])
        l += y.astype(np.float64).sum(-1) * fac.astype(np.float64)
    out = np.where(l[..., None] > 0, o / np.where(l > 0, l, 1.0)[..., None], 0.0)
    return out * vs[:, :, None, :]


def attn_int8_decode(q_i8, q_scale, k_i8, k_scale, v, num_splits):
    """Split-KV decode: q_i8 [B,Hq,D], q_scale [B,Hq] -> out [B,Hq,D] float64,
    via per-split partials and the LSE merge (reference attn_decode.cuh:68-71,129,430-466)."""
    B, Hq, D = q_i8.shape
    N = k_i8.shape[2]
    s_all = logits(scores_i32(q_i8[:, :, None, :], k_i8), q_scale[..., None], k_scale, Hq)[:, :, 0, :]
    vv = v[:, kv_head_index(Hq, v.shape[1])].astype(np.float64)
    per = (N + num_splits - 1) // num_splits
    parts = []
    for sp in range(num_splits):
        n0, n1 = sp * per, min(N, (sp + 1) * per)
        if n1 <= n0:
            parts.append((np.zeros((B, Hq, D)), np.full((B, Hq), DEC_NEG_INF), np.zeros((B, Hq))))
            continue
        s = s_all[..., n0:n1].astype(np.float64)
        m = s.max(-1)
        p = np.exp2(s - m[..., None])
        parts.append((np.einsum("bhn,bhnd->bhd", p, vv[:, :, n0:n1]), m, p.sum(-1)))
    gm = np.max([pm for _, pm, _ in parts], axis=0)
    num = np.zeros((B, Hq, D))
    den = np.zeros((B, Hq))
    for o, m, l in parts:
        w = np.where(m == DEC_NEG_INF, 0.0, np.exp2(m - gm))
        num += o * w[..., None]
        den += l * w
    return np.where(den[..., None] > 0, num / np.where(den > 0, den, 1.0)[..., None], 0.0)


def attn_int8_decode_kv8(q_i8, q_scale, k_i8, k_scale, v_i8, v_scale, num_splits):
    """Split-KV decode over an int8 V cache with per-channel scale v_scale [B,Hkv,D]
    (reference attn_decode.cuh:141-224): per split, O = (sum_n p_n * v_i8[n]) *
    v_scale[d], then the same LSE merge as attn_int8_decode."""
    B, Hq, D = q_i8.shape
    N = k_i8.shape[2]
    idx = kv_head_index(Hq, v_i8.shape[1])
    s_all = logits(scores_i32(q_i8[:, :, None, :], k_i8), q_scale[..., None], k_scale, Hq)[:, :, 0, :]
    vv = v_i8[:, idx].astype(np.float64)
    vs = v_scale[:, idx].astype(np.float64)  # [B,Hq,D]
    per = (N + num_splits - 1) // num_splits
    gm = np.full((B, Hq), DEC_NEG_INF)
    parts = []
    for sp in range(num_splits):
        n0, n1 = sp * per, min(N, (sp + 1) * per)
        if n1 <= n0:
            parts.append((np.zeros((B, Hq, D)), np.full((B, Hq), DEC_NEG_INF), np.zeros((B, Hq))))
            continue
        s = s_all[..., n0:n1].astype(np.float64)
        m = s.max(-1)
        p = np.exp2(s - m[..., None])
        o = np.einsum("bhn,bhnd->bhd", p, vv[:, :, n0:n1]) * vs
        parts.append((o, m, p.sum(-1)))
        gm = np.maximum(gm, m)
    num = np.zeros((B, Hq, D))
    den = np.zeros((B, Hq))
    for o, m, l in parts:
        w = np.where(m == DEC_NEG_INF, 0.0, np.exp2(m - gm))
        num += o * w[..., None]
        den += l * w
    return np.where(den[..., None] > 0, num / np.where(den > 0, den, 1.0)[..., None], 0.0)


def paged_choose_num_splits(n_len_max: int, bhq: int) -> int:
    """Auto split count of the paged decode (reference attn_paged_decode.cu:14-31)."""
    if n_len_max <= 0 or bhq <= 0:
        return 1
    s_occ = (2048 + bhq - 1) // bhq
    s_lo = (n_len_max + 255) // 256
    s_hi = max(1, (n_len_max + 47) // 48)
    s = min(max(s_occ, s_lo), s_hi)
    return max(1, min(s, 256))


def gather_paged(cache, block_table, b, n, Hkv_axis=1):
    """Rows 0..n-1 of sequence b from a paged cache [num_blocks, Hkv, bs, ...] -> [Hkv, n, ...]."""
    bs = cache.shape[2]
    pos = np.arange(n)
    blk = np.asarray(block_table)[b, pos // bs]
    return np.swapaxes(cache[blk, :, pos % bs], 0, 1)


def attn_paged_decode(q_i8, q_scale, k_cache, k_scale, v_cache, v_scale, block_table,
                      context_lens, max_context_len, num_splits):
    """Paged split-KV decode (reference attn_paged_decode.cuh:126-262): q_i8 [B,Hq,D],
    q_scale [B,Hq]; sequence b has context_lens[b] keys at logical positions mapped
    through block_table; split s covers [s*per, min(len_b, (s+1)*per)) with
    per = ceil(max_context_len / ns); O accumulates p * v_i8 * v_scale[token];
    same LSE merge as attn_int8_decode. Returns [B,Hq,D] float64."""
    B, Hq, D = q_i8.shape
    Hkv = k_cache.shape[1]
    idx = kv_head_index(Hq, Hkv)
    per = (max_context_len + num_splits - 1) // num_splits
    out = np.zeros((B, Hq, D))
    for b in range(B):
        # a context length above max_context_len counts as max_context_len (this
        # build's contract; the reference leaves that case unchecked)
        n = min(int(context_lens[b]), int(max_context_len))
        if n == 0:
            continue
        kb = gather_paged(k_cache, block_table, b, n)[idx]          # [Hq, n, D]
        ksb = gather_paged(k_scale, block_table, b, n)[idx]         # [Hq, n]
        vb = gather_paged(v_cache, block_table, b, n)[idx].astype(np.float64)
        vsb = gather_paged(v_scale, block_table, b, n)[idx].astype(np.float64)
        acc = np.einsum("hd,hnd->hn", q_i8[b].astype(np.float64), kb.astype(np.float64))
        s_all = ((acc.astype(np.float32) * q_scale[b][:, None].astype(np.float32))
                 * ksb.astype(np.float32)).astype(np.float64)
        gm = np.full(Hq, DEC_NEG_INF)
        parts = []
        for sp in range(num_splits):
            n0, n1 = sp * per, min(n, (sp + 1) * per)
            if n1 <= n0:
                continue
            s = s_all[:, n0:n1]
            m = s.max(-1)
            p = np.exp2(s - m[:, None])
            o = np.einsum("hn,hnd->hd", p * vsb[:, n0:n1], vb[:, n0:n1])
            parts.append((o, m, p.sum(-1)))
            gm = np.maximum(gm, m)
        num = np.zeros((Hq, D))
        den = np.zeros(Hq)
        for o, m, l in parts:
            w = np.exp2(m - gm)
            num += o * w[:, None]
            den += l * w
        out[b] = np.where(den[:, None] > 0, num / np.where(den > 0, den, 1.0)[:, None], 0.0)
    return out


def attention_fp64(q, k, v, causal=False, scale=None):
    """Textbook softmax attention in float64 on real-valued q [B,Hq,M,D], k, v [B,Hkv,N,D]."""
    B, Hq, M, D = q.shape
    N = k.shape[2]
    idx = kv_head_index(Hq, k.shape[1])
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    s = np.matmul(q.astype(np.float64), np.swapaxes(k[:, idx].astype(np.float64), -1, -2)) * scale
    if causal:
        s = np.where(valid_mask(M, N, True), s, -np.inf)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.matmul(p, v[:, idx].astype(np.float64))

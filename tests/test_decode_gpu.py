"""GPU parity of split-KV decode against the oracle's per-split partials + LSE merge."""
import numpy as np
import pytest
import torch

import superl8_amd as sl8
from oracle import attention as oa
from oracle import quant as oqn
from superl8_amd import _C, quant
from tests.tolerances import assert_close_abs, assert_finite, assert_int8_quality

pytestmark = pytest.mark.gpu

DECODE_SHAPES = [  # reference tests/test_decode.py:28-43
    (1, 8, 8, 512, 64), (4, 8, 8, 1024, 128), (1, 16, 4, 2000, 128), (2, 8, 1, 777, 64),
    (1, 32, 8, 4096, 128), (1, 4, 4, 512, 256), (2, 8, 2, 1024, 256), (1, 16, 4, 777, 256),
    (1, 32, 1, 300, 128),  # MQA with 32 query heads per KV head
    (3, 6, 2, 5, 64),      # fewer keys than splits
    (2, 8, 2, 1000, 64), (1, 64, 8, 1500, 128), (1, 16, 2, 333, 256), (2, 8, 4, 999, 128),  # streaming paths
    (2, 8, 2, 1000, 32), (1, 16, 4, 777, 32), (1, 8, 8, 300, 32),  # head dim 32 (reference attn_decode.cu:195)
]


def _np(x):
    return x.detach().cpu().numpy()


def _qkv(shape, device):
    b, hq, hkv, n, d = shape
    q = torch.randn(b, hq, 1, d, device=device, dtype=torch.float16)
    k = torch.randn(b, hkv, n, d, device=device, dtype=torch.float16)
    v = torch.randn(b, hkv, n, d, device=device, dtype=torch.float16)
    return q, k, v


def _prep(q, k):
    q_i8, qs, k_i8, ks, _ = quant.quantize_qk(q, k)
    return q_i8, qs.reshape(q.shape[0], q.shape[1], 1).contiguous(), k_i8, ks.squeeze(-1).contiguous()


@pytest.mark.parametrize("shape", DECODE_SHAPES)
@pytest.mark.parametrize("ns", [-1, 1, 16, 256])
def test_kernel_matches_oracle(device, shape, ns):
    q, k, v = _qkv(shape, device)
    q_i8, qs, k_i8, ks = _prep(q, k)
    out = _C.attn_int8_decode(q_i8, qs, k_i8, ks, v, ns)
    n_splits = ns if ns > 0 else _C.choose_n_splits(shape[3], shape[0], shape[2])
    ref = oa.attn_int8_decode(_np(q_i8)[:, :, 0], _np(qs)[:, :, 0], _np(k_i8), _np(ks),
                              _np(v.float()), n_splits)
    assert out.shape == q.shape and out.dtype == torch.float16
    assert_close_abs(out[:, :, 0], ref, atol=2e-3, rtol=2e-3, what=f"decode {shape} ns={ns}")


@pytest.mark.parametrize("shape", DECODE_SHAPES)
@pytest.mark.parametrize("ns", [-1, 16])
def test_fp16_k_scale_matches_oracle(device, shape, ns):
    """fp16 per-token K scales (BASELINE config 3's cache format): the kernel
    widens them exactly, so the oracle on the same fp16 values is the bar."""
    q, k, v = _qkv(shape, device)
    q_i8, qs, k_i8, ks = _prep(q, k)
    ks16 = ks.half()
    out = _C.attn_int8_decode(q_i8, qs, k_i8, ks16, v, ns)
    n_splits = ns if ns > 0 else _C.choose_n_splits(shape[3], shape[0], shape[2])
    ref = oa.attn_int8_decode(_np(q_i8)[:, :, 0], _np(qs)[:, :, 0], _np(k_i8),
                              _np(ks16.float()), _np(v.float()), n_splits)
    assert_close_abs(out[:, :, 0], ref, atol=2e-3, rtol=2e-3, what=f"decode ks16 {shape} ns={ns}")
    # same keys with the fp32 contract on the widened scales: identical kernels after the load
    out32 = _C.attn_int8_decode(q_i8, qs, k_i8, ks16.float(), v, ns)
    assert torch.equal(out, out32)


@pytest.mark.parametrize("shape", DECODE_SHAPES[:8])
def test_end_to_end_quality(device, shape):
    q, k, v = _qkv(shape, device)
    out = sl8.attn_int8_decode(q, k, v)
    ref = oa.attention_fp64(_np(q.float()), _np(k.float()), _np(v.float()))
    assert_finite(out)
    assert_int8_quality(out, ref, what=f"decode {shape}")


@pytest.mark.parametrize("d", [64, 128])
def test_decode_matches_prefill(device, d):
    """reference tests/test_decode.py:60-66."""
    from tests.tolerances import cos_sim

    q, k, v = _qkv((2, 8, 2, 1536, d), device)
    a = sl8.attn_int8_decode(q, k, v)
    b = sl8.attn_int8_fwd(q, k, v)
    assert cos_sim(a, b) >= 0.999


def test_deterministic_and_validation(device):
    q, k, v = _qkv((2, 8, 8, 1024, 64), device)
    r0 = sl8.attn_int8_decode(q, k, v)
    for _ in range(3):
        assert torch.equal(sl8.attn_int8_decode(q, k, v), r0)
    q_i8, qs, k_i8, ks = _prep(q, k)
    with pytest.raises(RuntimeError, match="num_splits"):
        _C.attn_int8_decode(q_i8, qs, k_i8, ks, v, 0)
    with pytest.raises(RuntimeError, match="num_splits"):
        _C.attn_int8_decode(q_i8, qs, k_i8, ks, v, 257)
    empty = _C.attn_int8_decode(q_i8, qs, k_i8[:, :, :0].contiguous(), ks[:, :, :0].contiguous(),
                                v[:, :, :0].contiguous(), -1)
    assert not empty.any()


@pytest.mark.parametrize("ks16", [False, True])
def test_config3_shape_against_oracle(device, ks16):
    """BASELINE config 3 (B16 Hq32 Hkv8 N32768 D128, 16 splits) as the config
    states it: the K cache is N(0,1) fp16 K quantised per token (codes and scales
    checked bit-exact against the oracle on the compared sequences), its scales
    kept as fp32 (the reference contract) or fp16 (the config text). The output of
    all 16 sequences (every query head) is checked against the oracle, the K
    codes of 4 sequences bit for bit."""
    torch.manual_seed(3)
    B, Hq, Hkv, N, D = 16, 32, 8, 32768, 128
    q = torch.randn(B, Hq, 1, D, device=device, dtype=torch.float16)
    k = torch.randn(B, Hkv, N, D, device=device, dtype=torch.float16)
    v = torch.randn(B, Hkv, N, D, device=device, dtype=torch.float16)
    k_i8, ks = _C.quantize_i8_rowwise(k.reshape(-1, D))
    k_i8, ks = k_i8.reshape(B, Hkv, N, D), ks.reshape(B, Hkv, N)
    for b in (0, 5, 10, 15):
        rq, rs = oqn.quantize_rows(_np(k[b].float()).reshape(-1, D))
        np.testing.assert_array_equal(_np(k_i8[b]).reshape(-1, D), rq)
        np.testing.assert_array_equal(_np(ks[b]).reshape(-1), rs)
    del k
    if ks16:
        ks = ks.half()
    q_i8, qs = _C.quantize_i8_rowwise(q.reshape(-1, D))
    qs = (qs * 0.1275).reshape(B, Hq, 1).contiguous()
    q_i8 = q_i8.reshape(B, Hq, 1, D)
    out = _C.attn_int8_decode(q_i8, qs, k_i8, ks, v, 16)
    for b in range(B):
        ref = oa.attn_int8_decode(_np(q_i8[b:b + 1])[:, :, 0], _np(qs[b:b + 1])[:, :, 0],
                                  _np(k_i8[b:b + 1]), _np(ks[b:b + 1].float()),
                                  _np(v[b:b + 1].float()), 16)
        assert_close_abs(out[b:b + 1, :, 0], ref, atol=2e-3, rtol=2e-3, what=f"config3 b={b}")


# ---------------------------------------------------------------------------
# int8 V cache (reference attn_decode.cuh:141-224, ops.py:531-584,671-727)
# ---------------------------------------------------------------------------
def _kv8(v):
    v_i8, vs = _C.quantize_v_perchannel(v)
    return v_i8, vs.squeeze(-2).contiguous()


@pytest.mark.parametrize("shape", DECODE_SHAPES)
@pytest.mark.parametrize("ns", [-1, 1, 16])
def test_kv8_kernel_matches_oracle(device, shape, ns):
    q, k, v = _qkv(shape, device)
    q_i8, qs, k_i8, ks = _prep(q, k)
    v_i8, vs = _kv8(v)
    out = _C.attn_int8_decode_kv8(q_i8, qs, k_i8, ks, v_i8, vs, ns)
    n_splits = ns if ns > 0 else _C.choose_n_splits(shape[3], shape[0], shape[2])
    ref = oa.attn_int8_decode_kv8(_np(q_i8)[:, :, 0], _np(qs)[:, :, 0], _np(k_i8), _np(ks),
                                  _np(v_i8), _np(vs), n_splits)
    assert out.shape == q.shape and out.dtype == torch.float16
    assert_close_abs(out[:, :, 0], ref, atol=2e-3, rtol=2e-3, what=f"decode_kv8 {shape} ns={ns}")


@pytest.mark.parametrize("shape", [(1, 8, 8, 512, 64), (2, 32, 8, 3000, 128), (1, 16, 2, 333, 256)])
@pytest.mark.parametrize("rotate", [False, True])
def test_decode_cached_end_to_end(device, shape, rotate):
    """quantize_kv_cache once, then attn_decode_cached per step: the reference's
    int8-PV quality bars against fp64 attention on the fp16 inputs."""
    q, k, v = _qkv(shape, device)
    cache = sl8.quantize_kv_cache(k, v, rotate=rotate)
    out = sl8.attn_decode_cached(q, *cache, rotate=rotate)
    ref = oa.attention_fp64(_np(q.float()), _np(k.float()), _np(v.float()))
    assert_finite(out)
    assert_int8_quality(out, ref, min_cos=0.998, max_rel_l1=0.03, min_sqnr_db=18,
                        what=f"decode_cached {shape}")


def test_decode_cached_rejects(device):
    q, k, v = _qkv((1, 4, 4, 64, 64), device)
    k_i8, ks, v_i8, vs_tok = sl8.quantize_kv_cache(k, v, v_quant="per_token")
    with pytest.raises(RuntimeError, match="per-token"):
        sl8.attn_decode_cached(q, k_i8, ks, v_i8, vs_tok)
    with pytest.raises(ValueError):
        sl8.quantize_kv_cache(k, v, v_quant="per_block")
    k_i8, ks, v_i8, vs = sl8.quantize_kv_cache(k, v)
    with pytest.raises(RuntimeError, match="int8"):
        _C.attn_int8_decode_kv8(k_i8[:, :, :1], ks[:, :, :1], k_i8, ks, v.contiguous(), vs)


# ---------------------------------------------------------------------------
# Paged int8 KV cache (reference attn_paged_decode.cuh, ops.py:730-849)
# ---------------------------------------------------------------------------

PAGED_CASES = [  # B, Hq, Hkv, D, block_size, lens
    (2, 8, 2, 64, 16, (50, 7)), (3, 32, 8, 128, 16, (1000, 1, 333)), (1, 16, 4, 256, 32, (257,)),
    (2, 8, 8, 128, 64, (64, 0)), (4, 12, 4, 64, 8, (9, 100, 31, 64)), (1, 32, 1, 128, 16, (600,)),
    (2, 8, 2, 32, 16, (50, 333)), (1, 16, 4, 32, 32, (257,)),  # head dim 32
    (2, 8, 2, 128, 12, (100, 37)), (1, 32, 8, 64, 24, (300,)),  # block sizes not powers of two
]


def _paged_cache(case, device, seed=0):
    B, Hq, Hkv, D, bs, lens = case
    g = torch.Generator().manual_seed(seed)
    nb_seq = [max(1, (n + bs - 1) // bs) for n in lens]
    nblk = sum(nb_seq) + 3
    kc = torch.randint(-127, 128, (nblk, Hkv, bs, D), generator=g, dtype=torch.int8)
    vc = torch.randint(-127, 128, (nblk, Hkv, bs, D), generator=g, dtype=torch.int8)
    ks = torch.rand(nblk, Hkv, bs, generator=g) * 0.02 + 1e-3
    vs = torch.rand(nblk, Hkv, bs, generator=g) * 0.02 + 1e-3
    perm = torch.randperm(nblk, generator=g)
    bt = torch.zeros(B, max(nb_seq), dtype=torch.int32)
    used = 0
    for b, nb in enumerate(nb_seq):
        bt[b, :nb] = perm[used:used + nb]
        used += nb
    q = torch.randint(-127, 128, (B, Hq, 1, D), generator=g, dtype=torch.int8)
    qs = torch.rand(B, Hq, 1, generator=g) * 0.01 + 1e-3
    ctx = torch.tensor(lens, dtype=torch.int32)
    return [t.to(device) for t in (q, qs, kc, ks, vc, vs, bt, ctx)]


@pytest.mark.parametrize("case", PAGED_CASES)
@pytest.mark.parametrize("ns", [-1, 1, 7])
def test_paged_kernel_matches_oracle(device, case, ns):
    B, Hq, Hkv, D, bs, lens = case
    q, qs, kc, ks, vc, vs, bt, ctx = _paged_cache(case, device)
    nmax = max(lens)
    out = _C.attn_paged_decode(q, qs, kc, ks, vc, vs, bt, ctx, bs, nmax, ns)
    n_splits = ns if ns > 0 else _C.paged_choose_n_splits(nmax, B * Hq)
    assert n_splits == oa.paged_choose_num_splits(nmax, B * Hq) or ns > 0
    ref = oa.attn_paged_decode(_np(q)[:, :, 0], _np(qs)[:, :, 0], _np(kc), _np(ks), _np(vc),
                               _np(vs), _np(bt), _np(ctx), nmax, n_splits)
    assert out.shape == (B, Hq, 1, D) and out.dtype == torch.float16
    assert_close_abs(out[:, :, 0], ref, atol=2e-3, rtol=2e-3, what=f"paged {case} ns={ns}")


@pytest.mark.parametrize("case", [(2, 8, 2, 128, 16, (50, 7)), (3, 32, 8, 128, 16, (1000, 1, 333)),
                                  (1, 16, 2, 128, 32, (100,)), (2, 16, 2, 64, 16, (20, 33))])
def test_paged_unwritten_slots_never_leak(device, case):
    """Slots past a sequence's length in its last block hold garbage (here NaN
    scales and arbitrary codes): the result equals the oracle's on the written
    rows, for block-aligned tiles (buffer copies of whole blocks) and others."""
    B, Hq, Hkv, D, bs, lens = case
    q, qs, kc, ks, vc, vs, bt, ctx = _paged_cache(case, device)
    ks, vs = ks.clone(), vs.clone()
    for b, n in enumerate(lens):
        if n % bs:
            blk = int(bt[b, n // bs])
            ks[blk, :, n % bs:] = float("nan")
            vs[blk, :, n % bs:] = float("nan")
    nmax = max(lens)
    for ns in (-1, 1, 4):
        out = _C.attn_paged_decode(q, qs, kc, ks, vc, vs, bt, ctx, bs, nmax, ns)
        n_splits = ns if ns > 0 else _C.paged_choose_n_splits(nmax, B * Hq)
        ref = oa.attn_paged_decode(_np(q)[:, :, 0], _np(qs)[:, :, 0], _np(kc), _np(ks), _np(vc),
                                   _np(vs), _np(bt), _np(ctx), nmax, n_splits)
        assert_finite(out)
        assert_close_abs(out[:, :, 0], ref, atol=2e-3, rtol=2e-3, what=f"paged garbage {case} ns={ns}")


@pytest.mark.parametrize("ns", [-1, 3])
def test_paged_context_above_max_is_clamped(device, ns):
    """context_lens[b] > max_context_len: keys past max_context_len (and the
    block-table entries behind them) are never read; the row decodes as if
    its length were max_context_len."""
    case = (2, 8, 2, 64, 16, (64, 40))
    B, Hq, Hkv, D, bs, lens = case
    q, qs, kc, ks, vc, vs, bt, ctx = _paged_cache(case, device)
    nmax = 40
    ctx_big = torch.tensor([64, 40], dtype=torch.int32, device=device)
    # row 0's keys 40..63 (which the clamp must leave out) would change the result
    ref64 = oa.attn_paged_decode(_np(q)[:, :, 0], _np(qs)[:, :, 0], _np(kc), _np(ks), _np(vc),
                                 _np(vs), _np(bt), np.array([64, 40]), 64, 1)
    out = _C.attn_paged_decode(q, qs, kc, ks, vc, vs, bt, ctx_big, bs, nmax, ns)
    n_splits = ns if ns > 0 else _C.paged_choose_n_splits(nmax, B * Hq)
    ref = oa.attn_paged_decode(_np(q)[:, :, 0], _np(qs)[:, :, 0], _np(kc), _np(ks), _np(vc),
                               _np(vs), _np(bt), _np(ctx_big), nmax, n_splits)
    ref40 = oa.attn_paged_decode(_np(q)[:, :, 0], _np(qs)[:, :, 0], _np(kc), _np(ks), _np(vc),
                                 _np(vs), _np(bt), np.array([40, 40]), nmax, n_splits)
    np.testing.assert_array_equal(ref, ref40)
    assert np.abs(ref64[0] - ref40[0]).max() > 1e-2
    assert_close_abs(out[:, :, 0], ref, atol=2e-3, rtol=2e-3, what="paged clamp")


@pytest.mark.parametrize("D", [32, 64, 128, 256])
def test_kv_write_paged_bit_exact(device, D):
    B, Hkv, nblk, bs = 3, 4, 5, 8
    g = torch.Generator().manual_seed(D)
    kn = (torch.randn(B, Hkv, D, generator=g) * 3).half()
    vn = torch.randn(B, Hkv, D, generator=g).half()
    kn[1, 2] = 0  # a zero row: scale 1, codes 0
    slots = torch.tensor([3, 8 * 4 + 7, 8 * 2], dtype=torch.int32)
    kc = torch.full((nblk, Hkv, bs, D), 5, dtype=torch.int8)
    vc = kc.clone()
    ks = torch.full((nblk, Hkv, bs), -1.0)
    vs = ks.clone()
    tens = [t.to(device) for t in (kn, vn, slots, kc, ks, vc, vs)]
    _C.kv_write_paged(*tens)
    rk, rks, rv, rvs = _np(kc).copy(), _np(ks).copy(), _np(vc).copy(), _np(vs).copy()
    oqn.kv_write_paged(_np(kn.float()), _np(vn.float()), _np(slots), rk, rks, rv, rvs)
    np.testing.assert_array_equal(_np(tens[3]), rk)
    np.testing.assert_array_equal(_np(tens[4]), rks)
    np.testing.assert_array_equal(_np(tens[5]), rv)
    np.testing.assert_array_equal(_np(tens[6]), rvs)


@pytest.mark.parametrize("D,lens", [(128, (40, 97, 1)), (64, (130,)), (32, (70, 5))])
def test_paged_end_to_end(device, D, lens):
    """Token-by-token quantize-on-write into a shuffled block pool, then one paged
    decode for the ragged batch: the reference's int8 quality bars against fp64
    attention on the fp16 K/V (per-token V, rotated K)."""
    B, Hq, Hkv, bs = len(lens), 8, 2, 16
    nmax = max(lens)
    nb_seq = [(n + bs - 1) // bs for n in lens]
    nblk = sum(nb_seq) + 2
    perm = torch.randperm(nblk, generator=torch.Generator().manual_seed(1))
    bt = torch.zeros(B, max(nb_seq), dtype=torch.int32)
    used = 0
    for b, nb in enumerate(nb_seq):
        bt[b, :nb] = perm[used:used + nb]
        used += nb
    bt = bt.to(device)
    kc = torch.zeros(nblk, Hkv, bs, D, dtype=torch.int8, device=device)
    vc = torch.zeros_like(kc)
    ks = torch.zeros(nblk, Hkv, bs, device=device)
    vs = torch.zeros_like(ks)
    k = torch.randn(B, Hkv, nmax, D, device=device, dtype=torch.float16)
    v = torch.randn(B, Hkv, nmax, D, device=device, dtype=torch.float16)
    for t in range(nmax):
        rows = [b for b in range(B) if t < lens[b]]
        idx = torch.tensor(rows, device=device)
        slots = torch.tensor([int(bt[b, t // bs]) * bs + t % bs for b in rows], dtype=torch.int32,
                             device=device)
        sl8.quantize_kv_write_paged(k[idx, :, t].contiguous(), v[idx, :, t].contiguous(), kc, ks,
                                    vc, vs, slots)
    q = torch.randn(B, Hq, 1, D, device=device, dtype=torch.float16)
    ctx = torch.tensor(lens, dtype=torch.int32, device=device)
    out = sl8.attn_paged_decode_cached(q, kc, ks, vc, vs, bt, ctx, bs, max_context_len=nmax)
    assert_finite(out)
    for b, n in enumerate(lens):
        ref = oa.attention_fp64(_np(q[b:b + 1].float()), _np(k[b:b + 1, :, :n].float()),
                                _np(v[b:b + 1, :, :n].float()))
        assert_int8_quality(out[b:b + 1], ref, min_cos=0.998, max_rel_l1=0.03, min_sqnr_db=18,
                            what=f"paged e2e b={b} n={n}")


def test_paged_rejects(device):
    q, qs, kc, ks, vc, vs, bt, ctx = _paged_cache(PAGED_CASES[0], device)
    with pytest.raises(RuntimeError, match="block_size"):
        _C.attn_paged_decode(q, qs, kc, ks, vc, vs, bt, ctx, 8, 50)
    with pytest.raises(RuntimeError, match="capacity"):
        _C.attn_paged_decode(q, qs, kc, ks, vc, vs, bt, ctx, 16, 10 ** 6)
    with pytest.raises(RuntimeError, match="int32"):
        _C.attn_paged_decode(q, qs, kc, ks, vc, vs, bt.long(), ctx, 16, 50)

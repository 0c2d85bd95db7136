"""GPU parity of the K8V3 paged decode (int8 K + 3-bit Lloyd-Max V) against the
oracle's per-split partials and LSE merge (reference tests/test_k8v3_paged_decode.py)."""
import numpy as np
import pytest
import torch

import superl8_amd as sl8
from oracle import attention as oa
from oracle import lloydmax as olm
from superl8_amd import _C
from superl8_amd.quant import lloydmax as lm
from superl8_amd.quant.rotation import rotate_last
from tests.tolerances import assert_close_abs, assert_finite, assert_int8_quality, cos_sim

pytestmark = pytest.mark.gpu

CASES = [  # B, Hq, Hkv, D, block_size, lens
    (3, 4, 4, 128, 16, (5, 33, 64)), (3, 4, 4, 256, 16, (5, 33, 64)), (3, 8, 4, 256, 16, (5, 33, 64)),
    (3, 32, 8, 128, 16, (1000, 1, 333)), (2, 16, 2, 128, 32, (257, 64)), (1, 8, 1, 256, 64, (600,)),
    (2, 8, 8, 128, 16, (64, 0)), (4, 12, 4, 128, 8, (9, 100, 31, 64)), (1, 16, 16, 128, 16, (77,)),
    # block sizes that are not powers of two (the kernel divides instead of shifting)
    (2, 8, 2, 128, 12, (100, 37)), (1, 32, 8, 256, 24, (300,)), (3, 4, 4, 128, 48, (5, 49, 200)),
]


def _np(x):
    return x.detach().cpu().numpy()


def _store(case, device, seed=0, codebook=None):
    B, Hq, Hkv, D, bs, lens = case
    rng = np.random.default_rng(seed)
    nb_seq = [max(1, (n + bs - 1) // bs) for n in lens]
    nblk = sum(nb_seq) + 3
    perm = rng.permutation(nblk)
    bt = np.zeros((B, max(nb_seq)), np.int32)
    used = 0
    for b, nb in enumerate(nb_seq):
        bt[b, :nb] = perm[used:used + nb]
        used += nb
    kc = rng.integers(-127, 128, (nblk, Hkv, bs, D)).astype(np.int8)
    ks = (rng.random((nblk, Hkv, bs)) * 0.02 + 1e-3).astype(np.float32)
    vp = olm.pack3(rng.integers(0, 8, (nblk, Hkv, bs, D)).astype(np.uint8))
    vn = (rng.random((nblk, Hkv, bs, D // 128)) * 20 + 1).astype(np.float32)
    cb = olm.gaussian_codebook(128) if codebook is None else codebook
    q = rng.integers(-127, 128, (B, Hq, 1, D)).astype(np.int8)
    qs = (rng.random((B, Hq, 1)) * 0.01 + 1e-3).astype(np.float32)
    ctx = np.array(lens, np.int32)
    return [torch.from_numpy(np.ascontiguousarray(t)).to(device)
            for t in (q, qs, kc, ks, vp, vn, cb, bt, ctx)]


def _ref(args, nmax, ns):
    q, qs, kc, ks, vp, vn, cb, bt, ctx = [_np(t) for t in args]
    return olm.attn_paged_decode_k8v3(q[:, :, 0], qs[:, :, 0], kc, ks, vp, vn, cb, bt, ctx, nmax, ns)


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("ns", [-1, 1, 2, 7])
def test_k8v3_kernel_matches_oracle(device, case, ns):
    B, Hq, Hkv, D, bs, lens = case
    args = _store(case, device)
    nmax = max(lens)
    out = _C.attn_paged_decode_k8v3(*args, bs, nmax, ns)
    n_splits = ns if ns > 0 else _C.paged_choose_n_splits(nmax, B * Hq)
    ref = _ref(args, nmax, n_splits)
    assert out.shape == (B, Hq, 1, D) and out.dtype == torch.float16
    assert_close_abs(out[:, :, 0], ref, atol=2e-3 * max(1.0, np.abs(ref).max()), rtol=2e-3,
                     what=f"k8v3 {case} ns={ns}")


def test_k8v3_value_table_rounds_twice(device):
    """One key: the output is the dequantised V row itself. codebook = norm =
    1 + 2^-12 gives fp16(fp32(product)) = 1.0, while a single rounding of the
    exact product would give 1 + 2^-10."""
    case = (1, 4, 4, 128, 16, (1,))
    args = _store(case, device, codebook=np.full(8, 1 + 2.0 ** -12, np.float32))
    args[5].fill_(1 + 2.0 ** -12)
    out = _C.attn_paged_decode_k8v3(*args, 16, 1, 1)
    assert (out == 1.0).all(), out.flatten()[:8]


def test_k8v3_fitted_codebook_and_every_code(device):
    """An arbitrary ascending codebook (a fitted one), every code value in every
    channel position: the exact per-element value table."""
    cb = np.array([-3.5, -1.25, -0.6, -0.1, 0.05, 0.7, 1.9, 4.25], np.float32)
    case = (2, 8, 2, 256, 16, (48, 17))
    args = _store(case, device, seed=3, codebook=cb)
    # code of channel d of token t = (d + t) % 8 in the first block of every row
    nblk, Hkv, bs, D = args[2].shape
    codes = (np.arange(D)[None, None, None, :] + np.arange(bs)[None, None, :, None]) % 8
    codes = np.broadcast_to(codes, (nblk, Hkv, bs, D)).astype(np.uint8)
    args[4] = torch.from_numpy(olm.pack3(codes)).to(device)
    for ns in (1, 3):
        out = _C.attn_paged_decode_k8v3(*args, 16, 48, ns)
        assert_close_abs(out[:, :, 0], _ref(args, 48, ns), atol=2e-3 * 20, rtol=2e-3,
                         what=f"fitted codebook ns={ns}")


@pytest.mark.parametrize("case", [(2, 8, 2, 128, 16, (50, 7)), (3, 32, 8, 128, 16, (1000, 1, 333)),
                                  (1, 16, 2, 256, 32, (100,))])
def test_k8v3_unwritten_slots_never_leak(device, case):
    """Slots past a sequence's length in its last block hold garbage (NaN norms
    and scales, arbitrary codes): the result equals the oracle's on the written rows."""
    B, Hq, Hkv, D, bs, lens = case
    args = _store(case, device)
    ks, vn, bt = args[3].clone(), args[5].clone(), args[7]
    for b, n in enumerate(lens):
        if n % bs:
            blk = int(bt[b, n // bs])
            ks[blk, :, n % bs:] = float("nan")
            vn[blk, :, n % bs:] = float("nan")
    args[3], args[5] = ks, vn
    nmax = max(lens)
    for ns in (-1, 1, 4):
        out = _C.attn_paged_decode_k8v3(*args, bs, nmax, ns)
        n_splits = ns if ns > 0 else _C.paged_choose_n_splits(nmax, B * Hq)
        assert_finite(out)
        assert_close_abs(out[:, :, 0], _ref(args, nmax, n_splits), atol=2e-2, rtol=2e-3,
                         what=f"k8v3 garbage {case} ns={ns}")


def test_k8v3_context_above_max_is_clamped(device):
    case = (2, 8, 2, 128, 16, (64, 40))
    args = _store(case, device)
    args[8] = torch.tensor([64, 40], dtype=torch.int32, device=device)
    out = _C.attn_paged_decode_k8v3(*args, 16, 40, 3)
    ref40 = _ref(args[:8] + [torch.tensor([40, 40], dtype=torch.int32)], 40, 3)
    assert_close_abs(out[:, :, 0], ref40, atol=2e-2, rtol=2e-3, what="k8v3 clamp")


def test_k8v3_zero_q_scale_is_the_mean_of_valid_rows(device):
    """q_scale = 0: every valid key gets p = 1 (the output is the mean of the
    valid dequantised V rows; keys past the split's end must not leak in)."""
    case = (2, 8, 4, 128, 16, (37, 70))
    args = _store(case, device, seed=11)
    args[1] = torch.zeros_like(args[1])
    for ns in (1, 3):
        out = _C.attn_paged_decode_k8v3(*args, 16, 70, ns)
        assert_finite(out)
        assert_close_abs(out[:, :, 0], _ref(args, 70, ns), atol=2e-2, rtol=2e-3,
                         what=f"zero q_scale ns={ns}")


@pytest.mark.parametrize("ns", [16, -1])
def test_k8v3_larger_batch_matches_oracle(device, ns):
    """Config 3's head layout (Hq 32, Hkv 8) on ragged sequences of a few
    thousand keys in scattered 16-key blocks."""
    case = (2, 32, 8, 128, 16, (4096, 3000))
    args = _store(case, device, seed=12)
    out = _C.attn_paged_decode_k8v3(*args, 16, 4096, ns)
    n_splits = ns if ns > 0 else _C.paged_choose_n_splits(4096, 2 * 32)
    assert_close_abs(out[:, :, 0], _ref(args, 4096, n_splits), atol=2e-2, rtol=2e-3,
                     what=f"k8v3 larger ns={ns}")


def test_k8v3_permuted_blocks_and_deterministic(device):
    """The same logical tokens under two block tables decode bitwise-identically,
    and repeated calls are bitwise-identical (reference test_k8v3_paged_decode.py:181-260)."""
    case = (1, 8, 4, 256, 16, (64,))
    args = _store(case, device, seed=4)
    nblk = args[2].shape[0]
    perm = torch.randperm(nblk, generator=torch.Generator().manual_seed(9)).to(device)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(nblk, device=device)
    moved = list(args)
    for i in (2, 3, 4, 5):  # physical block b moves to perm[b]
        t = torch.empty_like(args[i])
        t[perm] = args[i]
        moved[i] = t
    moved[7] = perm[args[7].long()].to(torch.int32)
    a = _C.attn_paged_decode_k8v3(*args, 16, 64, 2)
    b = _C.attn_paged_decode_k8v3(*moved, 16, 64, 2)
    assert torch.equal(a, b)
    for _ in range(2):
        assert torch.equal(_C.attn_paged_decode_k8v3(*args, 16, 64, 2), a)


def _write_store(k, v, lens, bs, device, codebook=None):
    """Token-by-token writes through ops.quantize_kv_write_paged_k8v3 into a shuffled pool."""
    B, Hkv, nmax, D = k.shape
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
    ks = torch.zeros(nblk, Hkv, bs, device=device)
    vp = torch.zeros(nblk, Hkv, bs, 3 * D // 32, dtype=torch.int32, device=device)
    vn = torch.zeros(nblk, Hkv, bs, D // 128, device=device)
    cb = None
    for t in range(nmax):
        rows = [b for b in range(B) if t < lens[b]]
        idx = torch.tensor(rows, device=device)
        slots = torch.tensor([int(bt[b, t // bs]) * bs + t % bs for b in rows], dtype=torch.int32,
                             device=device)
        cb = sl8.quantize_kv_write_paged_k8v3(k[idx, :, t].contiguous(), v[idx, :, t].contiguous(),
                                              kc, ks, vp, vn, slots, codebook=codebook)
    return kc, ks, vp, vn, cb, bt


@pytest.mark.parametrize("D", [128, 256])
def test_k8v3_end_to_end_codec_bars(device, D):
    """Write K/V token by token, decode the ragged batch through ops: against the
    representable store (the oracle on the same bytes) and, with the reference's
    codec bars, against fp64 attention on the original fp16 K/V
    (reference test_k8v3_paged_decode.py:118-182)."""
    torch.manual_seed(D)
    lens, bs, Hq, Hkv = [5, 33, 64], 16, 8, 4
    B, nmax = len(lens), max(lens)
    q = torch.randn(B, Hq, 1, D, device=device, dtype=torch.float16)
    k = torch.randn(B, Hkv, nmax, D, device=device, dtype=torch.float16)
    v = torch.randn(B, Hkv, nmax, D, device=device, dtype=torch.float16)
    kc, ks, vp, vn, cb, bt = _write_store(k, v, lens, bs, device)
    ctx = torch.tensor(lens, dtype=torch.int32, device=device)
    out = sl8.attn_paged_decode_k8v3(q, kc, ks, vp, vn, cb, bt, ctx, bs, num_splits=2)
    assert out.shape == (B, Hq, 1, D)
    assert_finite(out)
    # the same bytes through the oracle (q quantised by the same kernel as ops does)
    from superl8_amd.quant import LOG2E
    qr = rotate_last(q)
    q_i8, q_s = _C.quantize_i8_rowwise(qr.reshape(-1, D).contiguous())
    q_s = q_s * (D ** -0.5 * LOG2E)
    ref = olm.attn_paged_decode_k8v3(_np(q_i8).reshape(B, Hq, D), _np(q_s).reshape(B, Hq),
                                     _np(kc), _np(ks), _np(vp), _np(vn), _np(cb), _np(bt),
                                     np.array(lens), nmax, 2)
    assert_close_abs(out[:, :, 0], ref, atol=2e-3, rtol=2e-3, what=f"k8v3 e2e store D={D}")
    # codec-honest bars against true attention (reference test_k8v3_paged_decode.py:178-181)
    for b, n in enumerate(lens[:2]):
        tr = oa.attention_fp64(_np(q[b:b + 1].float()), _np(k[b:b + 1, :, :n].float()),
                               _np(v[b:b + 1, :, :n].float()))
        assert_int8_quality(out[b:b + 1], tr, min_cos=0.98, max_rel_l1=0.25, min_sqnr_db=12.0,
                            what=f"k8v3 codec D={D} b={b}")


def test_k8v3_splits_agree_and_match_dense_decode(device):
    """num_splits 1/2/4 agree (reference test_k8v3_paged_decode.py:208-231), and the
    fused decode matches the contiguous decode over the dequantised store
    (reference :263-297)."""
    torch.manual_seed(3)
    D, Hq, Hkv, lens, bs = 256, 8, 4, [5, 33, 64], 16
    B, nmax = len(lens), max(lens)
    q = torch.randn(B, Hq, 1, D, device=device, dtype=torch.float16)
    k = torch.randn(B, Hkv, nmax, D, device=device, dtype=torch.float16)
    v = torch.randn(B, Hkv, nmax, D, device=device, dtype=torch.float16)
    kc, ks, vp, vn, cb, bt = _write_store(k, v, lens, bs, device)
    ctx = torch.tensor(lens, dtype=torch.int32, device=device)
    outs = {ns: sl8.attn_paged_decode_k8v3(q, kc, ks, vp, vn, cb, bt, ctx, bs, num_splits=ns)
            for ns in (1, 2, 4)}
    for ns, o in outs.items():
        assert cos_sim(o, outs[4]) >= 0.99999, ns
    for b, n in enumerate(lens):
        blk = bt[b, torch.arange(n, device=device) // bs].long()
        off = torch.arange(n, device=device) % bs
        kd = (kc[blk, :, off].float() * ks[blk, :, off][..., None]).permute(1, 0, 2)[None]
        codes = lm.unpack_indices_lowbit(vp[blk, :, off], 3, D)
        vd = lm.dequantize_lloydmax(codes, vn[blk, :, off], cb).half().permute(1, 0, 2)[None]
        dense = sl8.attn_int8_decode(q[b:b + 1], rotate_last(kd).half().contiguous(),
                                     vd.contiguous(), scale=D ** -0.5)
        assert_int8_quality(outs[2][b:b + 1], _np(dense.float()), what=f"k8v3 vs dense b={b}")


def test_k8v3_rejects(device):
    """reference test_k8v3_paged_decode.py:300-331."""
    h_q, h_kv, bs = 4, 4, 16
    q = torch.randn(1, h_q, 1, 64, device=device, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="lloydmax"):
        sl8.attn_paged_decode_k8v3(
            q, torch.zeros(1, h_kv, bs, 64, dtype=torch.int8, device=device),
            torch.zeros(1, h_kv, bs, device=device),
            torch.zeros(1, h_kv, bs, 6, dtype=torch.int32, device=device),
            torch.zeros(1, h_kv, bs, 1, device=device), torch.zeros(8, device=device),
            torch.tensor([[0]], dtype=torch.int32, device=device),
            torch.tensor([8], dtype=torch.int32, device=device), bs)
    q = torch.randn(1, h_q, 1, 128, device=device, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        sl8.attn_paged_decode_k8v3(
            q, torch.zeros(2, h_kv, bs, 128, dtype=torch.int8, device=device),
            torch.ones(2, h_kv, bs, device=device),
            torch.zeros(1, h_kv, bs, 12, dtype=torch.int32, device=device),
            torch.ones(1, h_kv, bs, 1, device=device), torch.zeros(8, device=device),
            torch.tensor([[0]], dtype=torch.int32, device=device),
            torch.tensor([8], dtype=torch.int32, device=device), bs)
    args = _store((1, 4, 4, 128, 16, (8,)), device)
    with pytest.raises(RuntimeError, match="v_codebook"):
        _C.attn_paged_decode_k8v3(*args[:6], torch.zeros(7, device=device), *args[7:], 16, 8, 1)
    with pytest.raises(RuntimeError, match="num_splits"):
        _C.attn_paged_decode_k8v3(*args, 16, 8, 0)

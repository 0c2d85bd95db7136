"""GPU parity at the benchmark configurations' own shapes.

* config 1: attn_int8_fwd B1 H8 S512 D64 causal, the whole output against the oracle.
* config 5: attn_w8a8_fwd B2 Hq16 Hkv2 S8192 D256 causal, 1% of the head-dim
  channels of Q and K scaled by 20, accuracy gate bypassed. The full kernel
  runs; a 64-row query block of every query head of both batches (positions
  spread over the sequence, plus the first and the last block) is compared
  with the oracle against all its keys. At this shape the outlier rows move their softmax reference point
  several times (the lazy rescale), which only long rows with large outliers
  exercise. Reference test: tests/test_attn_fwd_w8a8_outliers.py.
"""
import numpy as np
import pytest
import torch

import superl8_amd as sl8
from oracle import attention as oa
from oracle import quant as oqn
from superl8_amd import _C, quant
from tests.tolerances import assert_close_abs, assert_finite, assert_int8_quality

pytestmark = pytest.mark.gpu


def _np(x):
    return x.detach().cpu().numpy()


def test_config1_prefill_full_shape(device):
    torch.manual_seed(1)
    q = torch.randn(1, 8, 512, 64, device=device, dtype=torch.float16)
    k = torch.randn(1, 8, 512, 64, device=device, dtype=torch.float16)
    v = torch.randn(1, 8, 512, 64, device=device, dtype=torch.float16)
    q_i8, qs, k_i8, ks, _ = quant.quantize_qk(q, k)
    qs, ks = qs.squeeze(-1).contiguous(), ks.squeeze(-1).contiguous()
    out = _C.attn_int8_fwd(q_i8, qs, k_i8, ks, v, True)
    ref, _ = oa.attn_int8_fwd(_np(q_i8), _np(qs), _np(k_i8), _np(ks), _np(v.float()), True)
    assert_finite(out)
    assert_close_abs(out, ref, atol=1e-2, what="config 1 vs oracle")
    assert_int8_quality(out, ref, min_cos=0.9999, max_rel_l1=3e-3, min_sqnr_db=40)
    # public API (prologue + kernel) vs fp32 attention: the reference's int8 gate
    pub = sl8.attn_int8_fwd(q, k, v, causal=True)
    fp = oa.attention_fp64(_np(q.float()), _np(k.float()), _np(v.float()), True)
    assert_int8_quality(pub, fp, what="config 1 public API vs fp attention")


def _config5_inputs(device):
    B, Hq, Hkv, S, D = 2, 16, 2, 8192, 256
    g = torch.Generator(device="cpu").manual_seed(5)
    idx = torch.randperm(D, generator=g)[:3]  # 1% of 256 channels
    torch.manual_seed(5)
    q = torch.randn(B, Hq, S, D, device=device, dtype=torch.float16)
    k = torch.randn(B, Hkv, S, D, device=device, dtype=torch.float16)
    v = torch.randn(B, Hkv, S, D, device=device, dtype=torch.float16)
    q[..., idx] *= 20
    k[..., idx] *= 20
    return q, k, v


# (batch, query head, first query row) of the 64-row blocks compared: every
# query head of both batches, at query positions spread over the sequence
# (first, last and interior blocks)
C5_BLOCKS = [(b, h, ((7 * h + 3 * b) % 128) * 64) for b in range(2) for h in range(16)] + \
    [(0, 0, 0), (1, 15, 8128)]


@pytest.mark.parametrize("qk_quant", ["per_row", "per_wave"])
@pytest.mark.parametrize("per_warp", [True, False])
def test_config5_w8a8_full_shape(device, per_warp, qk_quant):
    """per_wave: config 5's own text, Q/K quantised per wavefront tile (32 queries,
    64 keys) by quantize_qk_per_wave; its codes are checked bit-exact against the
    oracle on the compared rows' heads before the attention is."""
    q, k, v = _config5_inputs(device)
    Hq, Hkv = q.shape[1], k.shape[1]
    gsz = Hq // Hkv
    if qk_quant == "per_wave":
        q_i8, qs, k_i8, ks, _ = quant.quantize_qk_per_wave(q, k)
        for b, h, _r0 in C5_BLOCKS[:2]:
            kv = h // gsz
            r = oqn.quantize_qk_per_wave(_np(q[b:b + 1, h:h + 1]), _np(k[b:b + 1, kv:kv + 1]))
            np.testing.assert_array_equal(_np(q_i8[b:b + 1, h:h + 1]), r[0])
            np.testing.assert_array_equal(_np(qs[b:b + 1, h:h + 1, :, 0]), r[1])
            np.testing.assert_array_equal(_np(k_i8[b:b + 1, kv:kv + 1]), r[2])
            np.testing.assert_array_equal(_np(ks[b:b + 1, kv:kv + 1, :, 0]), r[3])
    else:
        q_i8, qs, k_i8, ks, _ = quant.quantize_qk(q, k)
    qs, ks = qs.squeeze(-1).contiguous(), ks.squeeze(-1).contiguous()
    v_i8, vs = _C.quantize_v_perchannel(v)
    vs = vs.squeeze(-2).contiguous()
    out = _C.attn_w8a8_fwd(q_i8, qs, k_i8, ks, v_i8, vs, True, 0, per_warp)
    assert_finite(out)
    # the public API with the gate bypassed runs the same kernel
    if per_warp and qk_quant == "per_row":
        pub = sl8.attn_int8_fwd(q, k, v, causal=True, int8_pv=True, internal_accuracy_gate=False)
        assert torch.equal(pub, out)
    del q, k, v
    outs, refs = [], []
    for b, h, r0 in C5_BLOCKS:
        kv = h // gsz
        sl = slice(r0, r0 + 64)
        # the block sees keys <= r0 + i (M = N, bottom-right causal)
        ref = oa.attn_w8a8_fwd(_np(q_i8[b:b + 1, h:h + 1, sl]), _np(qs[b:b + 1, h:h + 1, sl]),
                               _np(k_i8[b:b + 1, kv:kv + 1]), _np(ks[b:b + 1, kv:kv + 1]),
                               _np(v_i8[b:b + 1, kv:kv + 1]), _np(vs[b:b + 1, kv:kv + 1]),
                               True, r0, per_warp)
        got = out[b:b + 1, h:h + 1, sl]
        assert_close_abs(got, ref, atol=2e-2, what=f"config 5 block {(b, h, r0)}")
        outs.append(_np(got.float()))
        refs.append(ref)
    assert_int8_quality(np.concatenate(outs), np.concatenate(refs), min_cos=0.9999,
                        max_rel_l1=5e-3, min_sqnr_db=35, what="config 5 blocks vs oracle")

"""GPU parity of the fused fp16 prologue (sl8_quantize_qk).

Its outputs must equal the separate kernels (k_mean, smooth+quantise, Q
quantise) and the oracle bit for bit, and its gate flag must equal the torch
evaluation the reference performs (reference superl8/quant/core.py:113-145).
"""
import numpy as np
import pytest
import torch

from oracle import quant as oqn
from superl8_amd import _C, ops, quant

pytestmark = pytest.mark.gpu

LOG2E = quant.LOG2E
# (B, Hq, Hkv, M, N, D): ragged key counts across mean chunks (512) and quantise
# blocks (128), M = 1 decode, more Q rows than the grid-stride cap covers at once
SHAPES = [(1, 8, 2, 512, 512, 64), (2, 6, 3, 33, 777, 128), (1, 4, 1, 5, 1, 256),
          (1, 2, 2, 1, 70001, 64), (1, 32, 8, 4096, 4096, 128), (2, 16, 2, 300, 1025, 256),
          (3, 4, 4, 1, 130, 128)]


def _np(x):
    return x.detach().cpu().numpy()


def _torch_gate(q, thr=12.0):
    a = q.float().abs()
    return bool(((a.amax(-1) / (a.median(-1).values + 1e-10)) > thr).any())


@pytest.mark.parametrize("B,Hq,Hkv,M,N,D", SHAPES)
def test_fused_prologue_matches_separate_kernels(device, B, Hq, Hkv, M, N, D):
    g = torch.Generator(device="cpu").manual_seed(B * 1000 + N + D)
    q = (torch.randn(B, Hq, M, D, generator=g) * 1.5).half().to(device)
    k = (torch.randn(B, Hkv, N, D, generator=g) * 2).half().to(device)
    k[..., 5] += 7.0
    mul = (1.0 / D ** 0.5) * LOG2E
    qi, qs, ki, ks, km, flag = _C.quantize_qk_fused(q, k, mul, 12.0)
    m_ref = _C.k_mean(k)
    qi_ref, qs_ref = _C.quantize_rows_centered(q, None, mul)
    ki_ref, ks_ref = _C.quantize_rows_centered(k, m_ref, 1.0)
    assert torch.equal(km, m_ref)
    assert torch.equal(qi, qi_ref) and torch.equal(qs, qs_ref)
    assert torch.equal(ki, ki_ref) and torch.equal(ks, ks_ref)
    assert bool(flag.item()) == _torch_gate(q)
    if q.numel() * k.numel() < 1 << 30 and N < 5000:
        rq, rqs, rk, rks, rm = oqn.quantize_qk(_np(q), _np(k))
        np.testing.assert_array_equal(_np(km), rm)
        np.testing.assert_array_equal(_np(qi), rq)
        np.testing.assert_array_equal(_np(qs), rqs)
        np.testing.assert_array_equal(_np(ki), rk)
        np.testing.assert_array_equal(_np(ks), rks)


@pytest.mark.parametrize("D", [64, 128, 256])
def test_fused_prologue_nonfinite_rows(device, D):
    """NaN and +-inf elements: the fused codes (reciprocal + exact-division
    fallback) equal the separate kernels' (IEEE division per element) bit for
    bit: a NaN element codes to -127 (the clamp fmaxf / fminf), an inf row has
    an inf scale, its inf element codes to -127 and its finite ones to 0."""
    g = torch.Generator(device="cpu").manual_seed(D + 7)
    q = torch.randn(1, 2, 40, D, generator=g).half().to(device)
    k = torch.randn(1, 1, 40, D, generator=g).half().to(device)
    q[0, 0, 3, 5] = float("nan")
    q[0, 1, 7, 0] = float("inf")
    q[0, 1, 8, D - 1] = float("-inf")
    q[0, 0, 9, :] = float("nan")
    qi, qs, _, _, _, _ = _C.quantize_qk_fused(q, k, 1.0, 0.0)
    qi_ref, qs_ref = _C.quantize_rows_centered(q, None, 1.0)
    assert torch.equal(qi, qi_ref)
    assert torch.equal(qs.isnan(), qs_ref.isnan()) and torch.equal(qs.nan_to_num(), qs_ref.nan_to_num())
    assert int(qi[0, 0, 3, 5]) == -127 and (qi[0, 0, 9] == -127).all()
    assert int(qi[0, 1, 7, 0]) == -127 and (qi[0, 1, 7, 1:] == 0).all()
    assert torch.isinf(qs[0, 1, 7]).all()
    # the finite rows are untouched by the others
    fin = torch.isfinite(q.float()).all(-1)
    qi2, qs2, _, _, _, _ = _C.quantize_qk_fused(torch.where(fin[..., None], q, 0), k, 1.0, 0.0)
    assert torch.equal(qi[fin], qi2[fin]) and torch.equal(qs[fin], qs2[fin])


@pytest.mark.parametrize("D", [64, 128, 256])
def test_fused_gate_decisions(device, D):
    torch.manual_seed(D)
    k = torch.randn(1, 2, 64, D, device=device, dtype=torch.float16)
    cases = []
    q = torch.randn(1, 4, 3000, D, device=device, dtype=torch.float16)
    cases.append(q.clone())                       # gaussian: ratio ~ 5
    q1 = q.clone(); q1[0, 3, 2999, 1] = 200.0     # one spike in the last row
    cases.append(q1)
    q2 = q.clone(); q2[0, 1, 17] = 0.0            # all-zero row: 0 / 1e-10 = 0
    cases.append(q2)
    q3 = q.clone(); q3[0, 2, 5, : D // 2 + 1] = 0.0; q3[0, 2, 5, D - 1] = 1e-3  # median 0
    cases.append(q3)
    q4 = q.clone(); q4[0, 0, 9, 0] = float("nan"); q4[0, 0, 9, 1] = 5e4  # NaN row never fires
    cases.append(q4)
    for c in cases:
        for thr in (3.0, 12.0, 1e6):
            _, _, _, _, _, flag = _C.quantize_qk_fused(c, k, 1.0, thr)
            ref, _ = _C.q_outlier_gate(c, thr)
            assert bool(flag.item()) == bool(ref.item()) == _torch_gate(c, thr), (thr,)


def test_gate_boundary_exact(device):
    """Rows built so that max/median lands on either side of the threshold by one ulp."""
    D = 128
    torch.manual_seed(3)
    k = torch.randn(1, 1, 16, D, device=device, dtype=torch.float16)
    for med, mx in [(1.0, 12.0), (1.0, 12.0078125), (0.5, 6.0), (0.5, 6.00390625), (2.0, 24.0)]:
        row = torch.full((D,), med, dtype=torch.float16)
        row[: D // 2 - 1] = med / 2
        row[-1] = mx
        q = row.reshape(1, 1, 1, D).to(device)
        _, _, _, _, _, flag = _C.quantize_qk_fused(q, k, 1.0, 12.0)
        assert bool(flag.item()) == _torch_gate(q), (med, mx)


def test_attn_fwd_routes_on_fused_gate(device):
    torch.manual_seed(11)
    q = torch.randn(1, 4, 256, 64, device=device, dtype=torch.float16)
    k = torch.randn(1, 2, 256, 64, device=device, dtype=torch.float16)
    v = torch.randn(1, 2, 256, 64, device=device, dtype=torch.float16)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
    o = ops.attn_int8_fwd(q, k, v, causal=True)
    assert (o.float() - ref.float()).abs().max().item() < 5e-2
    q[0, 1, 100, 7] = 300.0   # gate fires: the call returns full-precision SDPA exactly
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
    o = ops.attn_int8_fwd(q, k, v, causal=True)
    assert torch.equal(o, ref)


def test_fused_rejects(device):
    q = torch.randn(1, 1, 4, 96, device=device, dtype=torch.float16)
    with pytest.raises(RuntimeError):
        _C.quantize_qk_fused(q, q, 1.0)
    with pytest.raises(RuntimeError):
        _C.quantize_qk_fused(q.float()[..., :64].contiguous(), q.float()[..., :64].contiguous(), 1.0)


def test_gated_prefill_skips_or_matches(device):
    """sl8_attn_int8_fwd_gated through the C ABI: with the flag set every
    workgroup exits and the output buffer keeps its contents; with it clear the
    output is bit-identical to sl8_attn_int8_fwd's."""
    from superl8_amd import _lib
    from superl8_amd._lib import dtype_code

    torch.manual_seed(5)
    B, Hq, Hkv, M, N, D = 1, 4, 2, 200, 300, 128
    q = torch.randn(B, Hq, M, D, device=device, dtype=torch.float16)
    k = torch.randn(B, Hkv, N, D, device=device, dtype=torch.float16)
    v = torch.randn(B, Hkv, N, D, device=device, dtype=torch.float16)
    q_i8, qs, k_i8, ks, _ = quant.quantize_qk(q, k)
    qs, ks = qs.squeeze(-1).contiguous(), ks.squeeze(-1).contiguous()
    ref = _C.attn_int8_fwd(q_i8, qs, k_i8, ks, v, True)
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    for flag_val in (1, 0):
        flag = torch.full((1,), flag_val, device=device, dtype=torch.int32)
        out = torch.full_like(ref, 7.0)
        rc = lib.sl8_attn_int8_fwd_gated(q_i8.data_ptr(), qs.data_ptr(), k_i8.data_ptr(),
                                         ks.data_ptr(), v.data_ptr(), dtype_code(v.dtype),
                                         out.data_ptr(), None, B, Hq, Hkv, M, N, D, 1, -1,
                                         None, 0, flag.data_ptr(), stream)
        assert rc == 0, lib.sl8_last_error()
        torch.cuda.synchronize()
        if flag_val:
            assert torch.equal(out, torch.full_like(ref, 7.0))
        else:
            assert torch.equal(out, ref)


def test_public_prefill_deferred_gate_is_the_two_step_path(device):
    """ops.attn_int8_fwd reads the fused prologue's gate flag after launching the
    attention: a call whose gate stays quiet returns exactly prologue + kernel."""
    torch.manual_seed(6)
    q = torch.randn(2, 8, 300, 128, device=device, dtype=torch.float16)
    k = torch.randn(2, 2, 300, 128, device=device, dtype=torch.float16)
    v = torch.randn(2, 2, 300, 128, device=device, dtype=torch.float16)
    o = ops.attn_int8_fwd(q, k, v, causal=True)
    q_i8, qs, k_i8, ks, _ = quant.quantize_qk(q, k)
    two_step = _C.attn_int8_fwd(q_i8, qs.squeeze(-1).contiguous(), k_i8,
                                ks.squeeze(-1).contiguous(), v, True)
    assert torch.equal(o, two_step)


def test_public_prefill_gate_read_back_to_back(device):
    """Calls issued back to back, alternating inputs whose gate fires and stays
    quiet: each call's decision is its own (the flag is read from a pinned copy
    made right after its prologue, while its attention may still be running)."""
    torch.manual_seed(8)
    q = torch.randn(1, 4, 256, 128, device=device, dtype=torch.float16)
    k = torch.randn(1, 2, 256, 128, device=device, dtype=torch.float16)
    v = torch.randn(1, 2, 256, 128, device=device, dtype=torch.float16)
    q_out = q.clone()
    q_out[0, 1, 7, 3] = 300.0  # one dominated row: the gate fires for this input
    quiet = ops.attn_int8_fwd(q, k, v, causal=True)
    loud = ops.attn_int8_fwd(q_out, k, v, causal=True)
    fp_loud = torch.nn.functional.scaled_dot_product_attention(
        q_out, k, v, is_causal=True, enable_gqa=True)
    assert torch.allclose(loud.float(), fp_loud.float(), atol=2e-3, rtol=0)
    assert not torch.equal(quiet, loud)
    outs = [ops.attn_int8_fwd(x, k, v, causal=True) for x in (q, q_out, q, q, q_out, q_out, q)]
    torch.cuda.synchronize()
    for x, o in zip((q, q_out, q, q, q_out, q_out, q), outs):
        assert torch.equal(o, quiet if x is q else loud)

"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every fixture exactly (guards the checker).
GPU: the HIP kernels reproduce them to the parity bars.
"""
import os

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import q4k as oq
from oracle import quant as oqn
from tests.tolerances import assert_close_abs

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return dict(np.load(os.path.join(G, name), allow_pickle=False))


def test_oracle_reproduces_fixtures():
    f = _load("quant_rows.npz")
    q, s = oqn.quantize_rows(f["x"].astype(np.float32))
    np.testing.assert_array_equal(q, f["q"])
    np.testing.assert_array_equal(s, f["scale"])
    a = _load("attention.npz")
    q_i8, qs, k_i8, ks, km = oqn.quantize_qk(a["q"], a["k"])
    for got, key in ((q_i8, "q_i8"), (qs, "q_scale"), (k_i8, "k_i8"), (ks, "k_scale"), (km, "k_mean")):
        np.testing.assert_array_equal(got, a[key])
    np.testing.assert_array_equal(oa.scores_i32(q_i8, k_i8), a["scores"])
    out, lse = oa.attn_int8_fwd(q_i8, qs, k_i8, ks, a["v"].astype(np.float32), True)
    np.testing.assert_allclose(out, a["out_causal"], rtol=0, atol=1e-12)
    w = _load("q4k.npz")
    np.testing.assert_array_equal(oq.dequant(w["w"], 512), w["dequant"])
    np.testing.assert_allclose(oq.gemv(w["x_i8"], w["x_scale"], w["w"], 512), w["y"], rtol=1e-12)


@pytest.mark.gpu
def test_kernels_reproduce_fixtures(device):
    from superl8_amd import _C, quant

    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    f = _load("quant_rows.npz")
    q, s = _C.quantize_i8_rowwise(t(f["x"]))
    np.testing.assert_array_equal(q.cpu().numpy(), f["q"])
    np.testing.assert_array_equal(s.cpu().numpy(), f["scale"])
    a = _load("attention.npz")
    q_i8, qs, k_i8, ks, km = quant.quantize_qk(t(a["q"]), t(a["k"]))
    np.testing.assert_array_equal(q_i8.cpu().numpy(), a["q_i8"])
    np.testing.assert_array_equal(k_i8.cpu().numpy(), a["k_i8"])
    np.testing.assert_array_equal(ks.cpu().numpy()[..., 0], a["k_scale"])
    np.testing.assert_array_equal(_C.attn_int8_qk_scores(q_i8, k_i8).cpu().numpy(), a["scores"])
    qs2, ks2 = qs.squeeze(-1).contiguous(), ks.squeeze(-1).contiguous()
    out, lse = _C.attn_int8_fwd_train(q_i8, qs2, k_i8, ks2, t(a["v"]), True)
    assert_close_abs(out, a["out_causal"], atol=1e-2, what="golden prefill causal")
    # the kernel's row sums add the fp16-rounded P that enters the PV product
    # (2^-11 relative per term), as test_attn_fwd_gpu's LSE checks
    np.testing.assert_allclose(lse.cpu().numpy(), a["lse_causal"], rtol=0, atol=5e-4)
    out = _C.attn_int8_fwd(q_i8, qs2, k_i8, ks2, t(a["v"]), False)
    assert_close_abs(out, a["out_full"], atol=1e-2, what="golden prefill")
    v_i8, vs = _C.quantize_v_perchannel(t(a["v"]))
    np.testing.assert_array_equal(v_i8.cpu().numpy(), a["v_i8"])
    o8 = _C.attn_w8a8_fwd(q_i8, qs2, k_i8, ks2, v_i8, vs.squeeze(-2).contiguous(), True, 30, True)
    assert_close_abs(o8, a["out_w8a8_causal"], atol=2e-2, what="golden w8a8")
    d = _load("decode.npz")
    od = _C.attn_int8_decode(t(d["q_i8"]), t(d["q_scale"]), t(d["k_i8"]), t(d["k_scale"]),
                             t(d["v"]), int(d["num_splits"]))
    assert_close_abs(od[:, :, 0], d["out"], atol=2e-3, rtol=2e-3, what="golden decode")
    w = _load("q4k.npz")
    np.testing.assert_array_equal(_C.dequant_q4k(t(w["w"]), 512).cpu().numpy(), w["dequant"])
    y = _C.gemm_decode_q4k(t(w["x_i8"]), t(w["x_scale"]), t(w["w"]), torch.float32)
    np.testing.assert_allclose(y.cpu().numpy(), w["y"], rtol=1e-5, atol=1e-5)

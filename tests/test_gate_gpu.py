"""GPU parity of the on-device outlier gate (reference superl8/quant/core.py:113-145).

Per-row (max, lower median) must match the oracle bit for bit; the decision must
match the torch evaluation the reference performs (amax, median, fp32 ratio).
"""
import numpy as np
import pytest
import torch

from oracle import quant as oqn
from superl8_amd import _C, quant

pytestmark = pytest.mark.gpu


def _torch_gate(q, thr):
    a = q.float().abs()
    return bool(((a.amax(-1) / (a.median(-1).values + 1e-10)) > thr).any())


def _as_np(q):
    if q.dtype == torch.bfloat16:
        return oqn.bf16_bits_to_f32(q.view(torch.int16).cpu().numpy().view(np.uint16))
    return q.float().cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [32, 64, 72, 80, 128, 256])
@pytest.mark.parametrize("rows", [1, 3, 4, 5, 257, 4096])
def test_gate_stats_bit_exact(device, rows, D, dtype):
    g = torch.Generator(device="cpu").manual_seed(rows * 31 + D)
    q = (torch.randn(rows, D, generator=g) * 2.0).to(dtype).to(device)
    # edge rows: ties, zeros, one spike, all-equal, signed zeros
    if rows >= 5:
        q[0] = 0
        q[1] = 1.5
        q[2, :] = torch.tensor([-0.0, 0.0] * (D // 2), dtype=dtype)
        q[3, 7] = 300.0
        q[4, : D // 2] = 2.0
    flag, st = _C.q_outlier_gate(q, 12.0, stats=True)
    mx, md = oqn.q_outlier_stats(_as_np(q))
    got = st.cpu().numpy()
    np.testing.assert_array_equal(got[:, 0], mx)
    np.testing.assert_array_equal(got[:, 1], md)
    assert bool(flag.item()) == oqn.q_outlier_gate(_as_np(q), 12.0) == _torch_gate(q, 12.0)


@pytest.mark.parametrize("thr", [1.0, 3.0, 12.0, 1e9])
def test_gate_decision_matches_torch(device, thr):
    torch.manual_seed(5)
    for shape in [(2, 8, 333, 128), (1, 4, 17, 64), (1, 2, 40, 256)]:
        q = torch.randn(*shape, device=device, dtype=torch.float16)
        q[..., 3] *= 9.0
        flag, _ = _C.q_outlier_gate(q, thr)
        assert bool(flag.item()) == _torch_gate(q, thr)


def test_gate_single_spike_flips(device):
    q = torch.randn(4, 32, 100, 128, device=device, dtype=torch.bfloat16) * 0.5
    assert not quant.detect_q_outlier_domination(q)
    q[2, 17, 55, 9] = 400.0
    assert quant.detect_q_outlier_domination(q)
    assert _torch_gate(q, 12.0)


def test_gate_nan_row_never_fires(device):
    q = torch.randn(3, 64, device=device, dtype=torch.float32)
    q[1, 0] = float("nan")
    q[1, 1] = 1e6
    flag, st = _C.q_outlier_gate(q, 12.0, stats=True)
    assert bool(flag.item()) == _torch_gate(q, 12.0)
    assert torch.isnan(st[1]).all()


def test_gate_rejects(device):
    with pytest.raises(RuntimeError):
        _C.q_outlier_gate(torch.randn(2, 300, device=device, dtype=torch.float16))
    flag, st = _C.q_outlier_gate(torch.empty(0, 64, device=device, dtype=torch.float16), stats=True)
    assert flag.item() == 0 and st.shape == (0, 2)

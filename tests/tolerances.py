"""Accuracy gates, restating the reference's tests/tolerances.py:54-88.

int8 attention outputs are never compared with allclose against a float
oracle; they must clear cosine, relative-L1 and SQNR bars. Integer results
(codes, int32 scores, Q4_K dequant) are compared bit-exactly elsewhere.
"""
from __future__ import annotations

import numpy as np
import torch


def _f64(x):
    if isinstance(x, torch.Tensor):
        x = x.detach().float().cpu().numpy()
    return np.asarray(x, dtype=np.float64)


def sqnr_db(out, ref) -> float:
    o, r = _f64(out), _f64(ref)
    noise = ((o - r) ** 2).mean()
    if noise == 0:
        return float("inf")
    return float(10.0 * np.log10((r ** 2).mean() / noise))


def cos_sim(out, ref) -> float:
    o, r = _f64(out).ravel(), _f64(ref).ravel()
    return float(o @ r / max(np.linalg.norm(o) * np.linalg.norm(r), 1e-30))


def rel_l1(out, ref) -> float:
    o, r = _f64(out), _f64(ref)
    return float(np.abs(o - r).sum() / max(np.abs(r).sum(), 1e-12))


def assert_finite(t, what="output"):
    assert np.isfinite(_f64(t)).all(), f"{what} contains NaN/Inf"


def assert_int8_quality(out, ref, *, min_cos=0.999, max_rel_l1=0.02, min_sqnr_db=20.0,
                        what="int8 output"):
    """The reference's int8 accuracy gate (cos >= 0.999, rel-L1 <= 0.02, SQNR >= 20 dB)."""
    assert_finite(out, what)
    c, l1, s = cos_sim(out, ref), rel_l1(out, ref), sqnr_db(out, ref)
    assert c >= min_cos, f"{what}: cos-sim {c:.6f} < {min_cos}"
    assert l1 <= max_rel_l1, f"{what}: rel-L1 {l1:.4f} > {max_rel_l1}"
    assert s >= min_sqnr_db, f"{what}: SQNR {s:.1f} dB < {min_sqnr_db} dB"


def assert_close_abs(out, ref, atol, rtol=0.0, what="output"):
    o, r = _f64(out), _f64(ref)
    err = np.abs(o - r)
    lim = atol + rtol * np.abs(r)
    bad = err > lim
    assert not bad.any(), (f"{what}: {bad.sum()} / {bad.size} elements off; max err "
                           f"{err.max():.3e} (atol {atol}, rtol {rtol})")

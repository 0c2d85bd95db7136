"""Write the small seeded golden fixtures under tests/golden/ from the pinned oracle.

    python tests/golden/make_golden.py

The reference repository ships no fixture files (its tests are seeded-random), so
these vectors come from oracle/, after oracle/ is pinned by tests/test_oracle.py.
They freeze the oracle's outputs (a regression guard for the oracle itself) and give
the GPU tests fixed inputs/outputs independent of RNG state.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attention as oa  # noqa: E402
from oracle import q4k as oq  # noqa: E402
from oracle import quant as oqn  # noqa: E402


def main():
    r = np.random.default_rng(20261201)
    # per-row quantisation (incl. zero row and outlier row)
    x = (r.standard_normal((6, 96)) * 3).astype(np.float16)
    x[2] = 0
    x[4, 17] = 60.0
    q, s = oqn.quantize_rows(x.astype(np.float32))
    np.savez(os.path.join(HERE, "quant_rows.npz"), x=x, q=q, scale=s)
    # quantize_qk (smoothing + fold)
    qh = r.standard_normal((1, 4, 40, 64)).astype(np.float16)
    kh = (r.standard_normal((1, 2, 70, 64)) + 0.5).astype(np.float16)
    vh = r.standard_normal((1, 2, 70, 64)).astype(np.float16)
    q_i8, qs, k_i8, ks, km = oqn.quantize_qk(qh, kh)
    out_c, lse_c = oa.attn_int8_fwd(q_i8, qs, k_i8, ks, vh.astype(np.float32), True)
    out_n, _ = oa.attn_int8_fwd(q_i8, qs, k_i8, ks, vh.astype(np.float32), False)
    v_i8, vs = oqn.quantize_v_perchannel(vh)
    out_w8 = oa.attn_w8a8_fwd(q_i8, qs, k_i8, ks, v_i8, vs, True, 70 - 40, True)
    np.savez(os.path.join(HERE, "attention.npz"), q=qh, k=kh, v=vh, q_i8=q_i8, q_scale=qs,
             k_i8=k_i8, k_scale=ks, k_mean=km, scores=oa.scores_i32(q_i8, k_i8),
             out_causal=out_c, lse_causal=lse_c, out_full=out_n, v_i8=v_i8, v_scale=vs,
             out_w8a8_causal=out_w8)
    # decode
    dq = r.standard_normal((1, 8, 1, 64)).astype(np.float16)
    dk = r.standard_normal((1, 2, 300, 64)).astype(np.float16)
    dv = r.standard_normal((1, 2, 300, 64)).astype(np.float16)
    a, b, c, d, _ = oqn.quantize_qk(dq, dk)
    dout = oa.attn_int8_decode(a[:, :, 0], b[:, :, 0], c, d, dv.astype(np.float32), 7)
    np.savez(os.path.join(HERE, "decode.npz"), q=dq, k=dk, v=dv, q_i8=a, q_scale=b, k_i8=c,
             k_scale=d, num_splits=7, out=dout)
    # Q4_K
    w = oq.random_weights(48, 512, seed=11)
    xi = r.integers(-127, 128, (3, 512), dtype=np.int8)
    xs = (r.random(3) * 0.05).astype(np.float32)
    np.savez(os.path.join(HERE, "q4k.npz"), w=w, K=512, dequant=oq.dequant(w, 512), x_i8=xi,
             x_scale=xs, y=oq.gemv(xi, xs, w, 512))


if __name__ == "__main__":
    main()

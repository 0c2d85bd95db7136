"""The allocation-free decode entry point (sl8_attn_int8_decode_noalloc), called
through the C ABI, against the workspace entry point (sl8_attn_int8_decode) on
the same inputs: the same kernels and split count, so the outputs are
bit-identical. Two calls in a row, the second smaller, check that the shared
scratch array's leftover contents from the first call never leak into the
second."""
import ctypes

import pytest
import torch

from superl8_amd import _C, _lib

pytestmark = pytest.mark.gpu


def _inputs(B, Hq, Hkv, N, D, seed, device):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randint(-127, 128, (B, Hq, 1, D), generator=g, dtype=torch.int8)
    qs = torch.rand(B, Hq, 1, generator=g) * 0.01 + 1e-3
    k = torch.randint(-127, 128, (B, Hkv, N, D), generator=g, dtype=torch.int8)
    ks = torch.rand(B, Hkv, N, generator=g) * 0.02 + 1e-3
    v = torch.randn(B, Hkv, N, D, generator=g).to(torch.float16)
    return [t.to(device) for t in (q, qs, k, ks, v)]


def _noalloc(q, qs, k, ks, v, num_splits):
    B, Hq, _, D = q.shape
    Hkv, N = k.shape[1], k.shape[2]
    out = torch.empty((B, Hq, 1, D), device=q.device, dtype=torch.float16)
    _lib.call("sl8_attn_int8_decode_noalloc", q.data_ptr(), qs.data_ptr(), k.data_ptr(),
              ks.data_ptr(), v.data_ptr(), out.data_ptr(), B, Hq, Hkv, N, D, num_splits,
              _lib.stream_of(q))
    return out


@pytest.mark.parametrize("num_splits", [-1, 16])
def test_noalloc_matches_workspace_entry(device, num_splits):
    # config 3's head layout at a shorter cache, then a smaller call that
    # uses fewer partials of the same scratch array
    for (B, Hq, Hkv, N, D, seed) in [(16, 32, 8, 4096, 128, 1), (2, 8, 2, 777, 64, 2)]:
        q, qs, k, ks, v = _inputs(B, Hq, Hkv, N, D, seed, device)
        got = _noalloc(q, qs, k, ks, v, num_splits)
        want = _C.attn_int8_decode(q, qs, k, ks, v, num_splits)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (B, Hq, Hkv, N, D, num_splits)


def test_noalloc_rejects_oversized_partials(device):
    lib = _lib.load()
    cap = lib.sl8_attn_int8_decode_noalloc_max_bytes()
    assert cap == 8 << 20
    # 256 splits x 64 x 32 query heads x (256 + 2) floats > 8 MiB
    B, Hq, Hkv, N, D = 64, 32, 8, 65536, 256
    assert lib.sl8_attn_int8_decode_workspace(B, Hq, D, 256) > cap
    rc = lib.sl8_attn_int8_decode_noalloc(None, None, None, None, None, None, B, Hq, Hkv, N, D, 256,
                                          None)
    assert rc != 0 and b"scratch" in lib.sl8_last_error()

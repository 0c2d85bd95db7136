"""The package served under the reference's module names (superl8_amd.alias):
the hot-path functions keep the reference's parameter names, kinds and
defaults (reference superl8/ops.py, lines cited per function) and ``_C`` the
reference binding names of this path (reference csrc/fni8_api.cpp). Signature
checks only: nothing here launches a kernel."""
import inspect

import pytest

from superl8_amd import alias

P, K = inspect.Parameter.POSITIONAL_OR_KEYWORD, inspect.Parameter.KEYWORD_ONLY
E = inspect.Parameter.empty

# (name, [(param, kind, default)]) as the reference declares them
REF_OPS = [
    ("attn_int8_fwd", [("q", P, E), ("k", P, E), ("v", P, E), ("causal", K, False), ("scale", K, None),
                       ("int8_pv", K, False), ("rotate", K, False), ("window_left", K, -1),
                       ("per_warp_quant", K, True), ("internal_accuracy_gate", K, True)]),   # ops.py:70-82
    ("attn_int8_decode", [("q", P, E), ("k", P, E), ("v", P, E), ("scale", K, None), ("rotate", K, False),
                          ("num_splits", K, None)]),                                      # ops.py:230-238
    ("quantize_kv_cache", [("k", P, E), ("v", P, E), ("rotate", K, False), ("v_quant", K, "per_channel")]),  # ops.py:531-533
    ("attn_decode_cached", [("q", P, E), ("k_i8", P, E), ("k_scale", P, E), ("v_i8", P, E), ("v_scale", P, E),
                            ("scale", K, None), ("rotate", K, False), ("num_splits", K, None)]),  # ops.py:671-681
    ("quantize_kv_write_paged", [("k_new", P, E), ("v_new", P, E), ("k_cache", P, E), ("k_scale", P, E),
                                 ("v_cache", P, E), ("v_scale", P, E), ("slot_mapping", P, E),
                                 ("rotate", K, True)]),                                    # ops.py:730-740
    ("attn_paged_decode_cached", [("q", P, E), ("k_cache", P, E), ("k_scale", P, E), ("v_cache", P, E),
                                  ("v_scale", P, E), ("block_table", P, E), ("context_lens", P, E),
                                  ("block_size", P, E), ("max_context_len", K, None), ("scale", K, None),
                                  ("rotate", K, True), ("num_splits", K, None)]),          # ops.py:778-792
    ("attn_paged_decode_k8v3", [("q", P, E), ("k_cache", P, E), ("k_scale", P, E), ("v_packed", P, E),
                                ("v_norm", P, E), ("v_codebook", P, E), ("block_table", P, E),
                                ("context_lens", P, E), ("block_size", P, E), ("max_context_len", K, None),
                                ("scale", K, None), ("rotate", K, True), ("num_splits", K, None)]),  # ops.py:852-866
    ("quantize_kv_cache_3bit", [("k", P, E), ("v", P, E), ("rotate", K, True), ("fit", K, True),
                                ("block_size", K, 128)]),                                  # ops.py:590-597
    ("dequantize_kv_cache_3bit", [("packed", P, E), ("d", P, E)]),                         # ops.py:658
    ("quantize_i8_rowwise", [("x", P, E)]),                                                # ops.py:975
    ("linear_q4k", [("x", P, E), ("w_bytes", P, E), ("bias", K, None), ("out_dtype", K, "torch.float16")]),  # ops.py:1254-1260
    ("linear", [("x", P, E), ("qt", P, E), ("bias", K, None), ("out_dtype", K, "torch.float16")]),  # ops.py:2088-2094
]

# _C functions of this path (reference csrc/fni8_api.cpp m.def names)
REF_C = ["quantize_i8_rowwise", "attn_int8_fwd", "attn_int8_fwd_train", "attn_w8a8_fwd", "attn_int8_decode",
         "attn_int8_decode_kv8", "attn_paged_decode", "attn_paged_decode_k8v3", "kv_write_paged", "gemm_q4k", "gemm_decode_q4k",
         "gemm_q5k", "gemm_q6k", "gemm_decode_q5k", "gemm_decode_q6k"]


@pytest.fixture()
def aliased():
    alias.install(force=True)
    yield
    alias.uninstall()


def _norm(d):
    return "torch.float16" if str(d) == "torch.float16" else d


@pytest.mark.parametrize("name,params", REF_OPS, ids=[n for n, _ in REF_OPS])
def test_ops_signatures_match_reference(aliased, name, params):
    from superl8 import ops  # the reference's import path

    got = [(p.name, p.kind, _norm(p.default)) for p in inspect.signature(getattr(ops, name)).parameters.values()]
    assert got == [(n, k, _norm(d)) for n, k, d in params]


def test_reference_import_paths_resolve(aliased):
    import superl8
    from superl8 import _C, format, gguf, quant  # noqa: F401
    from superl8.ops import attn_decode_cached, attn_int8_decode, attn_int8_fwd  # noqa: F401
    from superl8.quant import quantize_qk, smooth_k  # noqa: F401
    from superl8.quant.lloydmax import pack_indices_lowbit, quantize_lloydmax  # noqa: F401
    from superl8.quant.rotation import rotate_last  # noqa: F401

    assert superl8.attn_int8_fwd is attn_int8_fwd
    for fn in REF_C:
        assert callable(getattr(_C, fn)), fn
    assert hasattr(format, "QTensor")


def test_uninstall_removes_only_this_package():
    import sys

    alias.install(force=True)
    assert sys.modules["superl8"].__name__ == "superl8_amd"
    alias.uninstall()
    assert "superl8" not in sys.modules and "superl8.ops" not in sys.modules

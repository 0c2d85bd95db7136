"""ctypes binding of libsuperl8_hip.so (the C ABI declared in include/superl8_hip.h).

torch is imported first on purpose: the library links libamdhip64.so.7 by
soname and so binds to the HIP runtime torch has already loaded, sharing its
device context and streams.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("SL8_LIB", _PKG / "libsuperl8_hip.so"))

F16, BF16, F32 = 0, 1, 2
_DT = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}

_P, _I64, _I, _F, _SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t

# symbol -> (restype, argtypes)
SIGNATURES = {
    "sl8_last_error": (ctypes.c_char_p, []),
    "sl8_version": (ctypes.c_char_p, []),
    "sl8_quantize_i8_rowwise": (_I, [_P, _I, _I64, _I64, _P, _P, _P]),
    "sl8_k_mean_workspace": (_SZ, [_I64, _I64]),
    "sl8_k_mean": (_I, [_P, _I, _I64, _I64, _I64, _P, _P, _SZ, _P]),
    "sl8_quantize_i8_rows_centered": (_I, [_P, _I, _I64, _I64, _I64, _P, _F, _P, _P, _P]),
    "sl8_quantize_i8_row_groups": (_I, [_P, _I, _I64, _I64, _I64, _I64, _P, _F, _P, _P, _P]),
    "sl8_quantize_qk_workspace": (_SZ, [_I64, _I64, _I64, _I64]),
    "sl8_quantize_qk": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64, _F, _F, _P, _P, _P, _P, _P, _P,
                             _P, _SZ, _P]),
    "sl8_quantize_i8_cols": (_I, [_P, _I, _I64, _I64, _I64, _P, _P, _P]),
    "sl8_attn_int8_fwd_workspace": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "sl8_attn_int8_fwd": (_I, [_P, _P, _P, _P, _P, _I, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                               _I, _I64, _P, _SZ, _P]),
    "sl8_attn_int8_fwd_gated": (_I, [_P, _P, _P, _P, _P, _I, _P, _P, _I64, _I64, _I64, _I64, _I64,
                                     _I64, _I, _I64, _P, _SZ, _P, _P]),
    "sl8_attn_int8_qk_scores": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P, _SZ, _P]),
    "sl8_attn_w8a8_fwd_workspace": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "sl8_attn_w8a8_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                               _I, _I64, _I, _P, _SZ, _P]),
    "sl8_choose_num_splits": (_I, [_I64, _I64, _I64]),
    "sl8_attn_int8_decode_workspace": (_SZ, [_I64, _I64, _I64, _I64]),
    "sl8_attn_int8_decode": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                                  _P, _SZ, _P]),
    "sl8_attn_int8_decode_ks16": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                                       _P, _SZ, _P]),
    "sl8_attn_int8_decode_noalloc_max_bytes": (_SZ, []),
    "sl8_attn_int8_decode_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                                          _I64, _P]),
    "sl8_attn_int8_decode_kv8": (_I, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                                      _I64, _P, _SZ, _P]),
    "sl8_paged_choose_num_splits": (_I, [_I64, _I64]),
    "sl8_q_outlier_gate": (_I, [_P, _I, _I64, _I64, ctypes.c_float, _P, _P, _P]),
    "sl8_attn_paged_decode": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                   _I64, _I64, _I64, _I64, _I64, _P, _SZ, _P]),
    "sl8_attn_paged_decode_k8v3": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64,
                                        _I64, _I64, _I64, _I64, _I64, _I64, _P, _SZ, _P]),
    "sl8_kv_write_paged": (_I, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P]),
    "sl8_gemm_decode_q4k": (_I, [_P, _P, _P, _P, _I, _I64, _I64, _I64, _P]),
    "sl8_gemm_decode_q4k_xblock": (_I, [_P, _P, _P, _P, _I, _I64, _I64, _I64, _P]),
    "sl8_gemm_q4k": (_I, [_P, _P, _P, _P, _I, _I64, _I64, _I64, _P]),
    "sl8_dequant_q4k": (_I, [_P, _P, _I64, _I64, _P]),
    "sl8_gemm_q5k": (_I, [_P, _P, _P, _P, _I, _I64, _I64, _I64, _P]),
    "sl8_gemm_q6k": (_I, [_P, _P, _P, _P, _I, _I64, _I64, _I64, _P]),
    "sl8_gemm_decode_q5k": (_I, [_P, _P, _P, _P, _I, _I64, _I64, _I64, _P]),
    "sl8_gemm_decode_q6k": (_I, [_P, _P, _P, _P, _I, _I64, _I64, _I64, _P]),
    "sl8_dequant_q5k": (_I, [_P, _P, _I64, _I64, _P]),
    "sl8_dequant_q6k": (_I, [_P, _P, _I64, _I64, _P]),
}

_lib = None


def load(path: Path | None = None) -> ctypes.CDLL:
    """Load (once) and return the library; raise RuntimeError if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path or LIB_PATH)
    if not p.exists():
        raise RuntimeError(
            f"superl8 HIP library not found at {p}; build it with "
            f"`python -m superl8_amd.build` (hipcc, gfx950)"
        )
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError:
            continue
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def call(name: str, *args) -> int:
    lib = load()
    fn = getattr(lib, name, None)
    if fn is None or fn.argtypes is None:
        raise RuntimeError(f"{name} is not exported by {LIB_PATH}")
    rc = fn(*args)
    if isinstance(rc, int) and rc != 0 and SIGNATURES[name][0] is _I:
        raise RuntimeError(lib.sl8_last_error().decode())
    return rc


def dtype_code(dt: torch.dtype) -> int:
    return _DT[dt]


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream

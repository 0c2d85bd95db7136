"""Quantisation prologue (reference superl8/quant/__init__.py, hot-path subset)."""
from .core import (
    LOG2E,
    dequantize_int8_rowwise,
    detect_q_outlier_domination,
    quantize_int8_rowwise,
    quantize_qk,
    quantize_qk_gated,
    quantize_qk_per_wave,
    quantize_v_perchannel,
    quantize_v_rowwise,
    smooth_k,
)
from .lloydmax import (
    dequantize_lloydmax,
    fake_quant_lloydmax,
    gaussian_codebook,
    lloyd_max_fit,
    pack_indices_lowbit,
    quantize_lloydmax,
    unpack_indices_lowbit,
)
from .rotation import hadamard_matrix, rotate_last

__all__ = [
    "LOG2E", "dequantize_int8_rowwise", "detect_q_outlier_domination", "hadamard_matrix",
    "quantize_int8_rowwise", "quantize_qk", "quantize_qk_gated", "quantize_qk_per_wave", "quantize_v_perchannel", "quantize_v_rowwise",
    "rotate_last", "smooth_k",
    "dequantize_lloydmax", "fake_quant_lloydmax", "gaussian_codebook", "lloyd_max_fit",
    "pack_indices_lowbit", "quantize_lloydmax", "unpack_indices_lowbit",
]

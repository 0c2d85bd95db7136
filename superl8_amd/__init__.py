"""superl8 INT8 attention + GGUF k-quant linear hot path, MI355X (gfx950) native.

Drop-in for the reference package's hot-path surface: `ops` (attn_int8_fwd,
attn_int8_decode, quantize_kv_cache, attn_decode_cached, quantize_kv_write_paged,
attn_paged_decode_cached, attn_paged_decode_k8v3, quantize_kv_write_paged_k8v3,
quantize_kv_cache_3bit, dequantize_kv_cache_3bit, quantize_i8_rowwise, linear, linear_q4k, linear_q5k,
linear_q6k), `quant`, `format` (QTensor), `gguf` (the GGUF reader feeding
native k-quant bytes) and `_C` (the operator surface of the compiled extension,
here a C-ABI library).
"""
from . import _C  # noqa: F401
from .ops import (attn_decode_cached, attn_int8_decode, attn_int8_fwd, attn_paged_decode_cached,
                  attn_paged_decode_k8v3, dequantize_kv_cache_3bit, quantize_kv_cache_3bit,
                  quantize_kv_write_paged_k8v3, linear, linear_q4k, linear_q5k, linear_q6k, quantize_i8_rowwise, quantize_kv_cache,
                  quantize_kv_write_paged)

__all__ = ["attn_decode_cached", "attn_int8_decode", "attn_int8_fwd", "attn_paged_decode_cached",
           "attn_paged_decode_k8v3", "dequantize_kv_cache_3bit", "quantize_kv_cache_3bit",
           "quantize_kv_write_paged_k8v3",
           "linear", "linear_q4k", "linear_q5k", "linear_q6k", "quantize_i8_rowwise", "quantize_kv_cache",
           "quantize_kv_write_paged", "_C"]

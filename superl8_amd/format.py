"""Weight container of the k-quant linear path (reference superl8/format.py:209-300).

Only the schemes this hot path serves: ``gguf_kquant`` (native GGUF k-quant
bytes kept resident, byte-identical to the file; the sub-block scales live
inside the bytes) for the Q4_K / Q5_K / Q6_K kernels, and ``raw`` (a float
tensor stored as is).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

# Bytes per 256-weight super-block of the k-quant types served natively
# (reference format.py:209-214, the GGUF block sizes).
GGUF_KQUANT_BLOCK = {"q4_k": 144, "q5_k": 176, "q6_k": 210}
QK_K = 256


@dataclass
class QTensor:
    """A stored weight: ``data`` plus how to read it.

    ``gguf_kquant``: uint8 ``data`` [out, (in/256) * type_size], ``codebook`` the
    GGML type tag ('q4_k' / 'q5_k' / 'q6_k'), ``group_size`` 256.
    ``raw``: ``data`` used as is (norms, embeddings, float weights).
    """
    data: torch.Tensor
    scale: torch.Tensor | None = None
    scheme: str = "gguf_kquant"
    group_size: int = 0
    codebook: str = ""

    def validate(self) -> None:
        if self.scheme == "gguf_kquant":
            assert self.data.dtype == torch.uint8 and self.data.dim() == 2, \
                "gguf_kquant needs uint8 data [out, n_superblocks * type_size]"
            assert self.codebook in GGUF_KQUANT_BLOCK, (
                f"gguf_kquant type tag {self.codebook!r} "
                f"(expect one of {', '.join(sorted(GGUF_KQUANT_BLOCK))})")
            assert self.group_size == QK_K, f"gguf_kquant group_size must be {QK_K}"
            assert self.data.shape[-1] % GGUF_KQUANT_BLOCK[self.codebook] == 0, \
                f"{self.codebook} row bytes must be a multiple of {GGUF_KQUANT_BLOCK[self.codebook]}"
        elif self.scheme == "raw":
            pass
        else:
            raise AssertionError(f"unsupported scheme {self.scheme!r} on this path")

    @property
    def in_features(self) -> int:
        if self.scheme == "gguf_kquant":
            return self.data.shape[-1] // GGUF_KQUANT_BLOCK[self.codebook] * QK_K
        return self.data.shape[-1]

    @property
    def out_features(self) -> int:
        return self.data.shape[0]

"""Normalised Sylvester-Hadamard rotation of the head dim (reference
superl8/quant/rotation.py:28-51). Q.K^T is invariant under a shared orthogonal
rotation; rotating spreads channel outliers before int8 quantisation."""
import functools

import torch


@functools.lru_cache(maxsize=8)
def hadamard_matrix(d: int, device: str = "cpu", dtype: torch.dtype = torch.float32):
    """Normalised Sylvester-Hadamard M [d, d] (M @ M.T == I); d a power of two."""
    if d <= 0 or d & (d - 1):
        raise ValueError(f"Hadamard needs a power-of-two dim, got {d}")
    h = torch.ones(1, 1, dtype=torch.float32)
    while h.shape[0] < d:
        h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
    return (h / (d ** 0.5)).to(device=device, dtype=dtype)


def rotate_last(x: torch.Tensor) -> torch.Tensor:
    """x @ M over the last dim, in fp32, cast back to x's dtype."""
    m = hadamard_matrix(x.shape[-1], device=str(x.device), dtype=torch.float32)
    return (x.float() @ m).to(x.dtype)

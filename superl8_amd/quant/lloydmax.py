"""3-bit Lloyd-Max storage codec of the rotated KV cache (reference
superl8/quant/lloydmax.py:1-219): the V side of the K8V3 paged store that
`attn_paged_decode_k8v3` reads.

Format (per row, head dim D split into blocks of `block_size` channels):
  norm  = ||x_block||_2 (fp32; a zero block stores 1)
  code  = index of the nearest codebook level to x / norm, ties to the lower
          level (a value equal to a decision boundary takes the lower index)
  value = codebook[code] * norm
The default codebook is the 8-level MSE-optimal quantiser of a unit Gaussian
(Max, 1960) scaled by block_size^-1/2, the spread of one coordinate of a
rotated unit-norm block. Codes are packed LSB-first into int32 words: code i
of a row occupies bits 3i..3i+2 of the row's bit stream (so D*3 must be a
multiple of 32).

These are tensor-format helpers in torch (they run on the tensor's device);
the decode kernel consumes the packed store directly.
"""
from __future__ import annotations

import functools

import torch

# Reproduction levels of the 8-level Lloyd-Max quantiser for N(0, 1)
# (J. Max, "Quantizing for minimum distortion", IRE Trans. IT-6, 1960, table I),
# ascending; the reference stores the same six-digit values
# (superl8/quant/lloydmax.py:44-47).
STDNORMAL_LM8 = (-2.152135, -1.343909, -0.756096, -0.245098,
                 0.245098, 0.756096, 1.343909, 2.152135)


def lloydmax_bits_levels(bits: int) -> int:
    """Levels of a `bits`-bit code (reference lloydmax.py:50-53)."""
    if not 2 <= bits <= 8:
        raise AssertionError(f"bits must be in [2, 8], got {bits}")
    return 1 << bits


@functools.lru_cache(maxsize=16)
def gaussian_codebook(bits: int, block_size: int, device: str = "cpu") -> torch.Tensor:
    """Fixed codebook for unit-norm blocks of `block_size` channels: the N(0,1)
    levels times block_size^-1/2, each product formed in double precision and
    stored as fp32 (reference lloydmax.py:56-65)."""
    if bits != 3:
        raise AssertionError("the fixed Gaussian codebook is defined for 3 bits; fit one otherwise")
    sigma = block_size ** -0.5
    return torch.tensor([c * sigma for c in STDNORMAL_LM8], dtype=torch.float32, device=device)


def lloyd_max_fit(samples: torch.Tensor, levels: int, *, iters: int = 40,
                  tol: float = 1e-6) -> torch.Tensor:
    """MSE-optimal `levels` reproduction levels of the 1-D sample set (reference
    lloydmax.py:68-108): start at the sample quantiles (l + 1/2) / levels, then
    alternate nearest-level assignment and conditional means until no level moves
    by `tol`; an empty cell keeps its starting quantile. Runs in float64 on the
    CPU (fixed reduction order, so the fit is deterministic); returns fp32
    ascending levels on the samples' device."""
    x = samples.detach().flatten().double().cpu()
    if x.numel() == 0:
        return torch.zeros(levels, dtype=torch.float32, device=samples.device)
    n = x.numel()
    start = torch.quantile(x, torch.linspace(0.5 / levels, 1.0 - 0.5 / levels, levels,
                                             dtype=torch.float64))
    xs = torch.sort(x).values
    prefix = torch.cat([xs.new_zeros(1), torch.cumsum(xs, 0)])
    c, prev = start.clone(), None
    for _ in range(iters):
        cut = torch.searchsorted(xs, 0.5 * (c[1:] + c[:-1]), right=True)
        edges = torch.cat([cut.new_zeros(1), cut, cut.new_full((1,), n)])
        cnt = (edges[1:] - edges[:-1]).double()
        tot = prefix[edges[1:]] - prefix[edges[:-1]]
        nxt = torch.sort(torch.where(cnt > 0, tot / cnt.clamp_min(1.0), start)).values
        if prev is not None and (nxt - prev).abs().max() < tol:
            c = nxt
            break
        prev, c = c, nxt
    return c.to(device=samples.device, dtype=torch.float32)


def _blocks(x: torch.Tensor, block_size: int, dim: int):
    xf = x.float().movedim(dim, -1)
    d = xf.shape[-1]
    if d % block_size:
        raise AssertionError(f"last dim {d} not divisible by block_size {block_size}")
    return xf.reshape(*xf.shape[:-1], d // block_size, block_size), xf.shape


def quantize_lloydmax(x: torch.Tensor, *, bits: int = 3, block_size: int = 128, dim: int = -1,
                      codebook: torch.Tensor | None = None):
    """-> (codes uint8 [x.shape], norm fp32 [x.shape with dim -> dim // block_size],
    codebook fp32 [2^bits]) (reference lloydmax.py:118-145)."""
    lloydmax_bits_levels(bits)
    xb, flat_shape = _blocks(x, block_size, dim)
    norm = torch.sqrt((xb * xb).sum(-1, keepdim=True))
    norm = torch.where(norm == 0, torch.ones_like(norm), norm)
    unit = xb / norm
    cb = (gaussian_codebook(bits, block_size, x.device.type) if codebook is None
          else codebook.to(device=x.device, dtype=torch.float32))
    bounds = 0.5 * (cb[1:] + cb[:-1])
    codes = torch.bucketize(unit.reshape(*unit.shape[:-2], -1).contiguous(), bounds)
    codes = codes.reshape(flat_shape).movedim(-1, dim).to(torch.uint8)
    return codes, norm.squeeze(-1).movedim(-1, dim).float(), cb


def dequantize_lloydmax(codes: torch.Tensor, norm: torch.Tensor, codebook: torch.Tensor, *,
                        block_size: int = 128, dim: int = -1) -> torch.Tensor:
    """codebook[code] * norm of the code's block, fp32 (reference lloydmax.py:148-164)."""
    cb = codebook.to(device=codes.device, dtype=torch.float32)
    c = codes.long().movedim(dim, -1)
    nb = c.shape[-1] // block_size
    vals = cb[c].reshape(*c.shape[:-1], nb, block_size)
    nrm = norm.movedim(dim, -1).float().reshape(*c.shape[:-1], nb, 1)
    return (vals * nrm).reshape(c.shape).movedim(-1, dim)


def fake_quant_lloydmax(x: torch.Tensor, *, bits: int = 3, block_size: int = 128, dim: int = -1,
                        fit: bool = False, fit_iters: int = 40) -> torch.Tensor:
    """Quantise then dequantise in x's dtype; `fit` fits the codebook to the
    unit-normalised blocks of x first (reference lloydmax.py:167-193)."""
    codebook = None
    if fit:
        xb, _ = _blocks(x, block_size, dim)
        norm = torch.sqrt((xb * xb).sum(-1, keepdim=True))
        codebook = lloyd_max_fit(xb / torch.where(norm == 0, torch.ones_like(norm), norm),
                                 lloydmax_bits_levels(bits), iters=fit_iters)
    codes, norm, cb = quantize_lloydmax(x, bits=bits, block_size=block_size, dim=dim,
                                        codebook=codebook)
    return dequantize_lloydmax(codes, norm, cb, block_size=block_size, dim=dim).to(x.dtype)


def pack_indices_lowbit(indices: torch.Tensor, bits: int) -> torch.Tensor:
    """Unsigned `bits`-bit codes along the last dim -> int32 words, LSB-first
    (reference lloydmax.py:203-212); needs last_dim * bits % 32 == 0."""
    d = indices.shape[-1]
    if (d * bits) % 32:
        raise AssertionError(f"D*bits ({d}*{bits}) must be a multiple of 32")
    u = indices.to(torch.int64) & ((1 << bits) - 1)
    shifts = torch.arange(bits, device=indices.device)
    stream = ((u.unsqueeze(-1) >> shifts) & 1).reshape(*indices.shape[:-1], -1, 32)
    weights = torch.ones(32, dtype=torch.int64, device=indices.device) << torch.arange(
        32, device=indices.device)
    words = (stream * weights).sum(-1)
    return torch.where(words >= (1 << 31), words - (1 << 32), words).to(torch.int32)


def unpack_indices_lowbit(packed: torch.Tensor, bits: int, d: int) -> torch.Tensor:
    """Inverse of pack_indices_lowbit -> uint8 codes [..., d] (reference lloydmax.py:215-219)."""
    w = packed.to(torch.int64) & 0xFFFFFFFF
    stream = (w.unsqueeze(-1) >> torch.arange(32, device=packed.device)) & 1
    stream = stream.reshape(*packed.shape[:-1], d, bits)
    return (stream << torch.arange(bits, device=packed.device)).sum(-1).to(torch.uint8)

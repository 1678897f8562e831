"""TurboQuant MSE quantizer on HIP kernels.

Drop-in for leankv/turboquant/quantizer.py:
  MSEQuantized(indices, norms, bits)            (:22-27)
  _pack_indices / _unpack_indices               (:38-85) -- torch helpers, same layout
  TurboQuantMSE(dim, bits, device, dtype, seed) (:88-141)
      quantize(x)   -> one fused HIP launch: norm, x / (norm + 1e-10),
                       fp32-MFMA rotation, searchsorted, bit-pack
      dequantize(q) -> one HIP launch: unpack, centroid gather, rotation back, x norm
The inner-product variant TurboQuantProd (:144-237) is not part of this build
(no cache or decode path uses it).
"""

from __future__ import annotations

from typing import NamedTuple

import torch
import torch.nn.functional as F

from .. import kernels as _k
from .codebook import get_codebook_tensors
from .rotation import generate_rotation_matrix


class MSEQuantized(NamedTuple):
    indices: torch.Tensor  # (..., packed_len) uint8 bit-packed
    norms: torch.Tensor    # (...,) L2 norms, dtype of the quantized input
    bits: int


def _layout(bits: int) -> tuple[int, int]:
    if bits == 1:
        return 8, 1
    if bits == 2:
        return 4, 2
    if bits <= 4:
        return 2, 4
    return 1, 8


def _pack_indices(indices: torch.Tensor, bits: int) -> torch.Tensor:
    """Codes 0..2^bits-1 -> uint8; field i of a byte sits at bit i*width (3 bits use 4)."""
    if bits > 4:
        return indices.to(torch.uint8)
    vpb, width = _layout(bits)
    d = indices.shape[-1]
    pad = (-d) % vpb
    idx = indices.to(torch.uint8)
    if pad:
        idx = F.pad(idx, (0, pad), value=0)
    r = idx.reshape(*indices.shape[:-1], -1, vpb)
    shifts = torch.arange(vpb, device=indices.device, dtype=torch.uint8) * width
    return (r << shifts).sum(dim=-1, dtype=torch.uint8)


def _unpack_indices(packed: torch.Tensor, bits: int, d: int) -> torch.Tensor:
    if bits > 4:
        return packed.long()
    vpb, width = _layout(bits)
    shifts = torch.arange(vpb, device=packed.device, dtype=torch.uint8) * width
    u = (packed.unsqueeze(-1) >> shifts) & ((1 << width) - 1)
    return u.reshape(*packed.shape[:-1], -1)[..., :d].long()


class TurboQuantMSE(torch.nn.Module):
    """y = Pi (x / ||x||); per-coordinate nearest Lloyd-Max centroid; bit-packed codes."""

    def __init__(self, dim: int, bits: int = 3, device=None, dtype: torch.dtype = torch.float32, seed: int = 42):
        super().__init__()
        if dim != _k.HEAD_DIM:
            raise ValueError("TurboQuantMSE: the HIP kernels are built for dim %d, got %d" % (_k.HEAD_DIM, dim))
        if not 1 <= bits <= 4:
            raise ValueError("TurboQuantMSE: bits must be 1..4 (bit-packed codes), got %d" % bits)
        self.dim, self.bits, self.n_clusters = dim, bits, 2 ** bits
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.register_buffer("Pi", generate_rotation_matrix(dim, self.device, dtype, seed=seed))
        c, b = get_codebook_tensors(dim, bits, self.device, dtype)
        self.register_buffer("centroids", c)
        self.register_buffer("boundaries", b)
        self.register_buffer("decision_boundaries", b[1:-1].contiguous())

    def quantize(self, x: torch.Tensor) -> MSEQuantized:
        packed, norms = _k.tq_quantize(x, self.Pi, self.decision_boundaries, self.bits)
        return MSEQuantized(indices=packed, norms=norms, bits=self.bits)

    def dequantize(self, q: MSEQuantized) -> torch.Tensor:
        return _k.tq_dequantize(q.indices, q.norms, self.Pi, self.centroids, q.bits, out_dtype=torch.float32)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.dequantize(self.quantize(x))

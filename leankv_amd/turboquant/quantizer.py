"""TurboQuant MSE quantizer on HIP kernels.

Drop-in for leankv/turboquant/quantizer.py:
  MSEQuantized(indices, norms, bits)            (:22-27)
  _pack_indices / _unpack_indices               (:38-85) -- torch helpers, same layout
  TurboQuantMSE(dim, bits, device, dtype, seed) (:88-141)
      quantize(x)   -> one fused HIP launch: norm, x / (norm + 1e-10),
                       fp32-MFMA rotation, searchsorted, bit-pack
      dequantize(q) -> one HIP launch: unpack, centroid gather, rotation back, x norm
  ProdQuantized(mse_indices, qjl_signs, residual_norms, norms, mse_bits)  (:29-35)
  TurboQuantProd(dim, bits, device, dtype, seed)  (:144-237) -- MSE at bits - 1
      plus a 1-bit QJL sketch of the residual (sign(r @ S^T), S ~ N(0, 1) with seed
      + 1000) and ||r||, an unbiased inner-product estimator:
      quantize(x)   -> one fused HIP launch (three fp32-MFMA products per vector)
      dequantize(q) -> one HIP launch: x_mse + (signs @ S) * (sqrt(pi/2)/d * ||r||)
"""

from __future__ import annotations

import math
from typing import NamedTuple

import torch
import torch.nn.functional as F

from .. import kernels as _k  # registers torch.ops.leankv
from .codebook import get_codebook_tensors
from .rotation import generate_qjl_matrix, generate_rotation_matrix


class MSEQuantized(NamedTuple):
    indices: torch.Tensor  # (..., packed_len) uint8 bit-packed
    norms: torch.Tensor    # (...,) L2 norms, dtype of the quantized input
    bits: int


class ProdQuantized(NamedTuple):
    mse_indices: torch.Tensor     # (..., packed_len) uint8 bit-packed, mse_bits per code
    qjl_signs: torch.Tensor       # (..., d / 8) uint8, bit i of byte j = sign of coordinate 8j + i
    residual_norms: torch.Tensor  # (...,) fp32 ||x - x_mse||
    norms: torch.Tensor           # (...,) L2 norms, dtype of the quantized input
    mse_bits: int


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
        packed, norms = torch.ops.leankv.tq_quantize(x, self.Pi, self.decision_boundaries, self.bits)
        return MSEQuantized(indices=packed, norms=norms, bits=self.bits)

    def dequantize(self, q: MSEQuantized) -> torch.Tensor:
        return torch.ops.leankv.tq_dequantize(q.indices, q.norms, self.Pi, self.centroids, q.bits, torch.float32)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.dequantize(self.quantize(x))


class TurboQuantProd(torch.nn.Module):
    """TurboQuant for inner products: TurboQuantMSE at bits - 1 on x, then 1-bit QJL on the residual.

    Signs of S r (S i.i.d. N(0, 1), seed + 1000) and ||r|| give the unbiased
    estimate <y, x> ~ <y, x_mse> + sqrt(pi/2)/d * ||r|| <S y, sign(S r)>.
    """

    def __init__(self, dim: int, bits: int = 3, device=None, dtype: torch.dtype = torch.float32, seed: int = 42):
        super().__init__()
        if bits < 2:
            raise AssertionError("Inner product TurboQuant requires at least 2 bits (1 for MSE + 1 for QJL)")
        self.dim, self.bits = dim, bits
        self.mse_quantizer = TurboQuantMSE(dim=dim, bits=bits - 1, device=device, dtype=dtype, seed=seed)
        self.device = self.mse_quantizer.device
        self.register_buffer("S", generate_qjl_matrix(dim, self.device, dtype, seed=seed + 1000))
        self.qjl_scale = math.sqrt(math.pi / 2.0) / dim

    def _pack_qjl_signs(self, projected: torch.Tensor) -> torch.Tensor:
        """Sign bits of `projected` (> 0 -> 1), 8 per byte, coordinate 8j + i at bit i of byte j."""
        signs = (projected > 0).to(torch.uint8)
        d = signs.shape[-1]
        if d % 8:
            signs = F.pad(signs, (0, 8 - d % 8), value=0)
        r = signs.reshape(*signs.shape[:-1], -1, 8)
        shifts = torch.arange(8, device=signs.device, dtype=torch.uint8)
        return (r << shifts).sum(dim=-1, dtype=torch.uint8)

    def _unpack_qjl_signs(self, packed: torch.Tensor) -> torch.Tensor:
        """Packed sign bytes -> float +1 / -1 per coordinate."""
        shifts = torch.arange(8, device=packed.device, dtype=torch.uint8)
        bits = ((packed.unsqueeze(-1) >> shifts) & 1).float()
        return 2.0 * bits.reshape(*packed.shape[:-1], -1)[..., : self.dim] - 1.0

    def quantize(self, x: torch.Tensor) -> ProdQuantized:
        m = self.mse_quantizer
        codes, norms, signs, rnorms = _k.tq_prod_quantize(x, m.Pi, m.decision_boundaries, m.centroids, self.S,
                                                          m.bits)
        return ProdQuantized(mse_indices=codes, qjl_signs=signs, residual_norms=rnorms, norms=norms,
                             mse_bits=m.bits)

    def dequantize(self, q: ProdQuantized) -> torch.Tensor:
        m = self.mse_quantizer
        return _k.tq_prod_dequantize(q.mse_indices, q.norms, q.qjl_signs, q.residual_norms, m.Pi, m.centroids,
                                     self.S, q.mse_bits, self.qjl_scale)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.dequantize(self.quantize(x))

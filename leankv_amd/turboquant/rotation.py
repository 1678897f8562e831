"""Random rotation for TurboQuant.

Drop-in for leankv/turboquant/rotation.py:
  generate_rotation_matrix(d, device, dtype, seed)  (:12-29) -- host side:
      seeded CPU torch.randn(d, d), QR, columns sign-fixed by sign(diag R) so the
      factorisation is unique; the same seed gives the same matrix as the reference.
  generate_qjl_matrix(d, device, dtype, seed)       (:32-42)
  rotate_forward(x, Pi) = x @ Pi^T, rotate_backward(y, Pi) = y @ Pi  (:45-52)
      -- on the GPU through the fp32-MFMA HIP kernel (head_dim 128).
"""

from __future__ import annotations

import torch

from .. import kernels as _k


def generate_rotation_matrix(d: int, device=None, dtype: torch.dtype = torch.float32, seed: int = 42) -> torch.Tensor:
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    G = torch.randn(d, d, generator=gen, dtype=torch.float32)
    Q, R = torch.linalg.qr(G)
    Q = Q * torch.sign(torch.diag(R)).unsqueeze(0)
    # LAPACK hands Q back column-major; the kernels take row-major pointers.
    return Q.to(device=device, dtype=dtype).contiguous()


def generate_qjl_matrix(d: int, device=None, dtype: torch.dtype = torch.float32, seed: int = 12345) -> torch.Tensor:
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    return torch.randn(d, d, generator=gen, dtype=torch.float32).to(device=device, dtype=dtype)


def rotate_forward(x: torch.Tensor, Pi: torch.Tensor) -> torch.Tensor:
    """y = x @ Pi^T (fp32 out), HIP fp32 MFMA."""
    return _k.tq_rotate(x, Pi, transpose=False)


def rotate_backward(y: torch.Tensor, Pi: torch.Tensor) -> torch.Tensor:
    """x = y @ Pi (fp32 out), HIP fp32 MFMA."""
    return _k.tq_rotate(y, Pi, transpose=True)

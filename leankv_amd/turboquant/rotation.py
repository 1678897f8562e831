"""Random rotation for TurboQuant.

Drop-in for leankv/turboquant/rotation.py:
  generate_rotation_matrix(d, device, dtype, seed)  (:12-29) -- host side:
      seeded CPU torch.randn(d, d), QR, columns sign-fixed by sign(diag R) so the
      factorisation is unique; the same seed gives the same matrix as the reference.
      Each (d, seed) is factorised once per process and handed out as copies.
  generate_qjl_matrix(d, device, dtype, seed)       (:32-42)
  rotate_forward(x, Pi) = x @ Pi^T, rotate_backward(y, Pi) = y @ Pi  (:45-52)
      -- on the GPU through the fp32-MFMA HIP kernel (head_dim 128).
"""

from __future__ import annotations

import functools

import torch

from .. import kernels as _k


@functools.lru_cache(maxsize=4096)
def _rotation_cpu(d: int, seed: int) -> torch.Tensor:
    """The fp32 CPU matrix of (d, seed), computed once per process (a 128 x 128 QR
    takes ~0.7 ms, and a cache of 32 layers asks for 64 of them).  Callers get copies."""
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    G = torch.randn(d, d, generator=gen, dtype=torch.float32)
    Q, R = torch.linalg.qr(G)
    Q = Q * torch.sign(torch.diag(R)).unsqueeze(0)
    # LAPACK hands Q back column-major; the kernels take row-major pointers.
    return Q.contiguous()


def generate_rotation_matrix(d: int, device=None, dtype: torch.dtype = torch.float32, seed: int = 42) -> torch.Tensor:
    return _rotation_cpu(int(d), int(seed)).to(device=device, dtype=dtype, copy=True)


def generate_rotation_matrices(d: int, seeds, device=None, dtype: torch.dtype = torch.float32) -> list:
    """[generate_rotation_matrix(d, device, dtype, s) for s in seeds], moved to the device in one copy:
    the matrices are row-major [d, d] slices of one [len(seeds), d, d] tensor."""
    seeds = [int(s) for s in seeds]
    if not seeds:
        return []
    allm = torch.stack([_rotation_cpu(int(d), s) for s in seeds]).to(device=device, dtype=dtype)
    return list(allm.unbind(0))


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

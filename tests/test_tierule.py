"""CPU self-check of the quantize tie rule (tests/tierule.py) that the GPU parity tests apply: it accepts a
second correct fp32 evaluation of y = u Pi^T (another summation order) and rejects plausible mistakes
(transposed rotation, a dropped term, a shifted boundary) planted in the oracle."""

import numpy as np
import pytest
import torch

from oracle import turboquant as oq
from tierule import _codes_match, _rotation_fp64


def _inputs():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(8192, 128, generator=g)
    x[:, [0, 31, 64, 127]] *= 10
    return x, oq.rotation_matrix(128, 42), oq.codebook_tensors(3)[1]


def _codes_from_y(y, b):
    return oq.pack_indices(torch.searchsorted(b[1:-1].contiguous(), torch.as_tensor(y).contiguous()).numpy(), 3)


def _sequential_fp32(u, P, order):
    acc = np.zeros((u.shape[0], P.shape[0]), dtype=np.float32)
    for k in order:
        acc = (acc + (u[:, k:k + 1] * P[None, :, k])).astype(np.float32)
    return acc


def test_tie_rule_accepts_another_fp32_summation_order():
    x, Pi, b = _inputs()
    p_ref, n, _ = oq.quantize(x, Pi, b, 3)
    u = (x / (n.unsqueeze(-1) + 1e-10)).numpy().astype(np.float32)
    y_alt = _sequential_fp32(u, Pi.numpy().astype(np.float32), range(127, -1, -1))
    y64, S = _rotation_fp64(x, Pi)
    flips = _codes_match(_codes_from_y(y_alt, b), p_ref, y64, S, b, 3)
    assert flips <= 8  # 1M coordinates: a handful of exact ties at most


@pytest.mark.parametrize("mistake", ["transposed_pi", "dropped_term", "shifted_boundary"])
def test_tie_rule_rejects_planted_mistakes(mistake):
    x, Pi, b = _inputs()
    p_ref, n, _ = oq.quantize(x, Pi, b, 3)
    u = (x / (n.unsqueeze(-1) + 1e-10)).float()
    if mistake == "transposed_pi":
        y_bad = torch.matmul(u, Pi)
    elif mistake == "dropped_term":
        y_bad = torch.matmul(u[:, :127], Pi.T[:127])
    else:
        y_bad = torch.matmul(u, Pi.T) + 1e-3  # a boundary off by a small constant
    y64, S = _rotation_fp64(x, Pi)
    with pytest.raises(AssertionError):
        _codes_match(_codes_from_y(y_bad, b), p_ref, y64, S, b, 3)

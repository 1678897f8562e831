"""Magnitude-threshold sparsification primitives (host side).

Mirrors leankv/teal/sparse_fns.py: SparsifyFn (:13-44) zeroes |x| <= t and
records the observed sparsity; compute_threshold_for_sparsity (:47-69) picks the
k-th smallest magnitude, k = int(s * n); compute_threshold_from_histogram
(:72-103) interpolates a histogram CDF.  These are torch ops used for the
hook-based correctness mode and for threshold selection; the decode hot path
never calls them (the HIP kernels fuse the threshold test).
"""

from __future__ import annotations

import torch


class SparsifyFn:
    """Zero activations with |x| <= threshold (strict '>' keeps), track sparsity."""

    def __init__(self, threshold: float = 0.0, enabled: bool = True):
        self.threshold = threshold
        self.enabled = enabled
        self._last_sparsity = 0.0

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if not self.enabled or self.threshold <= 0:
            return x
        keep = x.abs() > self.threshold
        self._last_sparsity = 1.0 - keep.float().mean().item()
        return x * keep

    @property
    def last_sparsity(self) -> float:
        return self._last_sparsity


def compute_threshold_for_sparsity(activations: torch.Tensor, target_sparsity: float) -> float:
    """Threshold t such that about target_sparsity of |activations| are <= t."""
    mags = activations.abs().flatten()
    k = int(target_sparsity * mags.numel())
    if k <= 0:
        return 0.0
    if k >= mags.numel():
        return mags.max().item()
    return torch.kthvalue(mags, k).values.item()


def compute_threshold_from_histogram(hist_counts: torch.Tensor, hist_edges: torch.Tensor,
                                     target_sparsity: float) -> float:
    """Threshold from a magnitude histogram by linear interpolation inside the CDF bin."""
    cdf = hist_counts.cumsum(0).float()
    cdf = cdf / cdf[-1]
    i = min(torch.searchsorted(cdf, target_sparsity).item(), len(hist_edges) - 2)
    if i > 0:
        frac = (target_sparsity - cdf[i - 1]) / (cdf[i] - cdf[i - 1] + 1e-10)
        t = hist_edges[i] + frac * (hist_edges[i + 1] - hist_edges[i])
    else:
        t = hist_edges[i]
    return t.item()

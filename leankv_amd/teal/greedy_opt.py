"""Block-wise greedy allocation of a global TEAL sparsity budget over projections (host side).

Drop-in for leankv/teal/greedy_opt.py (TEAL Algorithm 1): starting from zero
sparsity everywhere, each step raises the sparsity of the one (layer,
projection) whose next `step_size` increment prunes the least estimated L2
mass per parameter weight, until the parameter-weighted global sparsity reaches
the target; the chosen sparsities become thresholds through the activation
histograms.  Same inputs, outputs, step rule, 95 % cap and tie order (first
key in layer-major, PROJ_NAMES order wins) as greedy_opt.py:47-164; the band
error is the same fp32 sequential sum over histogram bins
(greedy_opt.py:167-197).  The only change is bookkeeping: a projection's
candidate error depends only on its own sparsity, so it is recomputed for the
projection that moved instead of for all of them on every step.
"""

from __future__ import annotations

from typing import Optional

import torch

from .calibrate import load_thresholds, save_thresholds  # noqa: F401  (the reference module exports both)
from .patching import PROJ_NAMES
from .sparse_fns import compute_threshold_from_histogram

# Relative parameter counts per projection type (greedy_opt.py:33-41).
_DEFAULT_PARAM_WEIGHTS = {
    "q_proj": 1.0,
    "k_proj": 0.25,
    "v_proj": 0.25,
    "o_proj": 1.0,
    "gate_proj": 3.5,
    "up_proj": 3.5,
    "down_proj": 3.5,
}

_CAP = 0.95  # greedy_opt.py:99


def _estimate_pruning_error(hist_data: dict, old_sparsity: float, new_sparsity: float) -> float:
    """Sum of (bin centre)^2 x count over the bins between the old and new sparsity levels of the CDF,
    accumulated in fp32 bin by bin (greedy_opt.py:167-197)."""
    counts = hist_data["counts"].float()
    edges = hist_data["edges"]
    total = counts.sum()
    if total == 0:
        return 0.0
    cdf = counts.cumsum(0) / total
    n = len(counts)
    lo = min(torch.searchsorted(cdf, old_sparsity).item(), n - 1)
    hi = min(torch.searchsorted(cdf, new_sparsity).item(), n - 1)
    error = 0.0
    for b in range(lo, hi + 1):
        centre = (edges[b] + edges[b + 1]) / 2.0
        error += (centre ** 2) * counts[b].item()
    return error


def greedy_optimize(histograms: dict, target_sparsity: float, num_layers: int,
                    param_weights: Optional[dict] = None, step_size: float = 0.05) -> dict:
    """{(layer, proj): {counts, edges}} histograms -> {layer: {proj: threshold}} (greedy_opt.py:47-164)."""
    if param_weights is None:
        param_weights = _DEFAULT_PARAM_WEIGHTS
    total_weight = sum(param_weights[p] for p in PROJ_NAMES) * num_layers
    level = {li: {p: 0.0 for p in PROJ_NAMES} for li in range(num_layers)}
    keys = [(li, p) for li in range(num_layers) for p in PROJ_NAMES if (li, p) in histograms]

    def candidate(key):
        cur = level[key[0]][key[1]]
        new = min(cur + step_size, _CAP)
        if new <= cur:
            return None
        err = _estimate_pruning_error(histograms[key], cur, new)
        return err / (param_weights[key[1]] + 1e-10), new

    cand = {k: candidate(k) for k in keys}
    current = 0.0
    while current < target_sparsity:
        best_key, best_err, best_new = None, float("inf"), 0.0
        for k in keys:  # layer-major, PROJ_NAMES order: the first of equal errors wins
            c = cand[k]
            if c is not None and c[0] < best_err:
                best_err, best_key, best_new = c[0], k, c[1]
        if best_key is None:
            break
        level[best_key[0]][best_key[1]] = best_new
        cand[best_key] = candidate(best_key)
        weighted = 0.0
        for li in range(num_layers):
            for p in PROJ_NAMES:
                weighted += level[li][p] * param_weights[p]
        current = weighted / total_weight

    thresholds = {}
    for li in range(num_layers):
        thresholds[li] = {}
        for p in PROJ_NAMES:
            s = level[li][p]
            if s > 0 and (li, p) in histograms:
                h = histograms[(li, p)]
                thresholds[li][p] = compute_threshold_from_histogram(h["counts"], h["edges"], s)
            else:
                thresholds[li][p] = 0.0
    return thresholds

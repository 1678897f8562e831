"""Per-projection TEAL thresholds from a calibration forward pass (host side).

Follows the reference's calibration_data path of apply_teal
(leankv/teal/patching.py:108-114, 241-256): the inputs each projection sees on
a few samples are collected with forward pre-hooks and the threshold is the
k-th smallest magnitude, k = int(sparsity * n) (sparse_fns.py:47-69).  The
sparsity may differ per projection; the result has the JSON layout that
apply_teal(thresholds=...) and save_thresholds use:
{layer: {proj_name: threshold}} (leankv/teal/greedy_opt.py:183-199).
"""

from __future__ import annotations

import json
import random
from typing import Callable, Union

import torch

from .patching import PROJ_NAMES, _get_layers, _get_projection
from .sparse_fns import compute_threshold_for_sparsity

SparsitySpec = Union[float, dict, Callable[[int, str], float]]


def uniform_random_sparsity(lo: float = 0.3, hi: float = 0.5, seed: int = 0) -> Callable[[int, str], float]:
    """Per-projection sparsity drawn from U[lo, hi] with a seeded generator."""
    rng = random.Random(seed)
    table: dict = {}

    def f(layer: int, proj: str) -> float:
        key = (layer, proj)
        if key not in table:
            table[key] = rng.uniform(lo, hi)
        return table[key]

    return f


@torch.no_grad()
def calibrate_thresholds(model, samples: list, sparsity: SparsitySpec, positions: slice | None = None) -> dict:
    """Run `samples` (token id tensors [1, S]) through `model`; return {layer: {proj: t}}.

    By default every position of every sample feeds the quantile, as the reference's calibration_data path
    does (patching.py:241-256).  ``positions`` keeps only those sequence positions of each sample (e.g.
    ``slice(-256, None)``: the last 256 tokens of a long prompt), so thresholds can be taken at the context a
    decode runs at: a projection's input statistics move with the context (an attention output averages
    over more values at a longer context and shrinks), and a threshold from short-context positions then
    drops more of the decode's inputs than its target sparsity asks."""
    layers = _get_layers(model)
    acts: dict = {}
    handles = []
    for li, layer in enumerate(layers):
        for pn in PROJ_NAMES:
            mod = _get_projection(layer, pn)

            def hook(module, args, key=(li, pn)):
                a = args[0].detach()
                if positions is not None:
                    a = a[..., positions, :]  # [B, S, D] -> the kept sequence positions
                acts.setdefault(key, []).append(a.reshape(-1, a.shape[-1]))

            handles.append(mod.register_forward_pre_hook(hook))
    try:
        for s in samples:
            model(s.to(model.device))
    finally:
        for h in handles:
            h.remove()
    out: dict = {}
    for (li, pn), xs in acts.items():
        if callable(sparsity):
            sp = sparsity(li, pn)
        elif isinstance(sparsity, dict):
            sp = sparsity.get(li, {}).get(pn, 0.0)
        else:
            sp = float(sparsity)
        x = torch.cat(xs, dim=0)
        out.setdefault(li, {})[pn] = compute_threshold_for_sparsity(x.float(), sp)
    return out


def save_thresholds(thresholds: dict, path: str) -> None:
    with open(path, "w") as f:
        json.dump({str(k): v for k, v in thresholds.items()}, f, indent=2)


def load_thresholds(path: str) -> dict:
    with open(path) as f:
        return {int(k): v for k, v in json.load(f).items()}

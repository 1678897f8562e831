"""TEAL calibration: activation-magnitude histograms at every projection input (host side).

Drop-in for leankv/teal/calibration.py: collect_activation_histograms runs the
model on calibration samples with forward pre-hooks on every TEAL projection
(PROJ_NAMES), first to find each input's largest magnitude (on the first 20
samples), then to bin |x| into `num_bins` equal bins over [0, 1.1 x max]
(values past the range land in the last bin); load_histograms reads the
per-projection files it saves.  The binning expression, bin range, file names
and file contents are the reference's (calibration.py:17-183, 186-199), so the
histograms feed greedy_opt.greedy_optimize unchanged.

One addition for machines without network access: `samples=` takes the
calibration token ids directly (a list of [1, S] tensors); without it the
samples come from `datasets.load_dataset(dataset_name, ...)` and the tokenizer
as in the reference (samples shorter than 32 tokens are skipped).
"""

from __future__ import annotations

import os
from typing import Optional

import torch

from .patching import PROJ_NAMES, _get_layers, _get_projection


def _load_samples(tokenizer, num_samples, seq_len, dataset_name, dataset_split, dataset_config) -> list:
    from datasets import load_dataset

    dataset = load_dataset(dataset_name, dataset_config, split=dataset_split, streaming=True)
    tokenizer.pad_token = tokenizer.pad_token or tokenizer.eos_token
    samples = []
    for i, example in enumerate(dataset):
        if i >= num_samples:
            break
        tokens = tokenizer(example.get("text", ""), return_tensors="pt", max_length=seq_len, truncation=True,
                           padding=False)
        if tokens["input_ids"].shape[1] >= 32:
            samples.append(tokens["input_ids"])
    return samples


@torch.no_grad()
def collect_activation_histograms(model, tokenizer=None, num_samples: int = 300, seq_len: int = 512,
                                  num_bins: int = 2000, dataset_name: str = "allenai/c4",
                                  dataset_split: str = "train", dataset_config: str = "en",
                                  save_dir: Optional[str] = None, samples: Optional[list] = None) -> dict:
    """{(layer, proj): {"counts", "edges", "max_val", "total"}} over the calibration samples."""
    if samples is None:
        if tokenizer is None:
            raise ValueError("collect_activation_histograms: pass samples= or a tokenizer for the dataset")
        samples = _load_samples(tokenizer, num_samples, seq_len, dataset_name, dataset_split, dataset_config)
    if not samples:
        raise ValueError("collect_activation_histograms: no calibration samples")
    layers = _get_layers(model)
    keys = [(li, p) for li in range(len(layers)) for p in PROJ_NAMES]

    def hooked(make):
        handles = []
        for li, layer in enumerate(layers):
            for p in PROJ_NAMES:
                handles.append(_get_projection(layer, p).register_forward_pre_hook(make((li, p))))
        return handles

    # pass 1: the largest magnitude of each projection input on the first 20 samples
    top = {k: 0.0 for k in keys}

    def range_hook(key):
        def fn(module, args):
            top[key] = max(top[key], args[0].abs().max().item())
        return fn

    handles = hooked(range_hook)
    try:
        for s in samples[: min(20, len(samples))]:
            model(s.to(model.device))
    finally:
        for h in handles:
            h.remove()

    # pass 2: |x| binned into num_bins over [0, 1.1 max]; past the range -> the last bin
    hist = {k: {"counts": torch.zeros(num_bins, dtype=torch.long), "max_val": top[k] * 1.1} for k in keys}

    def hist_hook(key):
        def fn(module, args):
            mag = args[0].abs().flatten()
            mv = hist[key]["max_val"]
            bins = (mag / (mv + 1e-10) * num_bins).long().clamp(0, num_bins - 1)
            hist[key]["counts"] += torch.bincount(bins, minlength=num_bins).cpu()
        return fn

    handles = hooked(hist_hook)
    try:
        for s in samples:
            model(s.to(model.device))
    finally:
        for h in handles:
            h.remove()

    results = {}
    for key, d in hist.items():
        results[key] = {"counts": d["counts"], "edges": torch.linspace(0, d["max_val"], num_bins + 1),
                        "max_val": d["max_val"], "total": d["counts"].sum().item()}
    if save_dir is not None:
        os.makedirs(save_dir, exist_ok=True)
        for (li, p), h in results.items():
            torch.save({"counts": h["counts"], "edges": h["edges"], "max_val": h["max_val"]},
                       os.path.join(save_dir, "layer%d_%s.pt" % (li, p)))
    return results


def load_histograms(hist_dir: str) -> dict:
    """Histograms saved by collect_activation_histograms: files layer{i}_{proj}.pt (calibration.py:186-199)."""
    results = {}
    for fname in os.listdir(hist_dir):
        if not fname.endswith(".pt"):
            continue
        layer, proj = fname[: -len(".pt")].split("_", 1)
        results[(int(layer.replace("layer", "")), proj)] = torch.load(os.path.join(hist_dir, fname),
                                                                       weights_only=True)
    return results

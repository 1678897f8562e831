"""CPU tests of the TEAL calibration pipeline: activation histograms and the greedy sparsity allocation.

greedy_optimize is pinned by golden vectors the reference's own greedy_opt.py
produced on seeded synthetic histograms (tests/golden/make_greedy_golden.py);
histogram collection by independently captured projection inputs.
"""

import json
import os

import numpy as np
import pytest
import torch

from leankv_amd.teal import greedy_opt as go
from leankv_amd.teal.calibration import collect_activation_histograms, load_histograms
from leankv_amd.teal.patching import PROJ_NAMES, _get_layers, _get_projection
from leankv_amd.teal.sparse_fns import compute_threshold_for_sparsity, compute_threshold_from_histogram

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "greedy_opt_cases.json")


def _hists(case):
    bins = case["bins"]
    return {(h["layer"], h["proj"]): {"counts": torch.tensor(h["counts"], dtype=torch.long),
                                      "edges": torch.linspace(0, h["max_val"], bins + 1)}
            for h in case["histograms"]}


@pytest.mark.parametrize("i", [0, 1, 2])
def test_greedy_optimize_matches_reference_golden(i):
    case = json.load(open(GOLDEN))[i]
    st = case["setting"]
    th = go.greedy_optimize(_hists(case), st["target"], 3, param_weights=st["weights"], step_size=st["step"])
    ref = {int(k): v for k, v in case["thresholds"].items()}
    assert th == ref


def test_greedy_optimize_properties():
    case = json.load(open(GOLDEN))[0]
    hists = _hists(case)
    # one projection's activations 10x larger: pruning it costs more, so it ends no sparser than its peers
    big = dict(hists)
    h = hists[(1, "o_proj")]
    big[(1, "o_proj")] = {"counts": h["counts"], "edges": h["edges"] * 10}
    th = go.greedy_optimize(big, 0.4, 3)
    levels = {}
    for li in range(3):
        for p in PROJ_NAMES:
            t = th[li][p]
            hh = big[(li, p)]
            # recover the sparsity each threshold stands for from its histogram CDF
            cdf = (hh["counts"].cumsum(0).float() / hh["counts"].sum()).numpy()
            edges = hh["edges"].numpy()
            levels[(li, p)] = float(np.interp(t, edges[1:], cdf)) if t > 0 else 0.0
    assert levels[(1, "o_proj")] <= levels[(0, "o_proj")] + 1e-6
    assert levels[(1, "o_proj")] <= levels[(2, "o_proj")] + 1e-6
    w = go._DEFAULT_PARAM_WEIGHTS
    glob = sum(levels[k] * w[k[1]] for k in levels) / (sum(w.values()) * 3)
    assert 0.38 <= glob <= 0.47  # reaches the 40 % budget within about one step
    assert all(v <= 0.95 + 1e-6 for v in levels.values())


def _tiny_model():
    from transformers import MistralConfig, MistralForCausalLM

    cfg = MistralConfig(vocab_size=200, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                        num_attention_heads=2, num_key_value_heads=1, head_dim=64, max_position_embeddings=128)
    torch.manual_seed(0)
    return MistralForCausalLM(cfg).eval()


def test_collect_histograms_counts_and_range():
    model = _tiny_model()
    g = torch.Generator().manual_seed(1)
    samples = [torch.randint(0, 200, (1, n), generator=g) for n in (16, 9, 23)]
    # the projection inputs, captured independently
    seen = {}
    handles = []
    for li, layer in enumerate(_get_layers(model)):
        for p in PROJ_NAMES:
            def hk(m, args, key=(li, p)):
                seen.setdefault(key, []).append(args[0].detach().reshape(-1).clone())
            handles.append(_get_projection(layer, p).register_forward_pre_hook(hk))
    with torch.no_grad():
        for s in samples:
            model(s)
    for hd in handles:
        hd.remove()
    hists = collect_activation_histograms(model, samples=samples, num_bins=500)
    assert set(hists) == set(seen)
    for key, h in hists.items():
        x = torch.cat(seen[key]).abs()
        assert h["total"] == x.numel() == int(h["counts"].sum())
        assert h["max_val"] == pytest.approx(1.1 * float(x.max()), rel=1e-6)
        assert float(h["edges"][-1]) == pytest.approx(h["max_val"], rel=1e-6)
        # the histogram's 40 % threshold lies within one bin of the exact kth-value threshold
        t_hist = compute_threshold_from_histogram(h["counts"], h["edges"], 0.4)
        t_exact = compute_threshold_for_sparsity(x, 0.4)
        assert abs(t_hist - t_exact) <= float(h["edges"][1] - h["edges"][0]) + 1e-7


def test_histograms_save_load_and_thresholds_roundtrip(tmp_path):
    from leankv_amd.teal.patching import apply_teal

    model = _tiny_model()
    g = torch.Generator().manual_seed(2)
    samples = [torch.randint(0, 200, (1, 12), generator=g) for _ in range(2)]
    hists = collect_activation_histograms(model, samples=samples, num_bins=100, save_dir=str(tmp_path / "h"))
    back = load_histograms(str(tmp_path / "h"))
    assert set(back) == set(hists)
    for k in hists:
        assert torch.equal(back[k]["counts"], hists[k]["counts"])
        assert torch.equal(back[k]["edges"], hists[k]["edges"])
    th = go.greedy_optimize(hists, 0.4, 2)
    path = str(tmp_path / "thresholds.json")
    go.save_thresholds(th, path)
    assert go.load_thresholds(path) == th
    fns = apply_teal(model, thresholds_path=path)  # the reference's thresholds file layout is accepted
    assert len(fns) == 2 * len(PROJ_NAMES)


def test_calibrate_thresholds_positions_select_the_sequence_tail():
    """calibrate_thresholds(positions=slice(-8, None)) takes each projection's quantile over the last 8
    positions only.  Layer 0's q/k/v/gate... inputs of a position depend on that token alone before the first
    attention (q/k/v: RMSNorm of the embedding), so its q_proj threshold equals the one calibrated on the last 8
    tokens by themselves; its o_proj input (the attention output) depends on the whole context, so that one
    differs.  Slicing the wrong axis or end fails the first equality."""
    from leankv_amd.engine import random_mistral
    from leankv_amd.teal.calibrate import calibrate_thresholds

    tiny = dict(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                num_attention_heads=4, num_key_value_heads=2, head_dim=128)
    m = random_mistral(device="cpu", seed=5, **tiny)
    ids = torch.randint(0, 512, (1, 40), generator=torch.Generator().manual_seed(6))
    tail = calibrate_thresholds(m, [ids], 0.4, positions=slice(-8, None))
    alone = calibrate_thresholds(m, [ids[:, -8:]], 0.4)
    assert tail[0]["q_proj"] == alone[0]["q_proj"]
    assert tail[0]["o_proj"] != alone[0]["o_proj"]

"""Write golden vectors for the TEAL greedy sparsity allocation from the reference's own code.

greedy_optimize (leankv/teal/greedy_opt.py:47-164) picks, step by step, the
projection whose next sparsity increment prunes the least estimated L2 mass;
the estimate is an fp32 sum over histogram bins (:167-197) and ties go to the
first key in layer / PROJ_NAMES order, so the exact thresholds it returns are
pinned by no closed form.  This script imports that module from the read-only
reference checkout (in the build container only; nothing on the GPU box reads
/root/reference), runs it on seeded synthetic activation-magnitude histograms
(3 layers x 7 projections, 300 bins, Laplace-like magnitudes with a per-
projection scale and a few outliers) for three settings, and records inputs
and outputs.

Run:  python tests/golden/make_greedy_golden.py [/root/reference]
"""

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
PROJ_NAMES = ["q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"]


def synthetic_histograms(seed: int, layers: int = 3, bins: int = 300) -> dict:
    rng = np.random.default_rng(seed)
    out = {}
    for li in range(layers):
        for j, p in enumerate(PROJ_NAMES):
            scale = 0.02 * (1 + j) * (1 + 0.5 * li)
            mags = np.abs(rng.laplace(0.0, scale, size=20000))
            mags[:5] *= 8.0  # outliers stretch the range
            max_val = float(mags.max()) * 1.1
            counts = np.clip((mags / (max_val + 1e-10) * bins).astype(np.int64), 0, bins - 1)
            out[(li, p)] = {"counts": np.bincount(counts, minlength=bins).tolist(), "max_val": max_val}
    return out


def as_torch(hists: dict, bins: int) -> dict:
    return {k: {"counts": torch.tensor(v["counts"], dtype=torch.long),
                "edges": torch.linspace(0, v["max_val"], bins + 1)} for k, v in hists.items()}


SETTINGS = [
    {"seed": 1, "target": 0.4, "step": 0.05, "weights": None},
    {"seed": 2, "target": 0.5, "step": 0.1, "weights": None},
    {"seed": 3, "target": 0.3, "step": 0.05,
     "weights": {"q_proj": 1.0, "k_proj": 1.0, "v_proj": 1.0, "o_proj": 1.0, "gate_proj": 1.0, "up_proj": 1.0,
                 "down_proj": 1.0}},
]


def main(ref_root: str = "/root/reference") -> None:
    sys.dont_write_bytecode = True  # leave the read-only checkout untouched (no __pycache__)
    sys.path.insert(0, ref_root)
    from leankv.teal import greedy_opt as ref  # noqa: E402

    cases = []
    for st in SETTINGS:
        hists = synthetic_histograms(st["seed"])
        th = ref.greedy_optimize(as_torch(hists, 300), st["target"], 3, param_weights=st["weights"],
                                 step_size=st["step"])
        cases.append({
            "source": "leankv/teal/greedy_opt.py:greedy_optimize(histograms, %g, 3, step_size=%g)" % (
                st["target"], st["step"]),
            "setting": st,
            "bins": 300,
            "histograms": [{"layer": k[0], "proj": k[1], "counts": v["counts"], "max_val": v["max_val"]}
                           for k, v in hists.items()],
            "thresholds": {str(li): {p: float(t) for p, t in d.items()} for li, d in th.items()},
        })
    path = os.path.join(HERE, "greedy_opt_cases.json")
    with open(path, "w") as f:
        json.dump(cases, f)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main(*sys.argv[1:])

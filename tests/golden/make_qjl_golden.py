"""Write golden vectors for TurboQuantProd (MSE at bits - 1 + 1-bit QJL) from the reference's own code.

TurboQuantProd (leankv/turboquant/quantizer.py:144-237) draws its projection S
from torch.randn with seed + 1000 (rotation.py:32-42), takes the sign of the
projected residual as bit i of byte j for coordinate 8j + i, and rescales by
sqrt(pi/2) / d * ||r||.  The seed offset, the bit order and the sign convention
at exactly zero are fixed by that code alone, so this script imports the
module from the read-only reference checkout (in the build container only;
nothing on the GPU box reads /root/reference), runs quantize and dequantize on
seeded inputs for bits 2..4 (fp32) and bits 3 (fp16), and records inputs and
outputs.  The codebooks the reference would solve are handed to its in-memory
codebook cache from this repository's own golden codebooks (the reference
solver's recorded outputs), so nothing is written inside the checkout.

Run:  python tests/golden/make_qjl_golden.py [/root/reference]
"""

import hashlib
import json
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROWS = 4
CASES = [(2, torch.float32, 11), (3, torch.float32, 12), (4, torch.float32, 13), (3, torch.float16, 14)]


def main(ref_root: str = "/root/reference") -> None:
    sys.dont_write_bytecode = True  # leave the read-only checkout untouched (no __pycache__)
    sys.path.insert(0, ref_root)
    from leankv.turboquant import codebook as ref_codebook  # noqa: E402
    from leankv.turboquant import quantizer as ref_quantizer  # noqa: E402

    for bits in (1, 2, 3):
        with open(os.path.join(HERE, "codebook_d128_b%d.json" % bits)) as f:
            ref_codebook._CODEBOOK_CACHE[(128, bits)] = json.load(f)

    cases = []
    for bits, dtype, seed in CASES:
        g = torch.Generator().manual_seed(seed)
        x = (torch.randn(ROWS, 128, generator=g) * 0.7).to(dtype)
        x[0, 5] = 4.0  # one outlier coordinate
        tq = ref_quantizer.TurboQuantProd(128, bits=bits, device=torch.device("cpu"), seed=42)
        q = tq.quantize(x)
        xr = tq.dequantize(q)
        S = tq.S.contiguous()
        cases.append({
            "source": "leankv/turboquant/quantizer.py:TurboQuantProd(128, bits=%d, seed=42) quantize + dequantize"
                      % bits,
            "bits": bits,
            "dtype": str(dtype).replace("torch.", ""),
            "x": x.float().tolist(),
            "mse_indices": q.mse_indices.tolist(),
            "qjl_signs": q.qjl_signs.tolist(),
            "residual_norms": q.residual_norms.tolist(),
            "norms": q.norms.float().tolist(),
            "mse_bits": q.mse_bits,
            "dequantized": xr.tolist(),
            "qjl_scale": tq.qjl_scale,
            "S_sha256": hashlib.sha256(S.numpy().tobytes()).hexdigest(),
            "S_row0": S[0].tolist(),
        })
    path = os.path.join(HERE, "qjl_prod_cases.json")
    with open(path, "w") as f:
        json.dump(cases, f)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main(*sys.argv[1:])

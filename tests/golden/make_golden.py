"""Write the Lloyd-Max codebook golden fixtures from the reference's own solver.

The codebook is the one value on the decode path that no closed form, invariant
or library routine pins bit-for-bit: the reference solves the continuous
Lloyd-Max problem with scipy quadrature and stops early (|dcost| < 1e-12,
<= 200 iterations, quantile initialisation on a 10 000-point grid), so the
float32 centroids and decision boundaries it ships to the kernels depend on
that exact solver run (reference: leankv/turboquant/codebook.py:62-129).

This script imports that one module from the read-only reference checkout (in
the build container only; nothing on the GPU box reads /root/reference) and
records, for d=128 and bits 1..4, the float64 lists the solver returns plus the
float32 bit patterns the reference hands to torch
(leankv/turboquant/codebook.py:163-170).

Run:  python tests/golden/make_golden.py [/root/reference]
"""

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def main(ref_root: str = "/root/reference") -> None:
    sys.dont_write_bytecode = True  # leave the read-only checkout untouched (no __pycache__)
    sys.path.insert(0, ref_root)
    # Import the solver module directly: get_codebook() would try to create a
    # cache directory inside the read-only checkout (codebook.py:143).
    from leankv.turboquant import codebook as ref_codebook  # noqa: E402

    for bits in (1, 2, 3, 4):
        cb = ref_codebook.compute_lloyd_max_codebook(128, bits)
        out = {
            "source": "leankv/turboquant/codebook.py:compute_lloyd_max_codebook(128, %d)" % bits,
            "d": cb["d"],
            "bits": cb["bits"],
            "centroids": cb["centroids"],
            "boundaries": cb["boundaries"],
            "mse_per_coord": cb["mse_per_coord"],
            "mse_total": cb["mse_total"],
            "centroids_f32_hex": [
                "%08x" % v for v in np.asarray(cb["centroids"], np.float32).view(np.uint32)
            ],
            "boundaries_f32_hex": [
                "%08x" % v for v in np.asarray(cb["boundaries"], np.float32).view(np.uint32)
            ],
        }
        path = os.path.join(HERE, "codebook_d128_b%d.json" % bits)
        with open(path, "w") as f:
            json.dump(out, f, indent=1)
        print("wrote", path, "mse/coord=%.6e" % cb["mse_per_coord"])


if __name__ == "__main__":
    main(*sys.argv[1:])

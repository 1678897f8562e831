"""The tie rule of the quantize parity tests (shared by the GPU tests and their CPU self-check).

TurboQuantMSE.quantize (leankv/turboquant/quantizer.py:119-129) buckets y = u Pi^T, a 128-term fp32 dot
product per coordinate.  Two correct fp32 evaluations (torch's CPU matmul, the kernel's MFMA chain) round
differently, by at most (128 + 2) * 2^-24 * S_j with S_j = sum_k |u_k Pi_jk| (forward error bound of a dot
product plus the rounding of u), so a coordinate whose exact value lies that close to a decision boundary can
take the neighbouring code.  Codes must be bit-exact everywhere else.
"""

import numpy as np

from oracle import turboquant as oq

# Tie window in units of 2^-24 * S_j.  The flips measured at config 3 sit within 0.43 units (2.3 fp32 ulps of
# the boundary), so 4 units keeps a margin while a wrong index, sign or operand (errors of order S_j itself)
# still fails.
TIE_ULPS = 4.0


def _rotation_fp64(x, Pi, norms=None):
    """y = u Pi^T in fp64 and S = |u| |Pi|^T (per-coordinate sum of |u_k Pi_jk|) from the fp32 unit vector u that
    quantize builds, x / (norm + 1e-10) in x's dtype (quantizer.py:121-123); norms default to torch's."""
    x = x.cpu()
    n = x.norm(dim=-1) if norms is None else norms.to(x.dtype)
    u = (x / (n.unsqueeze(-1) + 1e-10)).float().double().numpy()
    P = Pi.double().numpy()
    return u @ P.T, np.abs(u) @ np.abs(P).T


def _codes_match(p_gpu, p_ref, y64, S, bounds, bits):
    """Bit-exact codes except coordinates within TIE_ULPS * 2^-24 * S of a boundary, which may take the
    neighbouring code; returns #flips."""
    cg = oq.unpack_indices(p_gpu, bits, 128)
    cr = oq.unpack_indices(p_ref, bits, 128)
    diff = cg != cr
    if not diff.any():
        return 0
    inner = bounds[1:-1].double().numpy()
    dist = np.abs(y64[..., None] - inner).min(-1)
    window = TIE_ULPS * 2.0 ** -24 * S
    bad = diff & (dist >= window)
    assert not bad.any(), "code mismatch outside the fp32 tie window: %d coords, worst %.3g units" % (
        int(bad.sum()), float((dist[bad] / (2.0 ** -24 * S[bad])).max()))
    assert (np.abs(cg.astype(int) - cr.astype(int))[diff] == 1).all()
    return int(diff.sum())

"""CPU restatement of TEAL sparsification + sparse GEMV (test infrastructure).

References (under /root/reference, read as text):
  leankv/teal/sparse_fns.py:32-39      SparsifyFn.__call__: x * (|x| > t)
  leankv/teal/sparse_fns.py:47-69      compute_threshold_for_sparsity (kthvalue)
  leankv/teal/kernels/sparse_gemv.py:77-87  y[n] += sum_{|x_z|>t} A[z,n] x_z
      (the Triton kernel compares |x| (fp16 widened) with the fp32 threshold)
  transformers/models/mistral/modeling_mistral.py:46-47  down(silu(gate x) * up x)
"""

from __future__ import annotations

import numpy as np
import torch


def keep_mask(x16: np.ndarray, threshold: float) -> np.ndarray:
    """|x| > t with |x| widened from fp16 and t rounded to fp32 (sparse_gemv.py:81-82)."""
    a = np.abs(np.asarray(x16, dtype=np.float16).astype(np.float32))
    return a > np.float32(threshold)


def sparsify(x16: np.ndarray, threshold: float) -> np.ndarray:
    """SparsifyFn semantics (sparse_fns.py:32-39) in the Triton path's fp32 compare."""
    x = np.asarray(x16, dtype=np.float16)
    return np.where(keep_mask(x, threshold), x, np.float16(0))


def threshold_for_sparsity(acts: torch.Tensor, target: float) -> float:
    """compute_threshold_for_sparsity (sparse_fns.py:47-69): k-th smallest |x|, k=int(s*n)."""
    mags = acts.detach().abs().flatten().cpu()
    k = int(target * mags.numel())
    if k <= 0:
        return 0.0
    if k >= mags.numel():
        return mags.max().item()
    return torch.kthvalue(mags, k).values.item()


def sparse_gemv(x16: np.ndarray, w16: np.ndarray, threshold: float) -> np.ndarray:
    """fp64 truth of W[N,Z] @ sparsify(x): only rows whose |x|>t contribute."""
    x = np.asarray(x16, dtype=np.float16).reshape(-1)
    W = np.asarray(w16, dtype=np.float16)
    m = keep_mask(x, threshold)
    xs = np.where(m, x.astype(np.float64), 0.0)
    cols = np.nonzero(m)[0]
    return W[:, cols].astype(np.float64) @ xs[cols]


def f16(v) -> np.ndarray:
    return np.asarray(v, dtype=np.float64).astype(np.float16)


def silu_f16(g16: np.ndarray) -> np.ndarray:
    """torch fp16 silu: computed in fp32 (opmath), rounded to fp16."""
    g = np.asarray(g16, dtype=np.float16).astype(np.float32)
    return (g / (np.float32(1) + np.exp(-g))).astype(np.float16)


def gateup_swiglu(x16, wg16, wu16, t_gate: float, t_up: float) -> np.ndarray:
    """fp16 h = silu(fp16(gate(x))) * fp16(up(x)) with TEAL-patched gate/up.

    Eager sequence of modeling_mistral.py:46-47 on the outputs of two
    sparse_gemv calls, each rounded to fp16 by the kernel wrapper
    (sparse_gemv.py:164).  The GEMV sums themselves are fp64 here.
    """
    g = f16(sparse_gemv(x16, wg16, t_gate))
    u = f16(sparse_gemv(x16, wu16, t_up))
    s = silu_f16(g)
    return (s.astype(np.float32) * u.astype(np.float32)).astype(np.float16)


def rel_err(actual, ref) -> float:
    a = np.asarray(actual, dtype=np.float64).reshape(-1)
    r = np.asarray(ref, dtype=np.float64).reshape(-1)
    den = np.linalg.norm(r)
    return float(np.linalg.norm(a - r) / (den if den > 0 else 1.0))


def max_rel_err(actual, ref) -> float:
    """max |a - r| / max |r| -- elementwise bound scaled by the largest output."""
    a = np.asarray(actual, dtype=np.float64).reshape(-1)
    r = np.asarray(ref, dtype=np.float64).reshape(-1)
    den = np.abs(r).max() if r.size else 0.0
    return float(np.abs(a - r).max() / (den if den > 0 else 1.0)) if r.size else 0.0

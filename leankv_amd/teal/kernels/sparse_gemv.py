"""TEAL sparse GEMV entry points with the reference's signatures, on HIP.

Drop-in for leankv/teal/kernels/sparse_gemv.py:
  sparse_gemv(x, weight, threshold, sparsity_bin)        (:143-181)
  batched_sparse_gemm(x, weight, threshold, sparsity_bin) (:184-226)
  prepare_weight_for_sparse_gemv(weight)                 (:229-234)
plus fusions with no single reference counterpart: sparse_gateup_swiglu
(the gate and up sparse_gemv calls of a TEAL-patched Mistral MLP and its
SwiGLU, x read once), sparse_qkv (the q, k and v sparse_gemv calls of an
attention layer, x read once) and their dense forms for a few decode rows,
batched_qkv and batched_gateup_swiglu (the batched_sparse_gemm calls with
threshold 0 that the reference's dense dispatch at B > 1 stands for, one
launch each).

These are the dispatcher boundary of the TEAL path: each call goes through
torch.ops.leankv (leankv_amd.kernels registers the ops, GPU + Meta), as the
reference's calls go through its Triton launcher.  sparsity_bin only keyed the
Triton autotuner; the HIP kernel picks its launch shape from (N, Z) and the
argument is accepted and ignored.
"""

from __future__ import annotations

import torch

from ... import kernels as _k  # registers torch.ops.leankv


def prepare_weight_for_sparse_gemv(weight: torch.Tensor) -> torch.Tensor:
    """Column-major copy of W[N, Z] (row z of the storage = weight column z)."""
    return weight.t().contiguous().t()


def sparse_gemv(x: torch.Tensor, weight: torch.Tensor, threshold: float, sparsity_bin: int = 5) -> torch.Tensor:
    """[1, 1, N] = sparse(x[1, 1, Z]) @ W^T for column-major fp16 W[N, Z]."""
    N, Z = weight.shape
    xh = x.reshape(Z)
    if xh.dtype != torch.float16:
        xh = xh.to(torch.float16)
    out = torch.ops.leankv.sparse_gemv(xh, weight, float(threshold)).reshape(1, 1, N)
    if x.dtype != torch.float16:
        out = out.to(x.dtype)
    return out


def batched_sparse_gemm(x: torch.Tensor, weight: torch.Tensor, threshold: float,
                        sparsity_bin: int = 5) -> torch.Tensor:
    """[B, N]: each row of x[B, Z] gets its own mask (sparse_gemv.py:184-226); one pass over the weight
    rows some row keeps (lkv_sparse_gemm_batched).  sparsity_bin is the reference's autotune key, unused."""
    N, Z = weight.shape
    xs = x.reshape(-1, Z).to(torch.float16).contiguous()
    out = _k.sparse_gemm_batched(xs, weight, threshold)
    return out if x.dtype == torch.float16 else out.to(x.dtype)


def sparse_gateup_swiglu(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, t_gate: float,
                         t_up: float) -> torch.Tensor:
    """fp16 [1, 1, N] = silu(gate(x)) * up(x) with TEAL thresholds on both inputs."""
    N, Z = w_gate.shape
    xh = x.reshape(Z)
    if xh.dtype != torch.float16:
        xh = xh.to(torch.float16)
    return torch.ops.leankv.sparse_gateup_swiglu(xh, w_gate, w_up, float(t_gate), float(t_up)).reshape(1, 1, N)


def sparse_qkv(x: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor, wv: torch.Tensor, tq: float, tk: float,
               tv: float):
    """fp16 (q, k, v) of one single-token x through three TEAL-patched projections (column-major weights)."""
    Z = wq.shape[1]
    xh = x.reshape(Z)
    if xh.dtype != torch.float16:
        xh = xh.to(torch.float16)
    return torch.ops.leankv.sparse_qkv(xh, wq, wk, wv, float(tq), float(tk), float(tv))


def batched_qkv(x: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor, wv: torch.Tensor,
                cos: torch.Tensor | None = None, sin: torch.Tensor | None = None):
    """fp16 (q, k, v) [rows, N_s] of x[rows, Z] through three column-major weights, threshold 0, one launch: each
    equal to its own batched_sparse_gemm(x, w, 0.0) call bit for bit; with cos / sin (one position's fp16 factors
    [128]) q and k come out rotated as HF's apply_rotary_pos_emb rotates them."""
    epi = _k.EPI_ROPE if cos is not None else _k.EPI_NONE
    return tuple(_k.sparse_gemm_batched_multi(x.to(torch.float16).contiguous(), [wq, wk, wv], [0.0, 0.0, 0.0], epi,
                                              cos=cos, sin=sin))


def batched_gateup_swiglu(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """fp16 [rows, N] = silu(gate(x)) * up(x) of x[rows, Z] with the fp16 roundings of HF's eager MLP, threshold 0,
    one launch: equal to F.silu(batched_sparse_gemm(x, w_gate, 0.0)) * batched_sparse_gemm(x, w_up, 0.0)."""
    return _k.sparse_gemm_batched_multi(x.to(torch.float16).contiguous(), [w_gate, w_up], [0.0, 0.0],
                                        _k.EPI_SWIGLU)[0]

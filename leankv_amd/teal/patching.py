"""Apply TEAL activation sparsity to a HuggingFace decoder, on HIP kernels.

Drop-in for leankv/teal/patching.py:
  apply_teal(model, sparsity, thresholds, thresholds_path, calibration_data,
             use_triton)                                   (:57-149)
  remove_teal(model), get_sparsity_report, print_sparsity_report (:186-238)
  _collect_input_activations                               (:241-256)

Threshold selection, the "exactly one source" rule and the hook-based
correctness mode are the reference's.  ``use_triton=True`` (name kept for
drop-in callers; ``use_hip`` is an alias) routes every projection with t > 0
to the HIP sparse GEMV at B=1 single-token decode and keeps the dense product
otherwise, the reference's dispatch rule (:169-180): a few decode rows on the
batched kernel with threshold 0, larger inputs on torch's F.linear.  In addition, when both
gate_proj and up_proj of a layer are patched, the MLP forward is patched so the
two projections and the SwiGLU run as one fused HIP kernel reading x once
(``fuse_mlp=False`` turns this off), and when q_proj, k_proj and v_proj are
all patched, the three run as one launch reading x once (``fuse_qkv=False``
turns this off): q_proj computes all three and k_proj / v_proj hand back
their share when called on the same input tensor.  Both fusions also take a
few decode rows (B > 1): the dense products as one batched launch, with the
SwiGLU in its reduce for gate/up, each result equal to the unfused calls'.
"""

from __future__ import annotations

import json
from typing import Optional

import torch
import torch.nn as nn

from .kernels.sparse_gemv import (batched_gateup_swiglu, batched_qkv, batched_sparse_gemm, prepare_weight_for_sparse_gemv,
                                  sparse_gateup_swiglu, sparse_gemv, sparse_qkv)
from .sparse_fns import SparsifyFn, compute_threshold_for_sparsity

PROJ_NAMES = ["q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"]
ATTN_PROJS = {"q_proj", "k_proj", "v_proj", "o_proj"}
MLP_PROJS = {"gate_proj", "up_proj", "down_proj"}


def _get_layers(model):
    if hasattr(model, "model") and hasattr(model.model, "layers"):
        return model.model.layers
    raise ValueError(
        "Cannot find transformer layers in model of type %s. Expected model.model.layers attribute." % type(model)
    )


def _get_projection(layer, proj_name: str) -> nn.Linear:
    return getattr(layer.self_attn if proj_name in ATTN_PROJS else layer.mlp, proj_name)


def _is_single_token(x: torch.Tensor) -> bool:
    return x.shape[-2] == 1 and (x.shape[0] if x.dim() == 3 else 1) == 1


def apply_teal(
    model,
    sparsity: Optional[float] = None,
    thresholds: Optional[dict] = None,
    thresholds_path: Optional[str] = None,
    calibration_data: Optional[list] = None,
    use_triton: bool = False,
    use_hip: Optional[bool] = None,
    fuse_mlp: bool = True,
    fuse_qkv: bool = True,
):
    """Install TEAL on all 7 projections of every layer; returns {(layer, proj): SparsifyFn}."""
    if sum(v is not None for v in (sparsity, thresholds, thresholds_path)) != 1:
        raise ValueError("Exactly one of sparsity, thresholds, or thresholds_path must be provided.")
    use_kernel = bool(use_triton if use_hip is None else use_hip)

    if thresholds_path is not None:
        with open(thresholds_path, "r") as f:
            thresholds = {int(k): v for k, v in json.load(f).items()}

    layers = _get_layers(model)
    sparsifiers = {}
    hooks = []
    for layer_idx, layer in enumerate(layers):
        for proj_name in PROJ_NAMES:
            proj = _get_projection(layer, proj_name)
            if thresholds is not None:
                t = thresholds.get(layer_idx, thresholds.get(str(layer_idx), {})).get(proj_name, 0.0)
            elif sparsity is not None and sparsity > 0:
                if calibration_data is not None:
                    with torch.no_grad():
                        acts = _collect_input_activations(model, proj, calibration_data)
                        t = compute_threshold_for_sparsity(acts, sparsity)
                else:
                    t = sparsity * 0.1
            else:
                t = 0.0
            sf = SparsifyFn(threshold=t, enabled=(t > 0))
            sparsifiers[(layer_idx, proj_name)] = sf
            if use_kernel and t > 0:
                _patch_linear_with_kernel(proj, t)
            else:
                def make_hook(fn):
                    def hook_fn(module, args):
                        return (fn(args[0]),) + args[1:]
                    return hook_fn
                hooks.append(proj.register_forward_pre_hook(make_hook(sf)))
        if use_kernel and fuse_mlp:
            _maybe_patch_mlp(layer.mlp)
        if use_kernel and fuse_qkv:
            _maybe_patch_qkv(layer.self_attn)

    if not hasattr(model, "_teal_hooks"):
        model._teal_hooks = []
    model._teal_hooks.extend(hooks)
    model._teal_sparsifiers = sparsifiers
    print("[TEAL] Using HIP sparse GEMV kernels (gfx950)" if use_kernel
          else "[TEAL] Using hook-based sparsification (correctness only)")
    return sparsifiers


def _rows(x: torch.Tensor, Z: int) -> int:
    """Rows of x as a [rows, Z] matrix (0 when its last dim is not Z)."""
    return x.numel() // Z if x.dim() > 0 and x.shape[-1] == Z and Z > 0 else 0


def _skinny_gateup(rows: int) -> bool:
    """Whether a fused gate/up + SwiGLU of `rows` decode rows runs as one batched launch with the SwiGLU in its
    reduce (else the MLP's own modules run).  Up to 32 rows the grouped launch reads x once for both products
    and saves the two elementwise kernels of the SwiGLU, where torch's GEMM only edges out the batched kernel
    on one projection alone (32 rows: 54.3 + 5.6 us against 2 x 24.0 + 4.9 + 4.6)."""
    return 1 < rows <= 32


def _skinny_dense(rows: int, N: int, Z: int) -> bool:
    """Whether a dense product of `rows` decode rows runs on the batched kernel (threshold 0) rather than torch's
    GEMM.  Measured on one MI355X, back-to-back calls at the Mistral-7B shapes over the column-major weight, torch
    vs the batched kernel in us: down [4096 x 14336] 50 / 25 for 8 rows, 49-52 / 26 for 12-16; q|k|v
    [6144 x 4096] 19 / 15 and o [4096 x 4096] 19 / 12-15 for 8-16 rows; gate/up [14336 x 4096] 23-24 / 24 for 8
    rows, 23 / 25 for 12-16 (torch's GEMM then wins by a little).  17-32 rows run as one group of 32 (two MFMA
    tiles per weight pass): q|k|v grouped 16.2 + 3.9 (reduce) against 14.4 + 2 x 9.3, o 13.8 + 4.2 against 14.4,
    down 28.3 + 4.2 against ~28; the decode step's fusions (RoPE, ring write, residual + RMSNorm) ride on these
    launches, so the rule keeps every projection but gate / up on the batched kernel up to 32 rows."""
    return 1 < rows <= 32 and (rows <= 8 or N <= 2 * Z)


def _patch_linear_with_kernel(linear: nn.Linear, threshold: float) -> None:
    """Relayout the weight column-major (permanent) and route B=1 decode to HIP.

    Other inputs take the dense product, as the reference dispatches them (patching.py:169-180): a few
    decode rows (B > 1, or a short chunk) on the batched kernel with threshold 0, so every nonzero input
    contributes (fp32 accumulate, fp16 out, as F.linear), larger inputs (prefill) on torch's GEMM."""
    with torch.no_grad():
        linear.weight.data = prepare_weight_for_sparse_gemv(linear.weight.data)
    N, Z = linear.weight.shape

    def sparse_forward(x):
        if _is_single_token(x):
            out = sparse_gemv(x.reshape(1, 1, x.shape[-1]), linear.weight, threshold)
            out = out.reshape(x.shape[:-1] + (N,))
            if linear.bias is not None:
                out = out + linear.bias
            return out
        rows = _rows(x, Z)
        if x.dtype == torch.float16 and linear.bias is None and _skinny_dense(rows, N, Z):
            return batched_sparse_gemm(x.reshape(rows, Z), linear.weight, 0.0).reshape(x.shape[:-1] + (N,))
        return torch.nn.functional.linear(x, linear.weight, linear.bias)

    linear._teal_original_forward = linear.forward
    linear.forward = sparse_forward
    linear._teal_patched = True
    linear._teal_threshold = threshold


# Reference name kept for callers that reach into the module.
def _patch_linear_with_triton(linear: nn.Linear, threshold: float, sparsity: float = 0.4) -> None:
    _patch_linear_with_kernel(linear, threshold)


def _is_silu(act) -> bool:
    """Whether the MLP activation is SiLU (torch's nn.SiLU, or transformers' own SiLU module that ACT2FN["silu"]
    returns), judged by what it computes on a few points."""
    if isinstance(act, nn.SiLU):
        return True
    try:
        probe = torch.tensor([-3.0, -0.5, 0.0, 0.7, 4.0])
        return bool(torch.allclose(act(probe), torch.nn.functional.silu(probe)))
    except Exception:
        return False


def _maybe_patch_mlp(mlp: nn.Module) -> None:
    """Fuse gate/up + SwiGLU when both projections carry a kernel patch."""
    gate, up, down = getattr(mlp, "gate_proj", None), getattr(mlp, "up_proj", None), getattr(mlp, "down_proj", None)
    if gate is None or up is None or down is None:
        return
    if not (getattr(gate, "_teal_patched", False) and getattr(up, "_teal_patched", False)):
        return
    if gate.bias is not None or up.bias is not None:
        return
    act = getattr(mlp, "act_fn", None)
    if act is None or not _is_silu(act):
        return
    original = mlp.forward

    def fused_forward(x):
        if _is_single_token(x):
            h = sparse_gateup_swiglu(x, gate.weight, up.weight, gate._teal_threshold, up._teal_threshold)
            h = h.reshape(x.shape[:-1] + (gate.weight.shape[0],))
            if x.dtype != torch.float16:
                h = h.to(x.dtype)
            return down(h)
        h = _gateup_rows(mlp, x)
        return original(x) if h is None else down(h)

    mlp._teal_original_forward = original
    mlp.forward = fused_forward
    mlp._teal_fused = True


def _gateup_rows(mlp: nn.Module, x: torch.Tensor) -> Optional[torch.Tensor]:
    """silu(gate_proj(x)) * up_proj(x) of a fused MLP for a few fp16 decode rows, as one batched launch with the
    SwiGLU in its reduce: the dense products the reference dispatches at B > 1 (patching.py:169-180; threshold 0)
    and HF's fp16 SwiGLU (modeling_mistral.py:46-47) bit for bit.  None when the rows take the modules' own path."""
    gate, up = mlp.gate_proj, mlp.up_proj
    N, Z = gate.weight.shape
    rows = _rows(x, Z)
    if x.dtype != torch.float16 or not _skinny_gateup(rows):
        return None
    return batched_gateup_swiglu(x.reshape(rows, Z), gate.weight, up.weight).reshape(x.shape[:-1] + (N,))


def _maybe_patch_qkv(attn: nn.Module) -> None:
    """One launch for q/k/v when all three carry a kernel patch (no bias).

    q_proj's forward runs the fused kernel on its input and keeps k and v;
    k_proj / v_proj return them when called on the very tensor q_proj saw
    (unchanged since: same object and version counter), which is how HF's
    attention calls them (modeling_mistral.py:150-152); any other input takes
    the projection's own sparse GEMV.  A few decode rows (B > 1) that all three
    projections send to the batched kernel run as one batched launch the same
    way, each output equal to the projection's own call."""
    projs = [getattr(attn, n, None) for n in ("q_proj", "k_proj", "v_proj")]
    if any(p is None or not getattr(p, "_teal_patched", False) or p.bias is not None for p in projs):
        return
    q, k, v = projs
    held: dict = {}

    def q_forward(x, single=q.forward):
        if not _is_single_token(x):
            held.clear()
            ys = _qkv_rows(attn, x)  # the three dense products of a few decode rows (threshold 0), one launch
            if ys is None:
                return single(x)
            yq, yk, yv = ys
        else:
            yq, yk, yv = sparse_qkv(x, q.weight, k.weight, v.weight, q._teal_threshold, k._teal_threshold,
                                    v._teal_threshold)
        held.clear()
        held.update(x=x, version=x._version, k=yk, v=yv)
        lead = x.shape[:-1]
        out = yq.reshape(lead + (q.weight.shape[0],))
        return out if x.dtype == torch.float16 else out.to(x.dtype)

    def share(proj, key):
        single = proj.forward

        def fwd(x):
            if held.get("x") is x and held.get("version") == x._version and key in held:
                y = held.pop(key)
                if "k" not in held and "v" not in held:
                    held.clear()
                y = y.reshape(x.shape[:-1] + (proj.weight.shape[0],))
                return y if x.dtype == torch.float16 else y.to(x.dtype)
            return single(x)

        return fwd

    k.forward = share(k, "k")
    v.forward = share(v, "v")
    q.forward = q_forward
    attn._teal_qkv_fused = True


def _qkv_rows(attn: nn.Module, x: torch.Tensor, cos: Optional[torch.Tensor] = None,
              sin: Optional[torch.Tensor] = None):
    """(q, k, v) [rows, N] of a fused q/k/v patch for a few fp16 decode rows that all three projections send to
    the batched kernel, as one launch, each equal to the projection's own call; with cos / sin (one position's
    fp16 RoPE factors [128]) q and k come out rotated as HF's apply_rotary_pos_emb rotates those outputs
    (modeling_mistral.py:51-81, heads of 128 dims).  None when the rows take the modules' own path."""
    ws = _qkv_fusable(attn, _rows(x, attn.q_proj.weight.shape[1]) if hasattr(attn, "q_proj") else 0, x.dtype)
    if ws is None or (cos is not None and (ws[0].shape[0] % 128 or ws[1].shape[0] % 128)):
        return None
    Z = ws[0].shape[1]
    return batched_qkv(x.reshape(-1, Z), *ws, cos, sin)


def _qkv_fusable(attn: nn.Module, rows: int, dtype):
    """The (q, k, v) weights of a fused q/k/v patch when `rows` decode rows of `dtype` run as one batched launch
    (every projection sends them to the batched kernel), else None."""
    if not getattr(attn, "_teal_qkv_fused", False) or dtype != torch.float16:
        return None
    q, k, v = attn.q_proj, attn.k_proj, attn.v_proj
    Z = q.weight.shape[1]
    if not all(_skinny_dense(rows, p.weight.shape[0], Z) for p in (q, k, v)):
        return None
    return q.weight, k.weight, v.weight


def remove_teal(model):
    """Remove TEAL hooks and restore patched forwards (weights stay column-major)."""
    if hasattr(model, "_teal_hooks"):
        for h in model._teal_hooks:
            h.remove()
        model._teal_hooks.clear()
    if hasattr(model, "_teal_sparsifiers"):
        del model._teal_sparsifiers
    try:
        layers = _get_layers(model)
    except ValueError:
        return
    for layer in layers:
        mods = [_get_projection(layer, p) for p in PROJ_NAMES] + [layer.mlp]
        if hasattr(layer.self_attn, "_teal_qkv_fused"):
            del layer.self_attn._teal_qkv_fused
        for m in mods:
            if hasattr(m, "_teal_original_forward"):
                m.forward = m._teal_original_forward
                del m._teal_original_forward
                for a in ("_teal_patched", "_teal_fused"):
                    if hasattr(m, a):
                        delattr(m, a)


def get_sparsity_report(model) -> dict:
    if not hasattr(model, "_teal_sparsifiers"):
        return {}
    return {k: sf.last_sparsity for k, sf in model._teal_sparsifiers.items()}


def print_sparsity_report(model):
    report = get_sparsity_report(model)
    if not report:
        print("No TEAL sparsifiers found on model.")
        return
    by_layer: dict = {}
    for (li, pn), s in report.items():
        by_layer.setdefault(li, {})[pn] = s
    print("%-8s" % "Layer" + "".join("%-12s" % p for p in PROJ_NAMES) + "%-8s" % "Avg")
    print("-" * (8 + 12 * 7 + 8))
    for li in sorted(by_layer):
        vals = [by_layer[li].get(p, 0.0) for p in PROJ_NAMES]
        print("%-8d" % li + "".join("%10.1f%%  " % (100 * v) for v in vals) + "%6.1f%%" % (100 * sum(vals) / len(vals)))


def _collect_input_activations(model, target_module, data_samples):
    """Inputs seen by target_module over up to 10 calibration samples (CPU copies)."""
    acts = []

    def hook_fn(module, args):
        acts.append(args[0].detach().cpu())

    handle = target_module.register_forward_pre_hook(hook_fn)
    try:
        for sample in data_samples[:10]:
            with torch.no_grad():
                model(sample.to(model.device))
    finally:
        handle.remove()
    return torch.cat(acts, dim=0)

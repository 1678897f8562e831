"""torch-facing wrappers of the leankv_amd HIP kernels (GPU only, no fallback).

Each wrapper validates dtypes/shapes/devices, takes raw device pointers and
the current HIP stream from torch, and calls one C entry point of
``libleankv_amd.so``.  ``*_out`` variants write into caller-owned buffers so
that a decode step can be captured in a HIP graph without allocations.

The functions are also registered as torch custom ops under the ``leankv``
namespace (``torch.ops.leankv.sparse_gemv`` ...) for callers that go through
the dispatcher; the Python entry points below skip the dispatcher.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from ._lib import LeanKVError, check, dtype_code, ptr, require_cuda, stream_handle, workspaces

HEAD_DIM = 128


def _lib_handle():
    return _lib.load()


# ----------------------------------------------------------------- TEAL GEMV
def colmajor_rows(weight: torch.Tensor) -> tuple[int, int]:
    """(N, Z) of a weight W[N, Z] stored column-major (strides (1, N))."""
    if weight.dim() != 2:
        raise LeanKVError("sparse_gemv: weight must be 2-D [N, Z], got %s" % (tuple(weight.shape),))
    N, Z = weight.shape
    if not weight.t().is_contiguous():
        raise LeanKVError(
            "sparse_gemv: weight must be column-major (strides (1, N)) as produced by "
            "prepare_weight_for_sparse_gemv; got strides %s" % (weight.stride(),)
        )
    return N, Z


def _check_x(x: torch.Tensor, Z: int, what: str) -> torch.Tensor:
    if x.dtype != torch.float16:
        raise LeanKVError("%s: x must be float16, got %s" % (what, x.dtype))
    if x.numel() != Z:
        raise LeanKVError("%s: x has %d elements, weight expects Z=%d" % (what, x.numel(), Z))
    return x.reshape(Z).contiguous()


def sparse_gemv_out(x: torch.Tensor, weight: torch.Tensor, threshold: float, out: torch.Tensor) -> torch.Tensor:
    """out[N] = W @ (x * (|x| > threshold)) with W[N, Z] column-major, fp32 accumulate."""
    N, Z = colmajor_rows(weight)
    require_cuda(x, weight, out)
    xf = _check_x(x, Z, "sparse_gemv")
    if weight.dtype != torch.float16 or out.dtype != torch.float16:
        raise LeanKVError("sparse_gemv: weight and out must be float16")
    if out.numel() != N or not out.is_contiguous():
        raise LeanKVError("sparse_gemv: out must be a contiguous float16 tensor of %d elements" % N)
    lib = _lib_handle()
    nbytes = lib.lkv_sparse_gemv_workspace_bytes(N, Z)
    ws = workspaces.get(x.device, "gemv", nbytes)
    check(
        lib.lkv_sparse_gemv(ptr(xf), ptr(weight), float(threshold), N, Z, ptr(out), ptr(ws), ws.numel(),
                            stream_handle(x.device)),
        "lkv_sparse_gemv",
    )
    return out


def sparse_gemv(x: torch.Tensor, weight: torch.Tensor, threshold: float) -> torch.Tensor:
    N, _ = colmajor_rows(weight)
    out = torch.empty(N, dtype=torch.float16, device=x.device)
    return sparse_gemv_out(x, weight, threshold, out)


def sparse_gemm_batched_out(x: torch.Tensor, weight: torch.Tensor, threshold: float, out: torch.Tensor) -> torch.Tensor:
    """out[b] = W @ (x[b] * (|x[b]| > threshold)) for every row b of x[B, Z]; W[N, Z] column-major."""
    N, Z = colmajor_rows(weight)
    require_cuda(x, weight, out)
    if x.dtype != torch.float16 or weight.dtype != torch.float16 or out.dtype != torch.float16:
        raise LeanKVError("sparse_gemm_batched: x, weight and out must be float16")
    if x.dim() != 2 or x.shape[1] != Z or not x.is_contiguous():
        raise LeanKVError("sparse_gemm_batched: x must be a contiguous float16 [B, %d] tensor" % Z)
    B = x.shape[0]
    if tuple(out.shape) != (B, N) or not out.is_contiguous():
        raise LeanKVError("sparse_gemm_batched: out must be a contiguous float16 [%d, %d] tensor" % (B, N))
    lib = _lib_handle()
    nbytes = lib.lkv_sparse_gemm_batched_workspace_bytes(B, N, Z)
    ws = workspaces.get(x.device, "gemm_b", nbytes)
    check(
        lib.lkv_sparse_gemm_batched(ptr(x), ptr(weight), float(threshold), B, N, Z, ptr(out), ptr(ws), ws.numel(),
                                    stream_handle(x.device)),
        "lkv_sparse_gemm_batched",
    )
    return out


def sparse_gemm_batched(x: torch.Tensor, weight: torch.Tensor, threshold: float) -> torch.Tensor:
    N, _ = colmajor_rows(weight)
    out = torch.empty(x.shape[0], N, dtype=torch.float16, device=x.device)
    return sparse_gemm_batched_out(x, weight, threshold, out)


EPI_NONE, EPI_SWIGLU, EPI_RESIDUAL, EPI_ROPE = 0, 1, 2, 3


def sparse_gemm_batched_multi_out(x: torch.Tensor, weights, thresholds, outs, epilogue: int = EPI_NONE,
                                  residual: torch.Tensor | None = None, cos: torch.Tensor | None = None,
                                  sin: torch.Tensor | None = None):
    """Up to 3 sparse_gemm_batched products of one x[B, Z] in one launch (lkv_sparse_gemm_batched_multi), each
    equal to its own sparse_gemm_batched call, with an epilogue in the reduce: EPI_NONE (outs[s] = product s),
    EPI_SWIGLU (two products g, u of one shape: outs[0] = fp16(fp16(silu(fp16 g)) * fp16 u)), EPI_RESIDUAL
    (one product: outs[0] = fp16(residual + fp16 product); outs[0] may be residual) or EPI_ROPE (q, k[, v]:
    rope_f16_ on the first two products' heads of 128 dims with the position's fp16 factors cos / sin [128])."""
    import ctypes

    n = len(weights)
    if not 1 <= n <= 3 or len(thresholds) != n:
        raise LeanKVError("sparse_gemm_batched_multi: 1 to 3 weights with one threshold each")
    shapes = [colmajor_rows(w) for w in weights]
    Z = shapes[0][1]
    if any(z != Z for _, z in shapes):
        raise LeanKVError("sparse_gemm_batched_multi: weights of different input sizes %s" % (shapes,))
    n_out = 1 if epilogue == EPI_SWIGLU else n
    if len(outs) != n_out:
        raise LeanKVError("sparse_gemm_batched_multi: %d outputs expected, got %d" % (n_out, len(outs)))
    require_cuda(x, *weights, *outs, residual)
    if x.dtype != torch.float16 or any(t.dtype != torch.float16 for t in (*weights, *outs)):
        raise LeanKVError("sparse_gemm_batched_multi: x, weights and outputs must be float16")
    if x.dim() != 2 or x.shape[1] != Z or not x.is_contiguous():
        raise LeanKVError("sparse_gemm_batched_multi: x must be a contiguous float16 [B, %d] tensor" % Z)
    B = x.shape[0]
    for o, (N, _) in zip(outs, shapes):
        if tuple(o.shape) != (B, N) or not o.is_contiguous():
            raise LeanKVError("sparse_gemm_batched_multi: outputs must be contiguous float16 [%d, %d]" % (B, N))
    if epilogue == EPI_RESIDUAL:
        if residual is None or residual.dtype != torch.float16 or tuple(residual.shape) != (B, shapes[0][0]) \
                or not residual.is_contiguous():
            raise LeanKVError("sparse_gemm_batched_multi: residual must be a contiguous float16 [%d, %d] tensor"
                              % (B, shapes[0][0]))
    elif residual is not None:
        raise LeanKVError("sparse_gemm_batched_multi: a residual needs the residual epilogue")
    if epilogue == EPI_ROPE:
        require_cuda(cos, sin)
        for f in (cos, sin):
            if f is None or f.dtype != torch.float16 or f.numel() != HEAD_DIM or not f.is_contiguous():
                raise LeanKVError("sparse_gemm_batched_multi: RoPE needs contiguous float16 cos / sin of %d"
                                  % HEAD_DIM)
    elif cos is not None or sin is not None:
        raise LeanKVError("sparse_gemm_batched_multi: RoPE factors need the RoPE epilogue")
    lib = _lib_handle()
    n_arr = (ctypes.c_int64 * n)(*[N for N, _ in shapes])
    nbytes = lib.lkv_sparse_gemm_batched_multi_workspace_bytes(B, n, n_arr, Z)
    ws = workspaces.get(x.device, "gemm_bm", nbytes)
    check(
        lib.lkv_sparse_gemm_batched_multi(ptr(x), B, n, (ctypes.c_void_p * n)(*[ptr(w) for w in weights]),
                                          (ctypes.c_float * n)(*[float(t) for t in thresholds]), n_arr, Z,
                                          int(epilogue), ptr(residual), ptr(cos), ptr(sin),
                                          (ctypes.c_void_p * n_out)(*[ptr(o) for o in outs]), ptr(ws), ws.numel(),
                                          stream_handle(x.device)),
        "lkv_sparse_gemm_batched_multi",
    )
    return outs


def sparse_gemm_batched_residual_rmsnorm_out(x: torch.Tensor, weight: torch.Tensor, threshold: float,
                                             residual: torch.Tensor, norm_w: torch.Tensor, eps: float,
                                             x_out: torch.Tensor, y_out: torch.Tensor):
    """x_out = fp16(residual + fp16(sparse_gemm_batched(x, weight, threshold))), y_out = rms_norm(x_out, norm_w,
    eps), in one product launch and one epilogue launch (lkv_sparse_gemm_batched_residual_rmsnorm); x_out may be
    residual.  Both equal the separate calls bit for bit."""
    N, Z = colmajor_rows(weight)
    require_cuda(x, weight, residual, norm_w, x_out, y_out)
    ts = (x, weight, residual, norm_w, x_out, y_out)
    if any(t.dtype != torch.float16 for t in ts):
        raise LeanKVError("sparse_gemm_batched_residual_rmsnorm: every tensor must be float16")
    if x.dim() != 2 or x.shape[1] != Z or not x.is_contiguous():
        raise LeanKVError("sparse_gemm_batched_residual_rmsnorm: x must be a contiguous float16 [B, %d] tensor" % Z)
    B = x.shape[0]
    for t in (residual, x_out, y_out):
        if tuple(t.shape) != (B, N) or not t.is_contiguous():
            raise LeanKVError("sparse_gemm_batched_residual_rmsnorm: residual and outputs must be contiguous "
                              "[%d, %d]" % (B, N))
    if norm_w.numel() != N or not norm_w.is_contiguous():
        raise LeanKVError("sparse_gemm_batched_residual_rmsnorm: norm weight of %d elements expected" % N)
    lib = _lib_handle()
    nbytes = lib.lkv_sparse_gemm_batched_workspace_bytes(B, N, Z)
    ws = workspaces.get(x.device, "gemm_bn", nbytes)
    check(lib.lkv_sparse_gemm_batched_residual_rmsnorm(ptr(x), ptr(weight), float(threshold), B, N, Z, ptr(residual),
                                                       ptr(norm_w), float(eps), ptr(x_out), ptr(y_out), ptr(ws),
                                                       ws.numel(), stream_handle(x.device)),
          "lkv_sparse_gemm_batched_residual_rmsnorm")
    return x_out, y_out


def sparse_gemm_batched_qkv_rope_out(x: torch.Tensor, weights, cos: torch.Tensor, sin: torch.Tensor, outs,
                                     k_hot: torch.Tensor | None = None, v_hot: torch.Tensor | None = None,
                                     pos_dev: torch.Tensor | None = None):
    """q, k, v = the three threshold-0 products of x[B, Z] with RoPE on q and k (sparse_gemm_batched_multi_out with
    EPI_ROPE), and with k_hot / v_hot [B * Hkv, hot_cap, 128] the new token of every row also written into ring
    slot pos % hot_cap (pos_dev: int32 device position), as lkv_tq_cache_append writes it
    (lkv_sparse_gemm_batched_qkv_rope)."""
    import ctypes

    if len(weights) != 3 or len(outs) != 3:
        raise LeanKVError("sparse_gemm_batched_qkv_rope: q, k and v weights and outputs")
    shapes = [colmajor_rows(w) for w in weights]
    Z = shapes[0][1]
    B = x.shape[0] if x.dim() == 2 else -1
    require_cuda(x, *weights, *outs, cos, sin, k_hot, v_hot, pos_dev)
    if x.dtype != torch.float16 or any(t.dtype != torch.float16 for t in (*weights, *outs, cos, sin)):
        raise LeanKVError("sparse_gemm_batched_qkv_rope: x, weights, outputs and RoPE factors must be float16")
    if x.dim() != 2 or x.shape[1] != Z or not x.is_contiguous() or any(z != Z for _, z in shapes):
        raise LeanKVError("sparse_gemm_batched_qkv_rope: x must be a contiguous float16 [B, %d] tensor" % Z)
    for o, (N, _) in zip(outs, shapes):
        if tuple(o.shape) != (B, N) or not o.is_contiguous():
            raise LeanKVError("sparse_gemm_batched_qkv_rope: outputs must be contiguous float16 [%d, %d]" % (B, N))
    for f in (cos, sin):
        if f.numel() != HEAD_DIM or not f.is_contiguous():
            raise LeanKVError("sparse_gemm_batched_qkv_rope: cos / sin must be contiguous, %d each" % HEAD_DIM)
    hot_cap = 1
    if k_hot is not None or v_hot is not None:
        if k_hot is None or v_hot is None or pos_dev is None or pos_dev.dtype != torch.int32:
            raise LeanKVError("sparse_gemm_batched_qkv_rope: k_hot, v_hot and an int32 position go together")
        hot_cap = k_hot.shape[-2]
        rows = B * shapes[1][0] // HEAD_DIM
        for t in (k_hot, v_hot):
            if t.dtype != torch.float16 or not t.is_contiguous() or t.numel() != rows * hot_cap * HEAD_DIM:
                raise LeanKVError("sparse_gemm_batched_qkv_rope: rings must be contiguous float16 [%d, %d, %d]"
                                  % (rows, hot_cap, HEAD_DIM))
    lib = _lib_handle()
    n_arr = (ctypes.c_int64 * 3)(*[N for N, _ in shapes])
    nbytes = lib.lkv_sparse_gemm_batched_multi_workspace_bytes(B, 3, n_arr, Z)
    ws = workspaces.get(x.device, "gemm_bm", nbytes)
    check(lib.lkv_sparse_gemm_batched_qkv_rope(ptr(x), B, (ctypes.c_void_p * 3)(*[ptr(w) for w in weights]),
                                               (ctypes.c_float * 3)(0.0, 0.0, 0.0), n_arr, Z, ptr(cos), ptr(sin),
                                               (ctypes.c_void_p * 3)(*[ptr(o) for o in outs]), ptr(k_hot),
                                               ptr(v_hot), ptr(pos_dev), hot_cap, ptr(ws), ws.numel(),
                                               stream_handle(x.device)),
          "lkv_sparse_gemm_batched_qkv_rope")
    return outs


def sparse_gemm_batched_multi(x: torch.Tensor, weights, thresholds, epilogue: int = EPI_NONE,
                              residual: torch.Tensor | None = None, cos: torch.Tensor | None = None,
                              sin: torch.Tensor | None = None):
    """sparse_gemm_batched_multi_out into fresh outputs (the list of them)."""
    N = [colmajor_rows(w)[0] for w in weights]
    outs = [torch.empty(x.shape[0], n, dtype=torch.float16, device=x.device)
            for n in (N[:1] if epilogue in (EPI_SWIGLU, EPI_RESIDUAL) else N)]
    return sparse_gemm_batched_multi_out(x, weights, thresholds, outs, epilogue, residual, cos, sin)


def sparse_gemv_partials(x: torch.Tensor, w_gate: torch.Tensor, t_gate: float, w_up: torch.Tensor | None = None,
                         t_up: float = 0.0, out: torch.Tensor | None = None) -> torch.Tensor:
    """Split-K partial sums only: fp32 [mats, N/256 slabs, chunks, 256] (mats = 2 with w_up).

    Summing dim 2 in chunk order and rounding to fp16 reproduces sparse_gemv
    (or, through SwiGLU, sparse_gateup_swiglu) bit for bit."""
    N, Z = colmajor_rows(w_gate)
    if w_up is not None and (colmajor_rows(w_up) != (N, Z) or w_up.dtype != torch.float16):
        raise LeanKVError("sparse_gemv_partials: up weight must match the gate weight")
    require_cuda(x, w_gate, w_up)
    xf = _check_x(x, Z, "sparse_gemv_partials")
    if w_gate.dtype != torch.float16:
        raise LeanKVError("sparse_gemv_partials: weights must be float16")
    lib = _lib_handle()
    shape = (2 if w_up is not None else 1, (N + 255) // 256, lib.lkv_sparse_gemv_chunks(N, Z), 256)
    if out is None:
        out = torch.empty(shape, dtype=torch.float32, device=x.device)
    if tuple(out.shape) != shape or out.dtype != torch.float32 or not out.is_contiguous():
        raise LeanKVError("sparse_gemv_partials: out must be a contiguous float32 tensor of shape %s" % (shape,))
    check(lib.lkv_sparse_gemv_partials(ptr(xf), ptr(w_gate), ptr(w_up), float(t_gate), float(t_up), N, Z, ptr(out),
                                       out.numel() * 4, stream_handle(x.device)), "lkv_sparse_gemv_partials")
    return out


def sparse_gateup_swiglu_out(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, t_gate: float,
                             t_up: float, out: torch.Tensor) -> torch.Tensor:
    """out[N] = fp16(silu(fp16(Wg x_g)) * fp16(Wu x_u)), x_g/x_u thresholded copies of x."""
    N, Z = colmajor_rows(w_gate)
    if tuple(w_up.shape) != (N, Z):
        raise LeanKVError("sparse_gateup_swiglu: gate/up weight shapes differ")
    colmajor_rows(w_up)
    require_cuda(x, w_gate, w_up, out)
    xf = _check_x(x, Z, "sparse_gateup_swiglu")
    if w_gate.dtype != torch.float16 or w_up.dtype != torch.float16 or out.dtype != torch.float16:
        raise LeanKVError("sparse_gateup_swiglu: weights and out must be float16")
    if out.numel() != N or not out.is_contiguous():
        raise LeanKVError("sparse_gateup_swiglu: out must be contiguous with %d elements" % N)
    lib = _lib_handle()
    nbytes = lib.lkv_sparse_gateup_workspace_bytes(N, Z)
    ws = workspaces.get(x.device, "gateup", nbytes)
    check(
        lib.lkv_sparse_gateup_swiglu(ptr(xf), ptr(w_gate), ptr(w_up), float(t_gate), float(t_up), N, Z,
                                     ptr(out), ptr(ws), ws.numel(), stream_handle(x.device)),
        "lkv_sparse_gateup_swiglu",
    )
    return out


def sparse_gateup_swiglu(x, w_gate, w_up, t_gate, t_up):
    N, _ = colmajor_rows(w_gate)
    out = torch.empty(N, dtype=torch.float16, device=x.device)
    return sparse_gateup_swiglu_out(x, w_gate, w_up, t_gate, t_up, out)


def sparse_qkv(x: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor, wv: torch.Tensor, tq: float, tk: float,
               tv: float, out: tuple | None = None):
    """(q, k, v) = three TEAL sparse GEMVs of one x (column-major weights [N_s, Z]) in one launch that reads x
    once; each equals the fused decode step's projection bit for bit."""
    ws_ = (wq, wk, wv)
    shapes = [colmajor_rows(w) for w in ws_]
    Z = shapes[0][1]
    if any(z != Z for _, z in shapes):
        raise LeanKVError("sparse_qkv: weights must share Z")
    require_cuda(x, *ws_)
    xf = _check_x(x, Z, "sparse_qkv")
    if any(w.dtype != torch.float16 for w in ws_):
        raise LeanKVError("sparse_qkv: weights must be float16")
    Ns = [n for n, _ in shapes]
    if out is None:
        out = tuple(torch.empty(n, dtype=torch.float16, device=x.device) for n in Ns)
    for o, n in zip(out, Ns):
        if o.dtype != torch.float16 or o.numel() != n or not o.is_contiguous():
            raise LeanKVError("sparse_qkv: outputs must be contiguous float16 with %s elements" % (Ns,))
    lib = _lib_handle()
    import ctypes

    n_arr = (ctypes.c_int64 * 3)(*Ns)
    nbytes = lib.lkv_sparse_gemv_multi_workspace_bytes(3, n_arr, Z)
    ws = workspaces.get(x.device, "qkv", nbytes)
    check(
        lib.lkv_sparse_gemv_multi(ptr(xf), 3, (ctypes.c_void_p * 3)(*[ptr(w) for w in ws_]),
                                  (ctypes.c_float * 3)(float(tq), float(tk), float(tv)), n_arr, Z,
                                  (ctypes.c_void_p * 3)(*[ptr(o) for o in out]), ptr(ws), ws.numel(),
                                  stream_handle(x.device)),
        "lkv_sparse_gemv_multi",
    )
    return tuple(out)


# ----------------------------------------------------------------- TurboQuant
def packed_row_bytes(bits: int) -> int:
    n = _lib_handle().lkv_tq_packed_row_bytes(int(bits))
    if n < 0:
        raise LeanKVError("TurboQuant: bits=%d cannot be bit-packed (1..4 supported)" % bits)
    return n


def _rows(x: torch.Tensor, what: str) -> int:
    if x.shape[-1] != HEAD_DIM:
        raise LeanKVError("%s: last dim must be %d, got %d" % (what, HEAD_DIM, x.shape[-1]))
    return x.numel() // HEAD_DIM


def _pi(Pi: torch.Tensor, device) -> torch.Tensor:
    """Row-major fp32 [128, 128] on `device` (no copy when it already is).

    torch.linalg.qr returns Q column-major, so a rotation built from it must be
    made contiguous before its pointer reaches a kernel.
    """
    if tuple(Pi.shape) != (HEAD_DIM, HEAD_DIM):
        raise LeanKVError("TurboQuant: rotation must be [128, 128], got %s" % (tuple(Pi.shape),))
    return Pi.to(device=device, dtype=torch.float32).contiguous()


def _vec(t: torch.Tensor, device, n: int | None = None, what: str = "table") -> torch.Tensor:
    v = t.to(device=device, dtype=torch.float32).contiguous()
    if n is not None and v.numel() != n:
        raise LeanKVError("TurboQuant: %s must have %d entries, got %d" % (what, n, v.numel()))
    return v


def tq_quantize(x: torch.Tensor, Pi: torch.Tensor, bounds: torch.Tensor, bits: int):
    """Fused norm / normalise / rotate (fp32 MFMA) / searchsorted / pack."""
    require_cuda(x)
    M = _rows(x, "tq_quantize")
    xc = x.contiguous()
    lib = _lib_handle()
    rb = packed_row_bytes(bits)
    packed = torch.empty(*x.shape[:-1], rb, dtype=torch.uint8, device=x.device)
    norms = torch.empty(x.shape[:-1], dtype=x.dtype, device=x.device)
    b = bounds.to(device=x.device, dtype=torch.float32).contiguous()
    if b.numel() != (1 << bits) - 1:
        raise LeanKVError("tq_quantize: %d decision boundaries for bits=%d" % (b.numel(), bits))
    Pc = _pi(Pi, x.device)  # held until the call returns: a temporary's memory could be reused
    check(
        lib.lkv_tq_quantize(ptr(xc), dtype_code(x.dtype), M, ptr(Pc), ptr(b), int(bits),
                            ptr(packed), ptr(norms), stream_handle(x.device)),
        "lkv_tq_quantize",
    )
    return packed, norms


def tq_quantize_rotated(y: torch.Tensor, bounds: torch.Tensor, bits: int) -> torch.Tensor:
    require_cuda(y)
    if y.dtype != torch.float32:
        raise LeanKVError("tq_quantize_rotated: y must be float32")
    M = _rows(y, "tq_quantize_rotated")
    yc = y.contiguous()
    packed = torch.empty(*y.shape[:-1], packed_row_bytes(bits), dtype=torch.uint8, device=y.device)
    b = bounds.to(device=y.device, dtype=torch.float32).contiguous()
    check(
        _lib_handle().lkv_tq_quantize_rotated(ptr(yc), M, ptr(b), int(bits), ptr(packed), stream_handle(y.device)),
        "lkv_tq_quantize_rotated",
    )
    return packed


def tq_dequantize(packed: torch.Tensor, norms: torch.Tensor, Pi: torch.Tensor, centroids: torch.Tensor,
                  bits: int, out_dtype: torch.dtype = torch.float32, out: torch.Tensor | None = None):
    require_cuda(packed, norms)
    rb = packed_row_bytes(bits)
    if packed.dtype != torch.uint8 or packed.shape[-1] != rb:
        raise LeanKVError("tq_dequantize: packed must be uint8 [..., %d]" % rb)
    M = packed.numel() // rb
    if norms.numel() != M:
        raise LeanKVError("tq_dequantize: %d norms for %d rows" % (norms.numel(), M))
    pc = packed.contiguous()
    nc = norms.contiguous()
    if out is None:
        out = torch.empty(*packed.shape[:-1], HEAD_DIM, dtype=out_dtype, device=packed.device)
    c = centroids.to(device=packed.device, dtype=torch.float32).contiguous()
    Pc = _pi(Pi, packed.device)
    check(
        _lib_handle().lkv_tq_dequantize(ptr(pc), ptr(nc), dtype_code(nc.dtype), M, ptr(Pc),
                                        ptr(c), int(bits), ptr(out), dtype_code(out.dtype),
                                        stream_handle(packed.device)),
        "lkv_tq_dequantize",
    )
    return out


def tq_rotate(x: torch.Tensor, Pi: torch.Tensor, transpose: bool = False) -> torch.Tensor:
    """x @ Pi^T (transpose=False, rotate_forward) or x @ Pi (rotate_backward), fp32 out."""
    require_cuda(x)
    M = _rows(x, "tq_rotate")
    xc = x.contiguous()
    y = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    Pc = _pi(Pi, x.device)
    check(
        _lib_handle().lkv_tq_rotate(ptr(xc), dtype_code(x.dtype), M, ptr(Pc), int(bool(transpose)),
                                    ptr(y), stream_handle(x.device)),
        "lkv_tq_rotate",
    )
    return y


def tq_prod_quantize(x: torch.Tensor, Pi: torch.Tensor, bounds: torch.Tensor, centroids: torch.Tensor,
                     S: torch.Tensor, mse_bits: int):
    """TurboQuantProd quantize in one launch: MSE codes at mse_bits, norms (x's dtype), the packed signs of
    (x - x_hat) @ S^T ([..., 16] uint8) and the residual norms (fp32)."""
    require_cuda(x)
    M = _rows(x, "tq_prod_quantize")
    rb = packed_row_bytes(mse_bits)
    xc = x.contiguous()
    b = _vec(bounds, x.device, (1 << mse_bits) - 1, "decision boundaries")
    c = _vec(centroids, x.device, 1 << mse_bits, "centroids")
    codes = torch.empty(*x.shape[:-1], rb, dtype=torch.uint8, device=x.device)
    norms = torch.empty(x.shape[:-1], dtype=x.dtype, device=x.device)
    signs = torch.empty(*x.shape[:-1], HEAD_DIM // 8, dtype=torch.uint8, device=x.device)
    rnorms = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    Pc, Sc = _pi(Pi, x.device), _pi(S, x.device)  # both alive until the call returns
    check(
        _lib_handle().lkv_tq_prod_quantize(ptr(xc), dtype_code(x.dtype), M, ptr(Pc), ptr(b), ptr(c),
                                           ptr(Sc), int(mse_bits), ptr(codes), ptr(norms), ptr(signs),
                                           ptr(rnorms), stream_handle(x.device)),
        "lkv_tq_prod_quantize",
    )
    return codes, norms, signs, rnorms


def tq_prod_dequantize(codes: torch.Tensor, norms: torch.Tensor, signs: torch.Tensor, rnorms: torch.Tensor,
                       Pi: torch.Tensor, centroids: torch.Tensor, S: torch.Tensor, mse_bits: int, qjl_scale: float,
                       out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """(centroid[codes] @ Pi) * norm + (signs @ S) * (qjl_scale * rnorm) in one launch."""
    require_cuda(codes, norms, signs, rnorms)
    rb = packed_row_bytes(mse_bits)
    if codes.dtype != torch.uint8 or codes.shape[-1] != rb:
        raise LeanKVError("tq_prod_dequantize: codes must be uint8 [..., %d]" % rb)
    M = codes.numel() // rb
    if signs.dtype != torch.uint8 or signs.numel() != M * (HEAD_DIM // 8):
        raise LeanKVError("tq_prod_dequantize: signs must be uint8 [..., %d] for %d rows" % (HEAD_DIM // 8, M))
    if norms.numel() != M or rnorms.numel() != M:
        raise LeanKVError("tq_prod_dequantize: %d norms / %d residual norms for %d rows"
                          % (norms.numel(), rnorms.numel(), M))
    nc = norms.contiguous()
    rn = rnorms.to(torch.float32).contiguous()
    c = _vec(centroids, codes.device, 1 << mse_bits, "centroids")
    out = torch.empty(*codes.shape[:-1], HEAD_DIM, dtype=out_dtype, device=codes.device)
    cc, sc = codes.contiguous(), signs.contiguous()
    Pc, Sc = _pi(Pi, codes.device), _pi(S, codes.device)
    check(
        _lib_handle().lkv_tq_prod_dequantize(ptr(cc), ptr(nc), dtype_code(nc.dtype),
                                             ptr(sc), ptr(rn), M, ptr(Pc), ptr(c),
                                             ptr(Sc), int(mse_bits), float(qjl_scale), ptr(out),
                                             dtype_code(out.dtype), stream_handle(codes.device)),
        "lkv_tq_prod_dequantize",
    )
    return out


def tq_cache_append(k_new, v_new, k_hot, v_hot, k_codes, k_norms, v_codes, v_norms, PiK, PiV, bounds, bits,
                    pos_dev) -> None:
    """Decode-step append on the static ring layout (see include/leankv_amd.h)."""
    require_cuda(k_new, v_new, k_hot, v_hot, k_codes, v_codes, pos_dev)
    R = k_new.numel() // HEAD_DIM
    hot_cap = k_hot.shape[-2]
    cap = k_codes.shape[-2]
    for t, nm in ((k_new, "k_new"), (v_new, "v_new"), (k_hot, "k_hot"), (v_hot, "v_hot")):
        if t.dtype != torch.float16 or not t.is_contiguous():
            raise LeanKVError("tq_cache_append: %s must be contiguous float16" % nm)
    if k_hot.numel() != R * hot_cap * HEAD_DIM or k_codes.numel() != R * cap * packed_row_bytes(bits):
        raise LeanKVError("tq_cache_append: buffer shapes disagree with %d rows" % R)
    if pos_dev.dtype != torch.int32:
        raise LeanKVError("tq_cache_append: pos must be an int32 device tensor")
    for t, nm in ((k_norms, "k_norms"), (v_norms, "v_norms")):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != R * cap:
            raise LeanKVError("tq_cache_append: %s must be contiguous float32 [R, cap]" % nm)
    if not (k_codes.is_contiguous() and v_codes.is_contiguous()) or v_codes.shape != k_codes.shape:
        raise LeanKVError("tq_cache_append: code stores must be contiguous and alike")
    dev = k_new.device
    PiK, PiV = _pi(PiK, dev), _pi(PiV, dev)
    bounds = _vec(bounds, dev, (1 << bits) - 1, "decision boundaries")
    check(
        _lib_handle().lkv_tq_cache_append(ptr(k_new), ptr(v_new), ptr(k_hot), ptr(v_hot), ptr(k_codes),
                                          ptr(k_norms), ptr(v_codes), ptr(v_norms), ptr(PiK), ptr(PiV),
                                          ptr(bounds), int(bits), ptr(pos_dev), R, hot_cap, cap,
                                          stream_handle(dev)),
        "lkv_tq_cache_append",
    )


def tq_cache_evict(layers, bounds, bits: int, pos_dev: torch.Tensor) -> None:
    """The eviction half of tq_cache_append for every layer in one launch (lkv_tq_cache_evict): layers is a list
    of (k_codes, k_norms, v_codes, v_norms, k_hot, v_hot, PiK, PiV) on the static ring layout, R = B x kv heads
    rows each; the token at position pos_dev - hot_cap leaves ring slot pos_dev % hot_cap for cold slot
    pos_dev - hot_cap.  Run before the step's ring write."""
    import ctypes

    class _Layer(ctypes.Structure):
        _fields_ = [(n, ctypes.c_void_p) for n in ("k_codes", "k_norms", "v_codes", "v_norms", "k_hot", "v_hot",
                                                   "PiK", "PiV")]

    if not layers:
        return
    if pos_dev.dtype != torch.int32:
        raise LeanKVError("tq_cache_evict: pos must be an int32 device tensor")
    k_hot0, k_codes0 = layers[0][4], layers[0][0]
    hot_cap, cap = k_hot0.shape[-2], k_codes0.shape[-2]
    R = k_hot0.numel() // (hot_cap * HEAD_DIM)
    rb = packed_row_bytes(bits)
    dev = k_hot0.device
    arr = (_Layer * len(layers))()
    keep = []
    for i, (kc, kn, vc, vn, kh, vh, PiK, PiV) in enumerate(layers):
        require_cuda(kc, kn, vc, vn, kh, vh, pos_dev)
        for t, nm in ((kh, "k_hot"), (vh, "v_hot")):
            if t.dtype != torch.float16 or not t.is_contiguous() or t.numel() != R * hot_cap * HEAD_DIM:
                raise LeanKVError("tq_cache_evict: %s of layer %d must be contiguous float16 [%d, %d, %d]"
                                  % (nm, i, R, hot_cap, HEAD_DIM))
        for t, nm in ((kc, "k_codes"), (vc, "v_codes")):
            if t.dtype != torch.uint8 or not t.is_contiguous() or t.numel() != R * cap * rb:
                raise LeanKVError("tq_cache_evict: %s of layer %d must be contiguous uint8 [%d, %d, %d]"
                                  % (nm, i, R, cap, rb))
        for t, nm in ((kn, "k_norms"), (vn, "v_norms")):
            if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != R * cap:
                raise LeanKVError("tq_cache_evict: %s of layer %d must be contiguous float32 [%d, %d]"
                                  % (nm, i, R, cap))
        pk, pv = _pi(PiK, dev), _pi(PiV, dev)
        keep += [pk, pv]
        arr[i] = _Layer(ptr(kc), ptr(kn), ptr(vc), ptr(vn), ptr(kh), ptr(vh), ptr(pk), ptr(pv))
    bd = _vec(bounds, dev, (1 << bits) - 1, "decision boundaries")
    check(_lib_handle().lkv_tq_cache_evict(arr, len(layers), R, hot_cap, cap, ptr(bd), int(bits), ptr(pos_dev),
                                           stream_handle(dev)), "lkv_tq_cache_evict")


def _check_code_rows(k_codes: torch.Tensor, v_codes: torch.Tensor, bits: int, what: str) -> None:
    rb = packed_row_bytes(bits)
    for t, nm in ((k_codes, "k_codes"), (v_codes, "v_codes")):
        if t.dtype != torch.uint8 or t.shape[-1] != rb:
            raise LeanKVError("%s: %s must be uint8 rows of %d bytes at %d bits, got %s %s"
                              % (what, nm, rb, bits, t.dtype, tuple(t.shape)))


def decode_attn_workspace_bytes(B: int, Hq: int, Hkv: int, max_len: int) -> int:
    return int(_lib_handle().lkv_tq_decode_attn_workspace_bytes(B, Hq, Hkv, max_len))


def tq_decode_attn_out(q, k_codes, k_norms, v_codes, v_norms, k_hot, v_hot, PiK, PiV, centroids, bits, seq_len_dev,
                       max_len: int, scale: float, out: torch.Tensor, workspace: torch.Tensor | None = None):
    """Single-query GQA attention over the packed cold cache + fp16 hot ring.

    q: fp16 [B, Hq, 128]; codes uint8 [B, Hkv, cap, packed_row_bytes(bits)]; norms fp32 [B, Hkv, cap];
    hot fp16 [B, Hkv, hot_cap, 128] (hot_cap <= 256); seq_len_dev int32 [1] (device); out fp16 [B, Hq, 128].
    """
    require_cuda(q, k_codes, v_codes, k_hot, v_hot, seq_len_dev, out)
    if q.dtype != torch.float16 or q.dim() != 3 or q.shape[-1] != HEAD_DIM or not q.is_contiguous():
        raise LeanKVError("tq_decode_attn: q must be contiguous float16 [B, Hq, 128]")
    B, Hq, _ = q.shape
    Hkv, cap = k_codes.shape[1], k_codes.shape[2]
    hot_cap = k_hot.shape[2]
    if out.shape != q.shape or out.dtype != torch.float16 or not out.is_contiguous():
        raise LeanKVError("tq_decode_attn: out must be contiguous float16 like q")
    for t, nm in ((k_codes, "k_codes"), (v_codes, "v_codes"), (k_norms, "k_norms"), (v_norms, "v_norms"),
                  (k_hot, "k_hot"), (v_hot, "v_hot")):
        if not t.is_contiguous():
            raise LeanKVError("tq_decode_attn: %s must be contiguous" % nm)
    if k_norms.dtype != torch.float32 or v_norms.dtype != torch.float32:
        raise LeanKVError("tq_decode_attn: norms must be float32")
    _check_code_rows(k_codes, v_codes, bits, "tq_decode_attn")
    if k_hot.dtype != torch.float16 or v_hot.dtype != torch.float16:
        raise LeanKVError("tq_decode_attn: hot window must be float16")
    if seq_len_dev.dtype != torch.int32:
        raise LeanKVError("tq_decode_attn: seq_len must be an int32 device tensor")
    dev = q.device
    PiK, PiV = _pi(PiK, dev), _pi(PiV, dev)
    centroids = _vec(centroids, dev, 1 << bits, "centroids")
    lib = _lib_handle()
    nbytes = lib.lkv_tq_decode_attn_workspace_bytes(B, Hq, Hkv, max_len)
    if workspace is None:
        workspace = workspaces.get(q.device, "attn", nbytes)
    check(
        lib.lkv_tq_decode_attn(ptr(q), ptr(k_codes), ptr(k_norms), ptr(v_codes), ptr(v_norms), ptr(k_hot),
                               ptr(v_hot), ptr(PiK), ptr(PiV), ptr(centroids), int(bits), ptr(seq_len_dev),
                               int(max_len), B, Hq, Hkv, cap, hot_cap, float(scale), ptr(out), ptr(workspace),
                               workspace.numel(), stream_handle(q.device)),
        "lkv_tq_decode_attn",
    )
    return out


def tq_decode_attn(q, k_codes, k_norms, v_codes, v_norms, k_hot, v_hot, PiK, PiV, centroids, bits, seq_len_dev,
                   max_len: int, scale: float | None = None):
    out = torch.empty_like(q)
    if scale is None:
        scale = 1.0 / math.sqrt(HEAD_DIM)
    return tq_decode_attn_out(q, k_codes, k_norms, v_codes, v_norms, k_hot, v_hot, PiK, PiV, centroids, bits,
                              seq_len_dev, max_len, scale, out)


def tq_prefill_attn_out(q, k_codes, k_norms, v_codes, v_norms, k_hot, v_hot, PiK, PiV, centroids, bits, kv_len: int,
                        scale: float, out: torch.Tensor, workspace: torch.Tensor | None = None):
    """Causal attention of the newest S tokens' queries over the packed cold cache + fp16 hot ring.

    q: fp16 [B, Hq, S, 128] (post-RoPE, positions kv_len - S ..); codes uint8 [B, Hkv, cap,
    packed_row_bytes(bits)]; norms fp32 [B, Hkv, cap]; hot fp16 [B, Hkv, hot_cap, 128]; out fp16 [B, Hq, S, 128].
    """
    require_cuda(q, k_codes, v_codes, k_hot, v_hot, out)
    if q.dtype != torch.float16 or q.dim() != 4 or q.shape[-1] != HEAD_DIM or not q.is_contiguous():
        raise LeanKVError("tq_prefill_attn: q must be contiguous float16 [B, Hq, S, 128]")
    B, Hq, S, _ = q.shape
    Hkv, cap = k_codes.shape[1], k_codes.shape[2]
    hot_cap = k_hot.shape[2]
    if out.shape != q.shape or out.dtype != torch.float16 or not out.is_contiguous():
        raise LeanKVError("tq_prefill_attn: out must be contiguous float16 like q")
    for t, nm in ((k_codes, "k_codes"), (v_codes, "v_codes"), (k_norms, "k_norms"), (v_norms, "v_norms"),
                  (k_hot, "k_hot"), (v_hot, "v_hot")):
        if not t.is_contiguous():
            raise LeanKVError("tq_prefill_attn: %s must be contiguous" % nm)
    if k_norms.dtype != torch.float32 or v_norms.dtype != torch.float32:
        raise LeanKVError("tq_prefill_attn: norms must be float32")
    _check_code_rows(k_codes, v_codes, bits, "tq_prefill_attn")
    if k_hot.dtype != torch.float16 or v_hot.dtype != torch.float16:
        raise LeanKVError("tq_prefill_attn: hot window must be float16")
    dev = q.device
    PiK, PiV = _pi(PiK, dev), _pi(PiV, dev)
    centroids = _vec(centroids, dev, 1 << bits, "centroids")
    lib = _lib_handle()
    nbytes = lib.lkv_tq_prefill_attn_workspace_bytes(B, Hq, Hkv, S, hot_cap)
    if workspace is None:
        workspace = workspaces.get(q.device, "prefill", nbytes)
    check(
        lib.lkv_tq_prefill_attn(ptr(q), ptr(k_codes), ptr(k_norms), ptr(v_codes), ptr(v_norms), ptr(k_hot),
                                ptr(v_hot), ptr(PiK), ptr(PiV), ptr(centroids), int(bits), int(kv_len), B, Hq, Hkv,
                                S, cap, hot_cap, float(scale), ptr(out), ptr(workspace), workspace.numel(),
                                stream_handle(q.device)),
        "lkv_tq_prefill_attn",
    )
    return out


def tq_prefill_attn(q, k_codes, k_norms, v_codes, v_norms, k_hot, v_hot, PiK, PiV, centroids, bits, kv_len: int,
                    scale: float | None = None):
    out = torch.empty_like(q)
    if scale is None:
        scale = 1.0 / math.sqrt(HEAD_DIM)
    return tq_prefill_attn_out(q, k_codes, k_norms, v_codes, v_norms, k_hot, v_hot, PiK, PiV, centroids, bits,
                               kv_len, scale, out)


def paged_decode_attn(q: torch.Tensor, kv_data: torch.Tensor, kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
                      kv_last_page_len: torch.Tensor, max_len: int, scale: float | None = None,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """Decode attention of q fp16 [B, Hq, 128] over a paged fp16 pool [max_pages, 2, page_size, Hkv, 128]
    with FlashInfer's CSR page table (int32 device tensors)."""
    require_cuda(q, kv_data, kv_indptr, kv_indices, kv_last_page_len)
    if q.dtype != torch.float16 or q.dim() != 3 or q.shape[-1] != HEAD_DIM or not q.is_contiguous():
        raise LeanKVError("paged_decode_attn: q must be contiguous float16 [B, Hq, 128]")
    if (kv_data.dtype != torch.float16 or kv_data.dim() != 5 or kv_data.shape[1] != 2
            or kv_data.shape[-1] != HEAD_DIM or not kv_data.is_contiguous()):
        raise LeanKVError("paged_decode_attn: kv_data must be contiguous float16 [max_pages, 2, page_size, Hkv, 128]")
    for t, nm in ((kv_indptr, "kv_indptr"), (kv_indices, "kv_indices"), (kv_last_page_len, "kv_last_page_len")):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise LeanKVError("paged_decode_attn: %s must be a contiguous int32 tensor" % nm)
    B, Hq, _ = q.shape
    max_pages, _, page_size, Hkv, _ = kv_data.shape
    if kv_indptr.numel() != B + 1 or kv_last_page_len.numel() != B:
        raise LeanKVError("paged_decode_attn: kv_indptr needs B + 1 entries and kv_last_page_len B")
    if out is None:
        out = torch.empty_like(q)
    if scale is None:
        scale = 1.0 / math.sqrt(HEAD_DIM)
    lib = _lib_handle()
    nbytes = lib.lkv_paged_decode_attn_workspace_bytes(B, Hq, Hkv, max_len)
    ws = workspaces.get(q.device, "paged", nbytes)
    check(
        lib.lkv_paged_decode_attn(ptr(q), ptr(kv_data), ptr(kv_indptr), ptr(kv_indices), ptr(kv_last_page_len), B,
                                  Hq, Hkv, page_size, max_pages, int(max_len), float(scale), ptr(out), ptr(ws),
                                  ws.numel(), stream_handle(q.device)),
        "lkv_paged_decode_attn",
    )
    return out


def tq_paged_decode_attn(q: torch.Tensor, k_codes: torch.Tensor, k_norms: torch.Tensor, v_codes: torch.Tensor,
                         v_norms: torch.Tensor, k_hot: torch.Tensor, v_hot: torch.Tensor, PiK: torch.Tensor,
                         PiV: torch.Tensor, centroids: torch.Tensor, bits: int, kv_indptr: torch.Tensor,
                         kv_indices: torch.Tensor, seq_lens: torch.Tensor, max_len: int, scale: float | None = None,
                         out: torch.Tensor | None = None) -> torch.Tensor:
    """Decode attention of q fp16 [B, Hq, 128] over a paged packed cache: code pools uint8
    [max_pages, Hkv, page_size, packed_row_bytes(bits)], norm pools fp32 [max_pages, Hkv, page_size], fp16 hot rings
    [B, Hkv, hot_cap, 128], FlashInfer's CSR page table and per-sequence lengths (int32 device tensors)."""
    require_cuda(q, k_codes, k_norms, v_codes, v_norms, k_hot, v_hot, kv_indptr, kv_indices, seq_lens)
    if q.dtype != torch.float16 or q.dim() != 3 or q.shape[-1] != HEAD_DIM or not q.is_contiguous():
        raise LeanKVError("tq_paged_decode_attn: q must be contiguous float16 [B, Hq, 128]")
    B, Hq, _ = q.shape
    rb = packed_row_bytes(bits)
    if k_codes.dim() != 4 or k_codes.dtype != torch.uint8 or k_codes.shape[-1] != rb:
        raise LeanKVError("tq_paged_decode_attn: code pools must be uint8 [max_pages, Hkv, page_size, %d] at %d bits"
                          % (rb, bits))
    max_pages, Hkv, page_size, _ = k_codes.shape
    for t, shape, dt, nm in ((v_codes, k_codes.shape, torch.uint8, "v_codes"),
                             (k_norms, k_codes.shape[:3], torch.float32, "k_norms"),
                             (v_norms, k_codes.shape[:3], torch.float32, "v_norms")):
        if tuple(t.shape) != tuple(shape) or t.dtype != dt or not t.is_contiguous():
            raise LeanKVError("tq_paged_decode_attn: %s must be contiguous %s %s" % (nm, dt, tuple(shape)))
    if not (k_codes.is_contiguous() and k_hot.is_contiguous() and v_hot.is_contiguous()):
        raise LeanKVError("tq_paged_decode_attn: pools and hot rings must be contiguous")
    if k_hot.dim() != 4 or tuple(k_hot.shape[:2]) != (B, Hkv) or k_hot.shape != v_hot.shape:
        raise LeanKVError("tq_paged_decode_attn: hot rings must be float16 [B, Hkv, hot_cap, 128]")
    for t, nm, n in ((kv_indptr, "kv_indptr", B + 1), (seq_lens, "seq_lens", B)):
        if t.dtype != torch.int32 or not t.is_contiguous() or t.numel() != n:
            raise LeanKVError("tq_paged_decode_attn: %s must be a contiguous int32 tensor of %d entries" % (nm, n))
    if kv_indices.dtype != torch.int32 or not kv_indices.is_contiguous():
        raise LeanKVError("tq_paged_decode_attn: kv_indices must be a contiguous int32 tensor")
    hot_cap = k_hot.shape[2]
    if out is None:
        out = torch.empty_like(q)
    if scale is None:
        scale = 1.0 / math.sqrt(HEAD_DIM)
    lib = _lib_handle()
    nbytes = lib.lkv_tq_paged_decode_attn_workspace_bytes(B, Hq, Hkv, int(max_len), page_size)
    ws = workspaces.get(q.device, "tq_paged", nbytes)
    PKc, PVc = _pi(PiK, q.device), _pi(PiV, q.device)  # alive until the call returns
    cen = _vec(centroids, q.device, 1 << bits, "centroids")
    check(
        lib.lkv_tq_paged_decode_attn(ptr(q), ptr(k_codes), ptr(k_norms), ptr(v_codes), ptr(v_norms), ptr(k_hot),
                                     ptr(v_hot), ptr(PKc), ptr(PVc), ptr(cen), int(bits),
                                     ptr(kv_indptr), ptr(kv_indices), ptr(seq_lens), B, Hq, Hkv, page_size, max_pages,
                                     int(max_len), hot_cap, float(scale), ptr(out), ptr(ws), ws.numel(),
                                     stream_handle(q.device)),
        "lkv_tq_paged_decode_attn",
    )
    return out


# ------------------------------------------------------------------ RMSNorm
def rms_norm_out(x: torch.Tensor, weight: torch.Tensor, eps: float, out: torch.Tensor) -> torch.Tensor:
    """out = RMSNorm(x) * weight over the last dim (fp16), rounded like HF MistralRMSNorm.

    Same summation order as the RMSNorm fused into the decode step's GEMV
    prologues (lkv_rmsnorm), so both give bit-identical activations."""
    require_cuda(x, weight, out)
    Z = x.shape[-1]
    if x.dtype != torch.float16 or weight.dtype != torch.float16 or out.dtype != torch.float16:
        raise LeanKVError("rms_norm: x, weight and out must be float16")
    if weight.numel() != Z or out.shape != x.shape or not out.is_contiguous():
        raise LeanKVError("rms_norm: weight must have %d elements and out the shape of x" % Z)
    xc = x.contiguous()
    M = xc.numel() // Z if Z else 0
    wc = weight.contiguous()
    check(_lib_handle().lkv_rmsnorm(ptr(xc), ptr(wc), float(eps), M, Z, ptr(out),
                                    stream_handle(x.device)), "lkv_rmsnorm")
    return out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    return rms_norm_out(x, weight, eps, torch.empty_like(x, memory_format=torch.contiguous_format))


# ------------------------------------------------------------------ RoPE
def rope_f16_(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> None:
    """In place: q [B, Hq, 128] and k [B, Hkv, 128] (contiguous fp16) rotated by the 128 fp16 factors of one
    position (cos, sin: 128 elements each), HF apply_rotary_pos_emb on fp16 tensors bit for bit (lkv_rope_f16)."""
    require_cuda(q, k, cos, sin)
    if any(t.dtype != torch.float16 for t in (q, k, cos, sin)):
        raise LeanKVError("rope_f16: q, k, cos and sin must be float16")
    if q.dim() != 3 or k.dim() != 3 or q.shape[0] != k.shape[0] or q.shape[-1] != HEAD_DIM or k.shape[-1] != HEAD_DIM:
        raise LeanKVError("rope_f16: q and k must be [B, H, %d] with the same B" % HEAD_DIM)
    if not (q.is_contiguous() and k.is_contiguous() and cos.is_contiguous() and sin.is_contiguous()):
        raise LeanKVError("rope_f16: q, k, cos and sin must be contiguous")
    if cos.numel() != HEAD_DIM or sin.numel() != HEAD_DIM:
        raise LeanKVError("rope_f16: cos and sin must hold %d factors" % HEAD_DIM)
    check(_lib_handle().lkv_rope_f16(ptr(q), ptr(k), ptr(cos), ptr(sin), q.shape[0], q.shape[1], k.shape[1],
                                     stream_handle(q.device)), "lkv_rope_f16")


# ------------------------------------------------------- torch custom ops
_LIB_DEF = None

# Schemas of torch.ops.leankv.*: the reference's kernel contracts (sparse_gemv.py:143-181,
# quantizer.py:119-137, rotation.py:45-52, cache.py:84-189 + sdpa_attention.py:79-105) as
# dispatcher ops.  Every functional op has an ``.out`` overload that writes caller-owned buffers,
# so a captured HIP graph holds no allocation; ``tq_cache_append`` mutates the cache in place.
_SCHEMAS = (
    "sparse_gemv(Tensor x, Tensor weight, float threshold) -> Tensor",
    "sparse_gemv.out(Tensor x, Tensor weight, float threshold, *, Tensor(a!) out) -> Tensor(a!)",
    "sparse_gateup_swiglu(Tensor x, Tensor w_gate, Tensor w_up, float t_gate, float t_up) -> Tensor",
    "sparse_gateup_swiglu.out(Tensor x, Tensor w_gate, Tensor w_up, float t_gate, float t_up, *, "
    "Tensor(a!) out) -> Tensor(a!)",
    "sparse_qkv(Tensor x, Tensor wq, Tensor wk, Tensor wv, float tq, float tk, float tv) -> (Tensor, Tensor, Tensor)",
    "sparse_qkv.out(Tensor x, Tensor wq, Tensor wk, Tensor wv, float tq, float tk, float tv, *, Tensor(a!) q, "
    "Tensor(b!) k, Tensor(c!) v) -> (Tensor(a!), Tensor(b!), Tensor(c!))",
    "tq_quantize(Tensor x, Tensor Pi, Tensor bounds, int bits) -> (Tensor, Tensor)",
    "tq_quantize_rotated(Tensor y, Tensor bounds, int bits) -> Tensor",
    "tq_dequantize(Tensor packed, Tensor norms, Tensor Pi, Tensor centroids, int bits, ScalarType? out_dtype=None) "
    "-> Tensor",
    "tq_rotate(Tensor x, Tensor Pi, bool transpose) -> Tensor",
    "rms_norm(Tensor x, Tensor weight, float eps) -> Tensor",
    "tq_cache_append(Tensor k_new, Tensor v_new, Tensor(a!) k_hot, Tensor(b!) v_hot, Tensor(c!) k_codes, "
    "Tensor(d!) k_norms, Tensor(e!) v_codes, Tensor(f!) v_norms, Tensor PiK, Tensor PiV, Tensor bounds, int bits, "
    "Tensor pos) -> ()",
    "tq_decode_attn(Tensor q, Tensor k_codes, Tensor k_norms, Tensor v_codes, Tensor v_norms, Tensor k_hot, "
    "Tensor v_hot, Tensor PiK, Tensor PiV, Tensor centroids, int bits, Tensor seq_len, int max_len, float scale) "
    "-> Tensor",
    "tq_decode_attn.out(Tensor q, Tensor k_codes, Tensor k_norms, Tensor v_codes, Tensor v_norms, Tensor k_hot, "
    "Tensor v_hot, Tensor PiK, Tensor PiV, Tensor centroids, int bits, Tensor seq_len, int max_len, float scale, *, "
    "Tensor(a!) out) -> Tensor(a!)",
    "tq_prefill_attn(Tensor q, Tensor k_codes, Tensor k_norms, Tensor v_codes, Tensor v_norms, Tensor k_hot, "
    "Tensor v_hot, Tensor PiK, Tensor PiV, Tensor centroids, int bits, int kv_len, float scale) -> Tensor",
    "tq_prefill_attn.out(Tensor q, Tensor k_codes, Tensor k_norms, Tensor v_codes, Tensor v_norms, Tensor k_hot, "
    "Tensor v_hot, Tensor PiK, Tensor PiV, Tensor centroids, int bits, int kv_len, float scale, *, "
    "Tensor(a!) out) -> Tensor(a!)",
)


def _impls():
    """name -> (device impl, meta impl)."""

    def m_gemv(x, w, t, out=None):
        return out if out is not None else x.new_empty(w.shape[0], dtype=torch.float16)

    def m_gateup(x, wg, wu, tg, tu, out=None):
        return out if out is not None else x.new_empty(wg.shape[0], dtype=torch.float16)

    def m_qkv(x, wq, wk, wv, tq, tk, tv, q=None, k=None, v=None):
        if q is not None:
            return q, k, v
        return tuple(x.new_empty(w.shape[0], dtype=torch.float16) for w in (wq, wk, wv))

    def m_quant(x, Pi, b, bits):
        rb = {1: 16, 2: 32}.get(int(bits), 64)
        return x.new_empty(*x.shape[:-1], rb, dtype=torch.uint8), x.new_empty(x.shape[:-1])

    def m_quant_rot(y, b, bits):
        rb = {1: 16, 2: 32}.get(int(bits), 64)
        return y.new_empty(*y.shape[:-1], rb, dtype=torch.uint8)

    def m_dequant(p, n, Pi, c, bits, out_dtype=None):
        return n.new_empty(*p.shape[:-1], HEAD_DIM, dtype=out_dtype or torch.float32)

    def m_rotate(x, Pi, tr):
        return x.new_empty(x.shape, dtype=torch.float32)

    def m_rms(x, w, eps):
        return torch.empty_like(x, memory_format=torch.contiguous_format)

    def m_append(*args):
        return None

    def m_attn(q, *args, out=None):
        return out if out is not None else torch.empty_like(q)

    return {
        "sparse_gemv": (lambda x, w, t: sparse_gemv(x, w, t), m_gemv),
        "sparse_gemv.out": (lambda x, w, t, out: sparse_gemv_out(x, w, t, out), m_gemv),
        "sparse_gateup_swiglu": (lambda x, wg, wu, tg, tu: sparse_gateup_swiglu(x, wg, wu, tg, tu), m_gateup),
        "sparse_gateup_swiglu.out": (lambda x, wg, wu, tg, tu, out: sparse_gateup_swiglu_out(x, wg, wu, tg, tu, out),
                                     m_gateup),
        "sparse_qkv": (lambda x, wq, wk, wv, tq, tk, tv: sparse_qkv(x, wq, wk, wv, tq, tk, tv), m_qkv),
        "sparse_qkv.out": (lambda x, wq, wk, wv, tq, tk, tv, q, k, v: sparse_qkv(x, wq, wk, wv, tq, tk, tv,
                                                                                out=(q, k, v)), m_qkv),
        "tq_quantize": (lambda x, Pi, b, bits: tq_quantize(x, Pi, b, bits), m_quant),
        "tq_quantize_rotated": (lambda y, b, bits: tq_quantize_rotated(y, b, bits), m_quant_rot),
        "tq_dequantize": (lambda p, n, Pi, c, bits, out_dtype=None: tq_dequantize(p, n, Pi, c, bits,
                                                                                   out_dtype or torch.float32),
                          m_dequant),
        "tq_rotate": (lambda x, Pi, tr: tq_rotate(x, Pi, tr), m_rotate),
        "rms_norm": (lambda x, w, eps: rms_norm(x, w, eps), m_rms),
        "tq_cache_append": (lambda *a: tq_cache_append(*a), m_append),
        "tq_decode_attn": (lambda *a: tq_decode_attn(*a), m_attn),
        "tq_decode_attn.out": (lambda *a, out: tq_decode_attn_out(*a, out), m_attn),
        "tq_prefill_attn": (lambda *a: tq_prefill_attn(*a), m_attn),
        "tq_prefill_attn.out": (lambda *a, out: tq_prefill_attn_out(*a, out), m_attn),
    }


def _register_ops() -> None:
    """Expose the kernels as torch.ops.leankv.* (GPU impl + Meta shape functions)."""
    global _LIB_DEF
    if _LIB_DEF is not None:
        return
    lib = torch.library.Library("leankv", "DEF")
    for schema in _SCHEMAS:
        lib.define(schema)
    for name, (dev, meta) in _impls().items():
        lib.impl(name, dev, "CUDA")
        lib.impl(name, meta, "Meta")
    _LIB_DEF = lib


def op_names() -> list:
    """Every registered torch.ops.leankv overload name ("sparse_gemv", "sparse_gemv.out", ...)."""
    return [s.split("(", 1)[0] for s in _SCHEMAS]


try:
    _register_ops()
except RuntimeError:  # already registered in this process (module reload)
    pass

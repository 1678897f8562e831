"""ctypes binding of ``libleankv_amd.so`` (the C ABI in include/leankv_amd.h).

torch is imported first on purpose: torch ships its own ``libamdhip64.so``
(SONAME libamdhip64.so.7); loading it before this library makes the dynamic
loader resolve our NEEDED entry to the same HIP runtime instance, so the
stream handles and device pointers torch hands us belong to our runtime too.

There is no fallback: if the library is missing, importing the kernels raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

from .build import LIB_PATH

LKV_OK = 0
LKV_DTYPE_F32 = 0
LKV_DTYPE_F16 = 1

_c_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_int = ctypes.c_int
_sz = ctypes.c_size_t

# name -> (restype, argtypes); the exact list exported by include/leankv_amd.h
SIGNATURES = {
    "lkv_version": (_int, []),
    "lkv_last_error": (ctypes.c_char_p, []),
    "lkv_sparse_gemv_workspace_bytes": (_sz, [_i64, _i64]),
    "lkv_sparse_gemv": (_int, [_c_p, _c_p, _f32, _i64, _i64, _c_p, _c_p, _sz, _c_p]),
    "lkv_sparse_gemv_noalloc_max_bytes": (_sz, []),
    "lkv_sparse_gemv_noalloc": (_int, [_c_p, _c_p, _f32, _i64, _i64, _c_p, _c_p]),
    "lkv_sparse_gateup_workspace_bytes": (_sz, [_i64, _i64]),
    "lkv_sparse_gateup_swiglu": (_int, [_c_p, _c_p, _c_p, _f32, _f32, _i64, _i64, _c_p, _c_p, _sz, _c_p]),
    "lkv_sparse_gemv_multi_workspace_bytes": (_sz, [_int, _c_p, _i64]),
    "lkv_sparse_gemv_multi": (_int, [_c_p, _int, _c_p, _c_p, _c_p, _i64, _c_p, _c_p, _sz, _c_p]),
    "lkv_sparse_gemv_chunks": (_int, [_i64, _i64]),
    "lkv_sparse_gemv_partials": (_int, [_c_p, _c_p, _c_p, _f32, _f32, _i64, _i64, _c_p, _sz, _c_p]),
    "lkv_tq_packed_row_bytes": (_int, [_int]),
    "lkv_tq_quantize": (_int, [_c_p, _int, _i64, _c_p, _c_p, _int, _c_p, _c_p, _c_p]),
    "lkv_tq_quantize_rotated": (_int, [_c_p, _i64, _c_p, _int, _c_p, _c_p]),
    "lkv_tq_dequantize": (_int, [_c_p, _c_p, _int, _i64, _c_p, _c_p, _int, _c_p, _int, _c_p]),
    "lkv_tq_rotate": (_int, [_c_p, _int, _i64, _c_p, _int, _c_p, _c_p]),
    "lkv_tq_prod_quantize": (_int, [_c_p, _int, _i64, _c_p, _c_p, _c_p, _c_p, _int, _c_p, _c_p, _c_p, _c_p, _c_p]),
    "lkv_tq_prod_dequantize": (_int, [_c_p, _c_p, _int, _c_p, _c_p, _i64, _c_p, _c_p, _c_p, _int, _f32, _c_p, _int,
                                      _c_p]),
    "lkv_tq_cache_append": (_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _int,
                                   _c_p, _i64, _i64, _i64, _c_p]),
    "lkv_tq_decode_attn_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "lkv_tq_decode_attn": (_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _int, _c_p,
                                  _i64, _i64, _i64, _i64, _i64, _i64, _f32, _c_p, _c_p, _sz, _c_p]),
    "lkv_sparse_gemm_batched_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "lkv_sparse_gemm_batched": (_int, [_c_p, _c_p, _f32, _i64, _i64, _i64, _c_p, _c_p, _sz, _c_p]),
    "lkv_sparse_gemm_batched_multi_workspace_bytes": (_sz, [_i64, _int, _c_p, _i64]),
    "lkv_sparse_gemm_batched_multi": (_int, [_c_p, _i64, _int, _c_p, _c_p, _c_p, _i64, _int, _c_p, _c_p, _c_p, _c_p,
                                             _c_p, _sz, _c_p]),
    "lkv_sparse_gemm_batched_residual_rmsnorm": (_int, [_c_p, _c_p, _f32, _i64, _i64, _i64, _c_p, _c_p, _f32, _c_p,
                                                        _c_p, _c_p, _sz, _c_p]),
    "lkv_sparse_gemm_batched_qkv_rope": (_int, [_c_p, _i64, _c_p, _c_p, _c_p, _i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                                _i64, _c_p, _sz, _c_p]),
    "lkv_tq_cache_evict": (_int, [_c_p, _i64, _i64, _i64, _i64, _c_p, _int, _c_p, _c_p]),
    "lkv_paged_decode_attn_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "lkv_tq_paged_decode_attn_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "lkv_tq_paged_decode_attn": (_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _int, _c_p, _c_p,
                                        _c_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _c_p, _c_p, _sz, _c_p]),
    "lkv_paged_decode_attn": (_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _c_p,
                                     _c_p, _sz, _c_p]),
    "lkv_tq_prefill_attn_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "lkv_tq_prefill_attn": (_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _int, _i64, _i64,
                                   _i64, _i64, _i64, _i64, _i64, _f32, _c_p, _c_p, _sz, _c_p]),
    "lkv_rmsnorm": (_int, [_c_p, _c_p, _f32, _i64, _i64, _c_p, _c_p]),
    "lkv_rope_f16": (_int, [_c_p, _c_p, _c_p, _c_p, _i64, _i64, _i64, _c_p]),
    "lkv_decode_workspace_bytes": (_sz, [_c_p]),
    "lkv_decode_workspace_layout": (_int, [_c_p, _c_p]),
    "lkv_decode_begin": (_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _sz, _c_p]),
    "lkv_decode_evict": (_int, [_c_p, _c_p, ctypes.c_int64, _c_p, _sz, _c_p]),
    "lkv_decode_layer_step": (_int, [_c_p, _c_p, _c_p, _c_p, _sz, _c_p]),
    "lkv_decode_layer_step_f16kv": (_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _sz, _c_p]),
    "lkv_decode_head": (_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i64, _c_p, _sz, _c_p]),
}


class DecodeDims(ctypes.Structure):
    """lkv_decode_dims (include/leankv_amd.h)."""

    _fields_ = [
        ("hidden", _i64), ("ffn", _i64), ("vocab", _i64), ("n_heads", _i64), ("n_kv_heads", _i64),
        ("max_len", _i64), ("cap", _i64), ("hot_cap", _i64), ("bits", ctypes.c_int32), ("eps", _f32),
        ("scale", _f32), ("bounds", _c_p), ("centroids", _c_p), ("rope_cos", _c_p), ("rope_sin", _c_p),
    ]


class DecodeLayer(ctypes.Structure):
    """lkv_decode_layer (include/leankv_amd.h)."""

    _fields_ = [
        ("input_norm", _c_p), ("post_norm", _c_p), ("wq", _c_p), ("wk", _c_p), ("wv", _c_p), ("wo", _c_p),
        ("wg", _c_p), ("wu", _c_p), ("wd", _c_p),
        ("tq", _f32), ("tk", _f32), ("tv", _f32), ("to", _f32), ("tg", _f32), ("tu", _f32), ("td", _f32),
        ("k_codes", _c_p), ("k_norms", _c_p), ("v_codes", _c_p), ("v_norms", _c_p), ("k_hot", _c_p),
        ("v_hot", _c_p), ("PiK", _c_p), ("PiV", _c_p),
    ]

class DecodeLayout(ctypes.Structure):
    """lkv_decode_layout (include/leankv_amd.h): byte offsets of a step's results in its workspace."""

    _fields_ = [
        ("part_q", _sz), ("part_k", _sz), ("part_v", _sz), ("part_o", _sz), ("part_gate", _sz), ("part_up", _sz),
        ("part_down", _sz), ("part_lm", _sz), ("q_rope", _sz), ("attn_out", _sz), ("total", _sz),
        ("chunks_qkv", ctypes.c_int32), ("chunks_o", ctypes.c_int32), ("chunks_gateup", ctypes.c_int32),
        ("chunks_down", ctypes.c_int32), ("chunks_lm", ctypes.c_int32),
    ]


_lib = None
_lock = threading.Lock()


class LeanKVError(RuntimeError):
    """Raised when a leankv_amd C entry point rejects a call or fails to launch."""


def load(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        # LKV_LIBRARY: another build of the same sources (the phase-stamp build, `python -m leankv_amd.build
        # --stamps`, used by bench.py --phases)
        p = path or os.environ.get("LKV_LIBRARY") or LIB_PATH
        if not os.path.exists(p):
            raise ImportError(
                "leankv_amd: %s is missing; build it with `python -m leankv_amd.build` "
                "(there is no CPU fallback)" % p
            )
        lib = ctypes.CDLL(p)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def last_error() -> str:
    return load().lkv_last_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc != LKV_OK:
        raise LeanKVError("%s failed (code %d): %s" % (what, rc, last_error()))


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return LKV_DTYPE_F32
    if dt == torch.float16:
        return LKV_DTYPE_F16
    raise TypeError("leankv_amd: unsupported dtype %s (float32/float16 only)" % dt)


def require_cuda(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise LeanKVError(
                "leankv_amd kernels run on the GPU only; got a tensor on %s" % t.device
            )


class _Workspaces:
    """Device workspaces, one per (device, key), grown on demand.

    No entry point reads workspace contents left by an earlier call, so a
    workspace is reused by later calls on the same stream without clearing
    (which also keeps the calls capturable in a HIP graph).
    """

    def __init__(self):
        self._bufs: dict[tuple[int, str], torch.Tensor] = {}

    def get(self, device: torch.device, key: str, nbytes: int) -> torch.Tensor:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        k = (idx, key)
        buf = self._bufs.get(k)
        if buf is None or buf.numel() < nbytes:
            size = max(nbytes, 256)
            if buf is not None:
                size = max(size, 2 * buf.numel())
            buf = torch.zeros(size, dtype=torch.uint8, device=device)
            self._bufs[k] = buf
        return buf


workspaces = _Workspaces()

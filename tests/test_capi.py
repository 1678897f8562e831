"""CPU tests of the C-ABI boundary: the library loads, exports every symbol the
header declares, and rejects bad arguments before it touches a GPU."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "leankv_amd.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(lkv_\w+)\s*\(", src)))


def test_header_declares_expected_entry_points():
    names = _declared()
    for n in ("lkv_sparse_gemv", "lkv_sparse_gateup_swiglu", "lkv_tq_quantize", "lkv_tq_quantize_rotated",
              "lkv_tq_dequantize", "lkv_tq_rotate", "lkv_tq_cache_append", "lkv_tq_decode_attn"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from leankv_amd import _lib

    lib = _lib.load()
    for n in _declared():
        assert hasattr(lib, n), n
    assert set(_declared()) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"
    assert lib.lkv_version() >= 100


def test_library_built_for_gfx950():
    from leankv_amd.build import LIB_PATH

    blob = open(LIB_PATH, "rb").read()
    assert b"gfx950" in blob


def test_row_bytes_and_workspace_queries():
    from leankv_amd import _lib

    lib = _lib.load()
    assert [lib.lkv_tq_packed_row_bytes(b) for b in (1, 2, 3, 4)] == [16, 32, 64, 64]
    assert lib.lkv_tq_packed_row_bytes(5) < 0
    assert lib.lkv_sparse_gemv_workspace_bytes(4096, 14336) > 0
    assert lib.lkv_sparse_gateup_workspace_bytes(14336, 4096) > lib.lkv_sparse_gemv_workspace_bytes(14336, 4096)
    assert lib.lkv_tq_decode_attn_workspace_bytes(16, 32, 8, 4160) >= 16 * 32 * 128 * 4


def test_invalid_arguments_rejected_without_launch():
    from leankv_amd import _lib

    lib = _lib.load()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    # N not a multiple of 8
    assert lib.lkv_sparse_gemv(p, p, 0.1, 12, 16, p, p, 1 << 20, None) == -1
    assert "multiple of 8" in _lib.last_error()
    # unsupported bits
    assert lib.lkv_tq_quantize(p, 0, 16, p, p, 5, p, p, None) == -1
    assert "bits" in _lib.last_error()
    # bad dtype code
    assert lib.lkv_tq_rotate(p, 7, 16, p, 0, p, None) == -1
    # GQA ratio not integral
    assert lib.lkv_tq_decode_attn(p, p, p, p, p, p, p, p, p, p, 3, p, 64, 1, 30, 8, 64, 64, 0.1, p, p,
                                  1 << 20, None) == -1
    # max_len beyond the cache
    assert lib.lkv_tq_decode_attn(p, p, p, p, p, p, p, p, p, p, 3, p, 1000, 1, 32, 8, 64, 64, 0.1, p, p,
                                  1 << 20, None) == -1
    assert "max_len" in _lib.last_error()
    # empty problems are no-ops
    assert lib.lkv_sparse_gemv(p, p, 0.1, 0, 16, p, p, 0, None) == 0
    assert lib.lkv_tq_quantize(p, 0, 0, p, p, 3, p, p, None) == 0


def test_python_wrappers_refuse_cpu_tensors():
    import torch

    from leankv_amd import kernels
    from leankv_amd._lib import LeanKVError

    w = torch.zeros(16, 8, dtype=torch.float16).t().contiguous().t()
    with pytest.raises(LeanKVError):
        kernels.sparse_gemv(torch.zeros(8, dtype=torch.float16), w, 0.1)
    with pytest.raises(LeanKVError):
        kernels.colmajor_rows(torch.zeros(16, 8, dtype=torch.float16))  # row-major weight

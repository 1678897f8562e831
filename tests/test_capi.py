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
              "lkv_tq_dequantize", "lkv_tq_rotate", "lkv_tq_cache_append", "lkv_tq_decode_attn",
              "lkv_tq_prefill_attn", "lkv_tq_prod_quantize", "lkv_tq_prod_dequantize",
              "lkv_tq_paged_decode_attn"):
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
    assert lib.lkv_sparse_gemv_noalloc_max_bytes() == 8 << 20


def test_invalid_arguments_rejected_without_launch():
    from leankv_amd import _lib

    lib = _lib.load()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    # N not a multiple of 8
    assert lib.lkv_sparse_gemv(p, p, 0.1, 12, 16, p, p, 1 << 20, None) == -1
    assert "multiple of 8" in _lib.last_error()
    # no-alloc GEMV: a shape whose partials exceed the scratch array is refused before any HIP call
    N, Z = 65536, 32767  # weight just under the 4 GiB descriptor range
    assert lib.lkv_sparse_gemv_workspace_bytes(N, Z) > lib.lkv_sparse_gemv_noalloc_max_bytes()
    assert lib.lkv_sparse_gemv_noalloc(p, p, 0.1, N, Z, p, None) == -1
    assert "scratch" in _lib.last_error()
    assert lib.lkv_sparse_gemv_noalloc(p, p, 0.1, 12, 16, p, None) == -1
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
    # prefill: query heads per kv head not a power of two <= 16, S beyond the cache, too few cold rows
    assert lib.lkv_tq_prefill_attn(p, p, p, p, p, p, p, p, p, p, 3, 100, 1, 12, 4, 100, 64, 64, 0.1, p, p,
                                   1 << 30, None) == -1
    assert "Hq/Hkv" in _lib.last_error()
    assert lib.lkv_tq_prefill_attn(p, p, p, p, p, p, p, p, p, p, 3, 100, 1, 8, 2, 101, 64, 64, 0.1, p, p,
                                   1 << 30, None) == -1
    assert "S <= kv_len" in _lib.last_error()
    assert lib.lkv_tq_prefill_attn(p, p, p, p, p, p, p, p, p, p, 3, 200, 1, 8, 2, 100, 64, 64, 0.1, p, p,
                                   1 << 30, None) == -1
    assert "exceed cap" in _lib.last_error()
    assert lib.lkv_tq_prefill_attn(p, p, p, p, p, p, p, p, p, p, 3, 100, 1, 8, 2, 100, 64, 64, 0.1, p, p,
                                   1024, None) == -1
    assert "workspace" in _lib.last_error()
    # the two hot rings rotated into the key / value domains (the kernel rotates its own queries)
    assert lib.lkv_tq_prefill_attn_workspace_bytes(1, 32, 8, 4096, 64) == 2 * 8 * 64 * 128 * 2
    # RoPE: negative sizes, null factors
    assert lib.lkv_rope_f16(p, p, p, p, -1, 32, 8, None) == -1
    assert "out of range" in _lib.last_error()
    assert lib.lkv_rope_f16(p, p, None, p, 2, 32, 8, None) == -1
    assert "null" in _lib.last_error()
    assert lib.lkv_rope_f16(None, None, None, None, 0, 32, 8, None) == 0  # nothing to do, nothing touched
    # batched sparse GEMM: N not a multiple of 8, workspace too small for a multi-chunk problem
    assert lib.lkv_sparse_gemm_batched(p, p, 0.1, 4, 12, 16, p, p, 1 << 20, None) == -1
    assert "multiple of 8" in _lib.last_error()
    assert lib.lkv_sparse_gemm_batched(p, p, 0.1, 4, 4096, 14336, p, p, 1024, None) == -1
    assert "workspace" in _lib.last_error()
    assert lib.lkv_sparse_gemm_batched_workspace_bytes(4, 4096, 14336) > 4 * 4096 * 4
    assert lib.lkv_sparse_gemm_batched(p, p, 0.1, 0, 4096, 14336, p, p, 0, None) == 0
    # grouped batched products: product count, epilogue / count pairing, SwiGLU shapes, residual, workspace
    def multi(n, Ns, epi, res=p, ws_bytes=1 << 30, B=4, Z=4096, rope=p):
        arr = (ctypes.c_int64 * max(n, 1))(*Ns)
        ptrs = (ctypes.c_void_p * max(n, 1))(*([p] * max(n, 1)))
        ts = (ctypes.c_float * max(n, 1))(*([0.0] * max(n, 1)))
        return lib.lkv_sparse_gemm_batched_multi(p, B, n, ptrs, ts, arr, Z, epi, res, rope, rope, ptrs, p, ws_bytes,
                                                 None)

    assert multi(0, [4096], 0) == -1 and "products" in _lib.last_error()
    assert multi(4, [8, 8, 8, 8], 0) == -1 and "products" in _lib.last_error()
    assert multi(1, [4096], 1) == -1 and "epilogue" in _lib.last_error()
    assert multi(2, [4096, 4096], 2) == -1 and "epilogue" in _lib.last_error()
    assert multi(2, [4096, 1024], 1) == -1 and "SwiGLU" in _lib.last_error()
    assert multi(1, [4096], 2, res=None) == -1 and "residual" in _lib.last_error()
    assert multi(3, [4096, 1020, 1024], 0) == -1 and "multiple of 8" in _lib.last_error()
    assert multi(3, [4096, 1024, 1024], 0, ws_bytes=1024) == -1 and "workspace" in _lib.last_error()
    assert multi(3, [4096, 1024, 1024], 0, B=0) == 0  # nothing to do, nothing touched
    assert multi(1, [4096], 3) == -1 and "epilogue" in _lib.last_error()  # RoPE takes q, k[, v]
    assert multi(3, [4096, 1000, 1024], 3) == -1 and "RoPE" in _lib.last_error()
    assert multi(3, [4096, 1024, 1024], 3, rope=None) == -1 and "RoPE factors" in _lib.last_error()
    assert multi(1, [4096], 4) == -1 and "epilogue" in _lib.last_error()  # the fused norm has its own entry
    # product + residual + RMSNorm: the fused norm's column limit, null norm weight, alignment
    rn = lib.lkv_sparse_gemm_batched_residual_rmsnorm
    assert rn(p, p, 0.0, 4, 16384, 4096, p, p, 1e-5, p, p, p, 1 << 30, None) == -1
    assert "8192" in _lib.last_error()
    assert rn(p, p, 0.0, 4, 4096, 4096, p, None, 1e-5, p, p, p, 1 << 30, None) == -1
    assert "RMSNorm weight" in _lib.last_error()
    q = ctypes.c_void_p(24)
    assert rn(p, p, 0.0, 4, 4096, 4096, q, p, 1e-5, p, p, p, 1 << 30, None) == -1
    assert "aligned" in _lib.last_error()
    assert rn(p, p, 0.0, 0, 4096, 4096, p, p, 1e-5, p, p, p, 0, None) == 0
    # q/k/v + RoPE + ring: rings go in pairs, k and v alike, a position with them
    qr = lib.lkv_sparse_gemm_batched_qkv_rope
    n3 = (ctypes.c_int64 * 3)(4096, 1024, 1024)
    p3 = (ctypes.c_void_p * 3)(p, p, p)
    t3 = (ctypes.c_float * 3)(0.0, 0.0, 0.0)
    assert qr(p, 4, p3, t3, n3, 4096, p, p, p3, p, None, p, 64, p, 1 << 30, None) == -1
    assert "rings" in _lib.last_error()
    assert qr(p, 4, p3, t3, n3, 4096, p, p, p3, p, p, None, 64, p, 1 << 30, None) == -1
    assert "position" in _lib.last_error()
    n3b = (ctypes.c_int64 * 3)(4096, 1024, 512)
    assert qr(p, 4, p3, t3, n3b, 4096, p, p, p3, p, p, p, 64, p, 1 << 30, None) == -1
    assert "k and v" in _lib.last_error()
    # batched eviction: sizes, bits, null layer table
    assert lib.lkv_tq_cache_evict(p, 2, -1, 64, 100, p, 3, p, None) == -1 and "bad sizes" in _lib.last_error()
    assert lib.lkv_tq_cache_evict(p, 2, 16, 64, 100, p, 5, p, None) == -1 and "bits" in _lib.last_error()
    assert lib.lkv_tq_cache_evict(None, 2, 16, 64, 100, p, 3, p, None) == -1 and "null" in _lib.last_error()
    assert lib.lkv_tq_cache_evict(None, 0, 16, 64, 100, None, 3, None, None) == 0
    qkv = (ctypes.c_int64 * 3)(4096, 1024, 1024)
    assert lib.lkv_sparse_gemm_batched_multi_workspace_bytes(16, 3, qkv, 4096) == sum(
        lib.lkv_sparse_gemm_batched_workspace_bytes(16, N, 4096) - 256 for N in (4096, 1024, 1024)) + 256
    # paged decode attention: GQA ratio, page size, workspace
    assert lib.lkv_paged_decode_attn(p, p, p, p, p, 1, 30, 8, 16, 64, 100, 0.1, p, p, 1 << 20, None) == -1
    assert "Hq/Hkv" in _lib.last_error()
    assert lib.lkv_paged_decode_attn(p, p, p, p, p, 1, 32, 8, 0, 64, 100, 0.1, p, p, 1 << 20, None) == -1
    assert "page_size" in _lib.last_error()
    assert lib.lkv_paged_decode_attn(p, p, p, p, p, 16, 32, 8, 16, 64, 4096, 0.1, p, p, 256, None) == -1
    assert "workspace" in _lib.last_error()
    assert lib.lkv_paged_decode_attn(p, p, p, p, p, 0, 32, 8, 16, 64, 100, 0.1, p, p, 0, None) == 0
    # TurboQuantProd: MSE bits outside 1..4, bad dtype codes
    assert lib.lkv_tq_prod_quantize(p, 0, 16, p, p, p, p, 0, p, p, p, p, None) == -1
    assert "mse_bits" in _lib.last_error()
    assert lib.lkv_tq_prod_quantize(p, 7, 16, p, p, p, p, 2, p, p, p, p, None) == -1
    assert lib.lkv_tq_prod_dequantize(p, p, 0, p, p, 16, p, p, p, 5, 0.01, p, 0, None) == -1
    assert "mse_bits" in _lib.last_error()
    assert lib.lkv_tq_prod_dequantize(p, p, 9, p, p, 16, p, p, p, 2, 0.01, p, 0, None) == -1
    assert lib.lkv_tq_prod_quantize(p, 0, 0, p, p, p, p, 2, p, p, p, p, None) == 0
    assert lib.lkv_tq_prod_dequantize(p, p, 0, p, p, 0, p, p, p, 2, 0.01, p, 0, None) == 0
    # paged packed attention: page size not a power of two in 16..128, pool past 2^32 bytes, bits
    assert lib.lkv_tq_paged_decode_attn(p, p, p, p, p, p, p, p, p, p, 3, p, p, p, 2, 32, 8, 24, 64, 100, 64, 0.1,
                                        p, p, 1 << 20, None) == -1
    assert "page_size" in _lib.last_error()
    assert lib.lkv_tq_paged_decode_attn(p, p, p, p, p, p, p, p, p, p, 3, p, p, p, 2, 32, 8, 16, 1 << 20, 100, 64,
                                        0.1, p, p, 1 << 20, None) == -1
    assert "2^32" in _lib.last_error()
    assert lib.lkv_tq_paged_decode_attn(p, p, p, p, p, p, p, p, p, p, 5, p, p, p, 2, 32, 8, 16, 64, 100, 64, 0.1,
                                        p, p, 1 << 20, None) == -1
    assert "bits" in _lib.last_error()
    # hot windows up to 256 slots (the combine's slot groups)
    assert lib.lkv_tq_paged_decode_attn(p, p, p, p, p, p, p, p, p, p, 2, p, p, p, 2, 32, 8, 16, 64, 100, 257, 0.1,
                                        p, p, 1 << 20, None) == -1
    assert "hot_cap" in _lib.last_error()
    assert lib.lkv_tq_decode_attn(p, p, p, p, p, p, p, p, p, p, 1, p, 64, 1, 32, 8, 64, 257, 0.1, p, p,
                                  1 << 20, None) == -1
    assert "hot_cap" in _lib.last_error()
    assert lib.lkv_tq_decode_attn(p, p, p, p, p, p, p, p, p, p, 0, p, 64, 1, 32, 8, 64, 64, 0.1, p, p,
                                  1 << 20, None) == -1
    assert "bits" in _lib.last_error()
    assert lib.lkv_tq_paged_decode_attn(p, p, p, p, p, p, p, p, p, p, 3, p, p, p, 16, 32, 8, 16, 64, 4096, 64,
                                        0.1, p, p, 256, None) == -1
    assert "workspace" in _lib.last_error()
    assert lib.lkv_tq_paged_decode_attn(p, p, p, p, p, p, p, p, p, p, 3, p, p, p, 0, 32, 8, 16, 64, 100, 64, 0.1,
                                        p, p, 0, None) == 0
    # empty problems are no-ops
    assert lib.lkv_tq_prefill_attn(p, p, p, p, p, p, p, p, p, p, 3, 100, 1, 8, 2, 0, 64, 64, 0.1, p, p, 0, None) == 0
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


def _mistral_dims(**kw):
    from leankv_amd import _lib

    d = dict(hidden=4096, ffn=14336, vocab=32768, n_heads=32, n_kv_heads=8, max_len=4224, cap=4160, hot_cap=64,
             bits=3, eps=1e-5, scale=128 ** -0.5, bounds=16, centroids=16, rope_cos=16, rope_sin=16)
    d.update(kw)
    return _lib.DecodeDims(**d)


def test_decode_struct_layout_matches_header():
    """ctypes mirrors of lkv_decode_dims / lkv_decode_layer have the C layout (field order, padding)."""
    from leankv_amd import _lib

    src = open(HEADER).read()
    for cls, cname in ((_lib.DecodeDims, "lkv_decode_dims"), (_lib.DecodeLayer, "lkv_decode_layer"),
                       (_lib.DecodeLayout, "lkv_decode_layout")):
        body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (cname, cname), src, flags=re.S).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        names = re.findall(r"(\w+)\s*(?=[,;])", body)
        assert [f[0] for f in cls._fields_] == names, cname
    assert ctypes.sizeof(_lib.DecodeDims) == 8 * 8 + 4 * 3 + 4 + 8 * 4  # 4 bytes of padding before bounds
    assert ctypes.sizeof(_lib.DecodeLayer) == 9 * 8 + 7 * 4 + 4 + 8 * 8
    assert ctypes.sizeof(_lib.DecodeLayout) == 11 * 8 + 5 * 4 + 4  # padded to 8-byte alignment


def test_decode_workspace_layout():
    """The layout query: regions in step order, inside the workspace, sized by their chunk counts."""
    from leankv_amd import _lib

    lib = _lib.load()
    d = _mistral_dims()
    lay = _lib.DecodeLayout()
    assert lib.lkv_decode_workspace_layout(ctypes.byref(d), ctypes.byref(lay)) == 0
    assert lay.total == lib.lkv_decode_workspace_bytes(ctypes.byref(d))
    slabs = lambda n: (n + 255) // 256  # noqa: E731
    assert lay.part_k - lay.part_q == slabs(4096) * lay.chunks_qkv * 256 * 4
    assert lay.part_v - lay.part_k == slabs(1024) * lay.chunks_qkv * 256 * 4
    assert lay.part_up - lay.part_gate == slabs(14336) * lay.chunks_gateup * 256 * 4
    # every chunk count covers its input dimension in chunks of 256, 512 or 1024 rows
    assert 4096 % lay.chunks_qkv == 0 and 4096 // lay.chunks_qkv in (256, 512, 1024)
    assert any(-(-14336 // bz) == lay.chunks_down for bz in (256, 512, 1024)) and lay.chunks_down > 1
    offs = [lay.part_q, lay.part_k, lay.part_v, lay.part_o, lay.part_gate, lay.part_up, lay.part_down, lay.part_lm,
            lay.q_rope, lay.attn_out]
    assert offs == sorted(offs) and offs[-1] + 4096 * 2 <= lay.total
    assert lib.lkv_decode_workspace_layout(ctypes.byref(_mistral_dims(bits=5)), ctypes.byref(lay)) == -1
    for bits in (1, 2, 4):  # every packing of quantizer.py:38-62; the plan does not depend on the width
        lay2 = _lib.DecodeLayout()
        assert lib.lkv_decode_workspace_layout(ctypes.byref(_mistral_dims(bits=bits)), ctypes.byref(lay2)) == 0
        assert lay2.total == lay.total
    assert lib.lkv_decode_workspace_layout(ctypes.byref(d), None) == -1


def test_decode_dims_validated_without_launch():
    from leankv_amd import _lib

    lib = _lib.load()
    ok = _mistral_dims()
    assert lib.lkv_decode_workspace_bytes(ctypes.byref(ok)) > 0
    for hot in (1, 128, 256):  # windows the step's combine walks (up to four groups of 64 slots)
        assert lib.lkv_decode_workspace_bytes(ctypes.byref(_mistral_dims(hot_cap=hot, cap=4224 - hot))) > 0, hot
    for bad, msg in ((dict(hidden=4000), "hidden"), (dict(n_heads=36), "n_heads"), (dict(n_kv_heads=2), "n_heads"),
                     (dict(bits=5), "bits"), (dict(bits=0), "bits"), (dict(hot_cap=257), "hot_cap"),
                     (dict(cap=100), "cap"),
                     (dict(rope_cos=None), "RoPE"), (dict(vocab=32770), "vocab")):
        d = _mistral_dims(**bad)
        assert lib.lkv_decode_workspace_bytes(ctypes.byref(d)) == 0, bad
        p = ctypes.c_void_p(16)
        assert lib.lkv_decode_begin(ctypes.byref(d), p, p, p, p, p, 1 << 30, None) == -1
        assert msg in _lib.last_error(), (bad, _lib.last_error())
    # workspace too small / null layer are rejected before any launch
    p = ctypes.c_void_p(16)
    assert lib.lkv_decode_begin(ctypes.byref(ok), p, p, p, p, p, 1024, None) == -1
    assert "workspace" in _lib.last_error()
    assert lib.lkv_decode_layer_step(ctypes.byref(ok), None, p, p, 1 << 30, None) == -1
    # eviction: null table, and a layer with a null cache pointer, are rejected before any launch
    assert lib.lkv_decode_evict(ctypes.byref(ok), None, 1, p, 1 << 30, None) == -1
    layers = (_lib.DecodeLayer * 2)()
    assert lib.lkv_decode_evict(ctypes.byref(ok), layers, 2, p, 1 << 30, None) == -1
    assert "layer 0" in _lib.last_error()
    assert lib.lkv_decode_evict(ctypes.byref(ok), layers, 2, p, 1024, None) == -1
    assert "workspace" in _lib.last_error()

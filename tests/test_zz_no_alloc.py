"""lkv_sparse_gemv_noalloc (the split-K partials in the library's own device
array, no workspace, no allocation) against lkv_sparse_gemv with a caller
workspace, through the C ABI: bit-identical outputs on consecutive calls of
decreasing size (the array keeps the previous call's partials), the
single-chunk shape, and the refusal of a shape beyond the array."""

import numpy as np
import pytest
import torch

from oracle import teal as ot

pytestmark = pytest.mark.gpu


def _case(N, Z, seed, q=0.4):
    g = torch.Generator().manual_seed(seed)
    W = (torch.randn(N, Z, generator=g) * 0.02).to(torch.float16)
    x = (torch.randn(Z, generator=g) * 0.05).to(torch.float16)
    k = int(q * Z)
    t = torch.kthvalue(x.float().abs(), k).values.item() if k > 0 else 0.0
    return W, x, t


def _both(lib, dev, N, Z, seed):
    from leankv_amd import _lib

    W, x, t = _case(N, Z, seed)
    wc = W.to(dev).t().contiguous().t()
    xd = x.to(dev)
    st = _lib.stream_handle(dev)
    y_ws = torch.empty(N, dtype=torch.float16, device=dev)
    nbytes = lib.lkv_sparse_gemv_workspace_bytes(N, Z)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    _lib.check(lib.lkv_sparse_gemv(xd.data_ptr(), wc.data_ptr(), t, N, Z, y_ws.data_ptr(), ws.data_ptr(), nbytes, st),
               "lkv_sparse_gemv")
    y_na = torch.full((N,), float("nan"), dtype=torch.float16, device=dev)
    _lib.check(lib.lkv_sparse_gemv_noalloc(xd.data_ptr(), wc.data_ptr(), t, N, Z, y_na.data_ptr(), st),
               "lkv_sparse_gemv_noalloc")
    torch.cuda.synchronize()
    return W, x, t, y_ws.cpu(), y_na.cpu()


def test_noalloc_equals_workspace_entry_on_consecutive_calls(cuda):
    from leankv_amd import _lib

    lib = _lib.load()
    print("noalloc case 1: N=4096 Z=14336 (config 1)", flush=True)
    W, x, t, y_ws, y_na = _both(lib, cuda, 4096, 14336, seed=0)
    assert torch.equal(y_ws.view(torch.int16), y_na.view(torch.int16))
    assert ot.rel_err(y_na.numpy(), ot.sparse_gemv(x.numpy(), W.numpy(), t)) < 1e-3
    print("noalloc case 2: N=1024 Z=4096 (smaller, after case 1)", flush=True)
    W, x, t, y_ws, y_na = _both(lib, cuda, 1024, 4096, seed=1)
    assert torch.equal(y_ws.view(torch.int16), y_na.view(torch.int16))
    assert ot.rel_err(y_na.numpy(), ot.sparse_gemv(x.numpy(), W.numpy(), t)) < 1e-3
    print("noalloc case 3: N=24 Z=100 (one chunk)", flush=True)
    W, x, t, y_ws, y_na = _both(lib, cuda, 24, 100, seed=2)
    assert torch.equal(y_ws.view(torch.int16), y_na.view(torch.int16))


def test_noalloc_refuses_shapes_beyond_the_array(cuda):
    from leankv_amd import _lib

    lib = _lib.load()
    N, Z = 65536, 32767  # weight just under the 4 GiB descriptor range
    assert lib.lkv_sparse_gemv_workspace_bytes(N, Z) > lib.lkv_sparse_gemv_noalloc_max_bytes()
    x = torch.zeros(16, dtype=torch.float16, device=cuda)
    rc = lib.lkv_sparse_gemv_noalloc(x.data_ptr(), x.data_ptr(), 0.1, N, Z, x.data_ptr(), _lib.stream_handle(cuda))
    assert rc == -1 and "scratch" in _lib.last_error()

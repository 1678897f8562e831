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


_CAPTURE_CHILD = r"""
import sys
sys.path.insert(0, sys.argv[1])
import torch
from leankv_amd import _lib

lib = _lib.load()
dev = torch.device("cuda:0")
N, Z = 4096, 14336
g = torch.Generator().manual_seed(3)
W = (torch.randn(N, Z, generator=g) * 0.02).to(torch.float16).to(dev).t().contiguous().t()
x = (torch.randn(Z, generator=g) * 0.05).to(torch.float16).to(dev)
t = float(torch.kthvalue(x.float().abs().cpu(), int(0.4 * Z)).values)
y_ws = torch.empty(N, dtype=torch.float16, device=dev)
nbytes = lib.lkv_sparse_gemv_workspace_bytes(N, Z)
ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
y_na = torch.zeros(N, dtype=torch.float16, device=dev)
torch.cuda.synchronize()
s = torch.cuda.Stream()
s.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
with torch.cuda.stream(s):
    with torch.cuda.graph(graph, stream=s):
        # this process's first lkv_sparse_gemv_noalloc call, made while the stream is being captured
        _lib.check(lib.lkv_sparse_gemv_noalloc(x.data_ptr(), W.data_ptr(), t, N, Z, y_na.data_ptr(),
                                               _lib.stream_handle(dev)), "lkv_sparse_gemv_noalloc")
torch.cuda.current_stream().wait_stream(s)
_lib.check(lib.lkv_sparse_gemv(x.data_ptr(), W.data_ptr(), t, N, Z, y_ws.data_ptr(), ws.data_ptr(), nbytes,
                               _lib.stream_handle(dev)), "lkv_sparse_gemv")
torch.cuda.synchronize()
want = y_ws.clone()
for r in range(3):
    y_na.zero_()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(y_na.view(torch.int16), want.view(torch.int16)), "replay %d differs" % r
    x.mul_(-1)  # eager work between replays; the graph reads x again, so the result flips sign exactly
    _lib.check(lib.lkv_sparse_gemv(x.data_ptr(), W.data_ptr(), t, N, Z, y_ws.data_ptr(), ws.data_ptr(), nbytes,
                                   _lib.stream_handle(dev)), "lkv_sparse_gemv")
    torch.cuda.synchronize()
    want = y_ws.clone()
print("capture ok")
"""


def test_noalloc_first_call_inside_graph_capture(cuda):
    """The entry point is for callers that cannot allocate, graph capture among them: a fresh process whose
    first lkv_sparse_gemv_noalloc call is made inside torch.cuda.graph capture (so the scratch array's address
    is looked up during the capture), the graph replayed three times with eager work between, each replay equal
    bit for bit to lkv_sparse_gemv on the current input."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("noalloc capture case: child process, N=4096 Z=14336", flush=True)
    r = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, root], capture_output=True, text=True, timeout=150)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0 and "capture ok" in r.stdout

"""torch.ops.leankv on the GPU: every registered overload vs the CPU oracle, and the out= overloads captured
in one HIP graph (torch.cuda.graph) and replayed on new inputs.

Tolerances as the kernel tests: projections within 1e-3 relative of fp64 (north star 1e-2), attention within
1e-2, rotations / dequantize within 1e-5, quantized bytes equal to the oracle's except near-tie coordinates.
"""

import numpy as np
import pytest
import torch

import leankv_amd.kernels as K
from oracle import teal as ot
from oracle import turboquant as oq

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3
ATTN_TOL = 1e-2


def _gemv_case(N, Z, seed, q=0.4):
    g = torch.Generator().manual_seed(seed)
    W = (torch.randn(N, Z, generator=g) * 0.02).half()
    x = (torch.randn(Z, generator=g)).half()
    t = ot.threshold_for_sparsity(x.float(), q)
    return W, x, t


def _cm(W, dev):
    return W.to(dev).t().contiguous().t()


def _cache_case(dev, B=1, Hq=32, Hkv=8, L=700, hot=64, seed=0):
    """A 3-bit cache of L tokens built with the oracle (cold codes + fp16 ring) and its reference K/V."""
    c, b = oq.codebook_tensors(3)
    PiK, PiV = oq.rotation_matrix(128, 42), oq.rotation_matrix(128, 43)
    g = torch.Generator().manual_seed(seed)
    Kf = torch.randn(B, Hkv, L, 128, generator=g).half()
    Vf = torch.randn(B, Hkv, L, 128, generator=g).half()
    cold = L - hot
    pk, nk, _ = oq.quantize(Kf[:, :, :cold].float(), PiK, b, 3)
    pv, nv, _ = oq.quantize(Vf[:, :, :cold].float(), PiV, b, 3)
    kh = torch.zeros(B, Hkv, hot, 128, dtype=torch.float16)
    vh = torch.zeros_like(kh)
    for p in range(cold, L):
        kh[:, :, p % hot] = Kf[:, :, p]
        vh[:, :, p % hot] = Vf[:, :, p]
    Kr = torch.cat([oq.dequantize(pk, nk, PiK, c, 3).half(), Kf[:, :, cold:]], dim=2)
    Vr = torch.cat([oq.dequantize(pv, nv, PiV, c, 3).half(), Vf[:, :, cold:]], dim=2)
    d = dict(k_codes=torch.from_numpy(pk).to(dev), k_norms=nk.float().to(dev), v_codes=torch.from_numpy(pv).to(dev),
             v_norms=nv.float().to(dev), k_hot=kh.to(dev), v_hot=vh.to(dev), PiK=PiK.to(dev), PiV=PiV.to(dev),
             c=c.to(dev), b=b[1:-1].contiguous().to(dev))
    return d, Kr, Vr


def _attn_args(d):
    return (d["k_codes"], d["k_norms"], d["v_codes"], d["v_norms"], d["k_hot"], d["v_hot"], d["PiK"], d["PiV"],
            d["c"], 3)


def test_op_sparse_gemv_and_out(cuda):
    W, x, t = _gemv_case(4096, 14336, 1)
    ref = ot.sparse_gemv(x.numpy(), W.numpy(), t)
    y = torch.ops.leankv.sparse_gemv(x.to(cuda), _cm(W, cuda), t)
    assert ot.rel_err(y.cpu().numpy(), ref) < GEMV_TOL
    out = torch.empty(4096, dtype=torch.float16, device=cuda)
    assert torch.ops.leankv.sparse_gemv.out(x.to(cuda), _cm(W, cuda), t, out=out) is out
    assert torch.equal(out, y)


def test_op_sparse_gateup_swiglu_and_out(cuda):
    Wg, x, tg = _gemv_case(14336, 4096, 2)
    Wu, _, _ = _gemv_case(14336, 4096, 3)
    tu = ot.threshold_for_sparsity(x.float(), 0.3)
    ref = ot.gateup_swiglu(x.numpy(), Wg.numpy(), Wu.numpy(), tg, tu)
    h = torch.ops.leankv.sparse_gateup_swiglu(x.to(cuda), _cm(Wg, cuda), _cm(Wu, cuda), tg, tu)
    assert ot.rel_err(h.cpu().numpy(), ref) < GEMV_TOL
    out = torch.empty_like(h)
    torch.ops.leankv.sparse_gateup_swiglu.out(x.to(cuda), _cm(Wg, cuda), _cm(Wu, cuda), tg, tu, out=out)
    assert torch.equal(out, h)


def test_op_sparse_qkv_three_thresholds(cuda):
    """q|k|v of one x in one launch, each projection at its own threshold (patching.py:169-177)."""
    g = torch.Generator().manual_seed(4)
    x = torch.randn(4096, generator=g).half()
    Ws = [(torch.randn(n, 4096, generator=g) * 0.02).half() for n in (4096, 1024, 1024)]
    ts = [ot.threshold_for_sparsity(x.float(), s) for s in (0.31, 0.42, 0.5)]
    outs = torch.ops.leankv.sparse_qkv(x.to(cuda), *[_cm(W, cuda) for W in Ws], *ts)
    for y, W, t in zip(outs, Ws, ts):
        assert ot.rel_err(y.cpu().numpy(), ot.sparse_gemv(x.numpy(), W.numpy(), t)) < GEMV_TOL
    bufs = tuple(torch.empty_like(o) for o in outs)
    got = torch.ops.leankv.sparse_qkv.out(x.to(cuda), *[_cm(W, cuda) for W in Ws], *ts, q=bufs[0], k=bufs[1],
                                          v=bufs[2])
    assert all(a is b for a, b in zip(got, bufs))
    assert all(torch.equal(a, b) for a, b in zip(bufs, outs))
    # different thresholds really select different rows: k at 42 % differs from k at q's 31 %
    k31 = torch.ops.leankv.sparse_gemv(x.to(cuda), _cm(Ws[1], cuda), ts[0])
    assert not torch.equal(k31, outs[1])


def test_op_tq_quantize_dequantize_rotate_rmsnorm(cuda):
    c, b = oq.codebook_tensors(3)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 8, 33, 128, generator=g)
    Pi = oq.rotation_matrix(128, 42)
    p, n = torch.ops.leankv.tq_quantize(x.to(cuda), Pi.to(cuda), b[1:-1].to(cuda), 3)
    p_ref, n_ref, y = oq.quantize(x, Pi, b, 3)
    mism = (p.cpu().numpy() != p_ref).mean()
    assert mism < 1e-3, mism
    torch.testing.assert_close(n.cpu(), n_ref, rtol=2e-6, atol=0)
    pr = torch.ops.leankv.tq_quantize_rotated(y.to(cuda), b[1:-1].to(cuda), 3)
    assert np.array_equal(pr.cpu().numpy(), p_ref)
    dq = torch.ops.leankv.tq_dequantize(torch.from_numpy(p_ref).to(cuda), n_ref.to(cuda), Pi.to(cuda), c.to(cuda), 3)
    torch.testing.assert_close(dq.cpu(), oq.dequantize(p_ref, n_ref, Pi, c, 3), rtol=1e-5, atol=1e-5)
    dq16 = torch.ops.leankv.tq_dequantize(torch.from_numpy(p_ref).to(cuda), n_ref.to(cuda), Pi.to(cuda), c.to(cuda),
                                          3, torch.float16)
    assert dq16.dtype == torch.float16
    r = torch.ops.leankv.tq_rotate(x.to(cuda), Pi.to(cuda), False)
    torch.testing.assert_close(r.cpu().double(), x.double() @ Pi.double().T, rtol=1e-5, atol=1e-5)
    h = (torch.randn(3, 4096, generator=g) * 2).half()
    w = (1 + 0.1 * torch.randn(4096, generator=g)).half()
    y16 = torch.ops.leankv.rms_norm(h.to(cuda), w.to(cuda), 1e-5).cpu()
    h64 = h.double()
    ref = (w.double() * (h64 * torch.rsqrt(h64.pow(2).mean(-1, keepdim=True) + 1e-5)).half().double()).half()
    assert (y16.double() - ref.double()).abs().max() <= 2 * 2 ** -10 * ref.double().abs().max()


def test_op_tq_cache_append_matches_oracle_cache(cuda):
    """Decode appends through the op equal the oracle's cache (cache.py:84-159) in codes, norms and ring."""
    c, b = oq.codebook_tensors(3)
    PiK, PiV = oq.rotation_matrix(128, 42), oq.rotation_matrix(128, 43)
    hot, cap, R = 16, 64, 8
    ref = oq.CacheRef(PiK, PiV, c, b, 3, hot=hot)
    kh = torch.zeros(1, R, hot, 128, dtype=torch.float16, device=cuda)
    vh = torch.zeros_like(kh)
    kc = torch.zeros(1, R, cap, 64, dtype=torch.uint8, device=cuda)
    vc = torch.zeros_like(kc)
    kn = torch.zeros(1, R, cap, dtype=torch.float32, device=cuda)
    vn = torch.zeros_like(kn)
    pos = torch.zeros(1, dtype=torch.int32, device=cuda)
    g = torch.Generator().manual_seed(6)
    for p in range(40):
        k = torch.randn(1, R, 1, 128, generator=g).half()
        v = torch.randn(1, R, 1, 128, generator=g).half()
        ref.update(k, v)
        pos.fill_(p)
        torch.ops.leankv.tq_cache_append(k.view(R, 128).to(cuda), v.view(R, 128).to(cuda), kh, vh, kc, kn, vc, vn,
                                         PiK.to(cuda), PiV.to(cuda), b[1:-1].to(cuda), 3, pos)
    cold = 40 - hot
    pk, nk, pv, nv = ref.cold_arrays()
    assert (kc[:, :, :cold].cpu().numpy() != pk).mean() < 1e-3
    assert (vc[:, :, :cold].cpu().numpy() != pv).mean() < 1e-3
    torch.testing.assert_close(kn[:, :, :cold].cpu(), nk, rtol=2e-6, atol=0)
    torch.testing.assert_close(vn[:, :, :cold].cpu(), nv, rtol=2e-6, atol=0)
    for p in range(cold, 40):
        assert torch.equal(kh[:, :, p % hot].cpu(), ref.hot_k[:, :, p - cold])
        assert torch.equal(vh[:, :, p % hot].cpu(), ref.hot_v[:, :, p - cold])


def test_op_tq_decode_attn_and_out(cuda):
    d, Kr, Vr = _cache_case(cuda, B=2, L=700, seed=7)
    g = torch.Generator().manual_seed(8)
    q = torch.randn(2, 32, 128, generator=g).half()
    seq = torch.tensor([700], dtype=torch.int32, device=cuda)
    out = torch.ops.leankv.tq_decode_attn(q.to(cuda), *_attn_args(d), seq, 700, 128 ** -0.5)
    ref = oq.decode_attention(q.unsqueeze(2), Kr, Vr).squeeze(2)
    assert ot.rel_err(out.cpu().numpy(), ref.numpy()) < ATTN_TOL
    buf = torch.empty_like(out)
    torch.ops.leankv.tq_decode_attn.out(q.to(cuda), *_attn_args(d), seq, 700, 128 ** -0.5, out=buf)
    assert torch.equal(buf, out)


def test_op_tq_prefill_attn_and_out(cuda):
    d, Kr, Vr = _cache_case(cuda, B=1, L=300, seed=9)
    S = 40
    g = torch.Generator().manual_seed(10)
    q = torch.randn(1, 32, S, 128, generator=g).half()
    out = torch.ops.leankv.tq_prefill_attn(q.to(cuda), *_attn_args(d), 300, 128 ** -0.5)
    ref = oq.prefill_attention(q, Kr, Vr)
    assert ot.rel_err(out.cpu().numpy(), ref.numpy()) < ATTN_TOL
    buf = torch.empty_like(out)
    torch.ops.leankv.tq_prefill_attn.out(q.to(cuda), *_attn_args(d), 300, 128 ** -0.5, out=buf)
    assert torch.equal(buf, out)


def test_out_ops_in_a_captured_graph(cuda):
    """The out= overloads captured once (torch.cuda.graph) and replayed on new inputs: each replay equals the
    eager ops on the same inputs bit for bit, with eager work and synchronisation between replays."""
    o = torch.ops.leankv
    W, x, t = _gemv_case(4096, 4096, 11)
    Wg, _, _ = _gemv_case(14336, 4096, 12)
    Wu, _, _ = _gemv_case(14336, 4096, 13)
    Wq = [_cm((torch.randn(n, 4096, generator=torch.Generator().manual_seed(n)) * 0.02).half(), cuda)
          for n in (4096, 1024, 1024)]
    W, Wg, Wu = _cm(W, cuda), _cm(Wg, cuda), _cm(Wu, cuda)
    d, _, _ = _cache_case(cuda, B=1, L=500, seed=14)
    xs = torch.empty(4096, dtype=torch.float16, device=cuda)
    qs = torch.empty(1, 32, 128, dtype=torch.float16, device=cuda)
    qp = torch.empty(1, 32, 16, 128, dtype=torch.float16, device=cuda)
    seq = torch.tensor([500], dtype=torch.int32, device=cuda)
    y = torch.empty(4096, dtype=torch.float16, device=cuda)
    h = torch.empty(14336, dtype=torch.float16, device=cuda)
    qkv = tuple(torch.empty(n, dtype=torch.float16, device=cuda) for n in (4096, 1024, 1024))
    a1 = torch.empty_like(qs)
    a2 = torch.empty_like(qp)

    def body():
        o.sparse_gemv.out(xs, W, t, out=y)
        o.sparse_gateup_swiglu.out(xs, Wg, Wu, t, t, out=h)
        o.sparse_qkv.out(xs, *Wq, t, t, t, q=qkv[0], k=qkv[1], v=qkv[2])
        o.tq_decode_attn.out(qs, *_attn_args(d), seq, 500, 128 ** -0.5, out=a1)
        o.tq_prefill_attn.out(qp, *_attn_args(d), 500, 128 ** -0.5, out=a2)

    def eager():
        return (o.sparse_gemv(xs, W, t), o.sparse_gateup_swiglu(xs, Wg, Wu, t, t), *o.sparse_qkv(xs, *Wq, t, t, t),
                o.tq_decode_attn(qs, *_attn_args(d), seq, 500, 128 ** -0.5),
                o.tq_prefill_attn(qp, *_attn_args(d), 500, 128 ** -0.5))

    gen = torch.Generator(device=cuda).manual_seed(15)

    def new_inputs():
        xs.copy_(torch.randn(4096, generator=gen, device=cuda).half())
        qs.copy_(torch.randn(qs.shape, generator=gen, device=cuda).half())
        qp.copy_(torch.randn(qp.shape, generator=gen, device=cuda).half())

    new_inputs()
    body()  # eager warm-up sizes every workspace before capture
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            body()
    torch.cuda.current_stream().wait_stream(s)
    for r in range(3):
        new_inputs()
        graph.replay()
        torch.cuda.synchronize()
        want = eager()
        got = (y, h, *qkv, a1, a2)
        for i, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(a, b), "replay %d, output %d differs from eager" % (r, i)
        _ = torch.zeros(1000, device=cuda).sum()  # unrelated eager work between replays


@pytest.mark.parametrize("N,Z,rows", [(4096, 14336, 2), (4096, 14336, 16), (14336, 4096, 8), (1024, 4096, 4),
                                      (14336, 4096, 16), (520, 333, 3), (4096, 4096, 12), (4096, 14336, 24),
                                      (1032, 333, 32), (14336, 4096, 32)])
def test_patched_linear_multi_row_is_dense(cuda, N, Z, rows):
    """A TEAL-patched projection called on several decode rows computes the dense product, as the reference's
    dispatch does (leankv/teal/patching.py:169-180), whether it runs on the batched kernel (threshold 0: up to 8
    rows, or 32 unless N > 2 Z) or on torch's F.linear; exact zeros in x contribute nothing either way."""
    import torch.nn as nn

    from leankv_amd.teal.patching import _patch_linear_with_kernel, _skinny_dense

    g = torch.Generator().manual_seed(N + Z + rows)
    lin = nn.Linear(Z, N, bias=False).half()
    with torch.no_grad():
        lin.weight.copy_((torch.randn(N, Z, generator=g) * 0.02).half())
    W = lin.weight.detach().clone()
    lin = lin.to(cuda)
    _patch_linear_with_kernel(lin, 0.5)  # a threshold that would drop ~60 % of the inputs at B = 1
    x = torch.randn(1, rows, Z, generator=g).half()
    x[0, 0, : Z // 3] = 0  # zero inputs in one row
    with torch.no_grad():
        y = lin(x.to(cuda)).cpu()
    ref = np.stack([ot.sparse_gemv(x[0, r].numpy(), W.numpy(), 0.0) for r in range(rows)])  # dense (threshold 0)
    assert tuple(y.shape) == (1, rows, N)
    assert ot.rel_err(y[0].numpy(), ref) < GEMV_TOL
    assert ot.max_rel_err(y[0].numpy(), ref) < 1e-2
    assert _skinny_dense(rows, N, Z) == (rows <= 8 or N <= 2 * Z)

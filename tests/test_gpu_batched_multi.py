"""GPU tests of lkv_sparse_gemm_batched_multi: up to three batched TEAL products of one x [B, Z] in one launch,
with the SwiGLU, the fp16 residual add or RoPE in the chunk reduce (and of
lkv_sparse_gemm_batched_residual_rmsnorm: the residual add and the next RMSNorm), and the TEAL patches that use
it for a few decode rows.  Bar: bit-exact against the single-product calls (lkv_sparse_gemm_batched, whose parity with the oracle
the kernel tests check) followed by torch's own fp16 SwiGLU / add; the dense patched MLP additionally within
1e-2 of an fp32 torch reference."""

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import teal as ot

pytestmark = pytest.mark.gpu


def _weight(N, Z, g, dev):
    """Column-major fp16 W[N, Z] (strides (1, N)), as prepare_weight_for_sparse_gemv lays it out."""
    return (torch.randn(N, Z, generator=g) * 0.02).to(torch.float16).to(dev).t().contiguous().t()


def _x(B, Z, seed, dev):
    torch.manual_seed(seed)
    return torch.distributions.Laplace(0.0, 0.05).sample((B, Z)).to(torch.float16).to(dev)


def _quantile_t(x, q):
    k = int(q * x.shape[1])
    return torch.kthvalue(x[0].float().abs().cpu(), k).values.item() if k > 0 else 0.0


# q|k|v shapes on both kernels (v_dot2 groups below 8 rows, matrix-core groups of 16 from 8), a ragged
# case, a one-chunk case (fp16 written by the GEMM kernel itself) and products whose chunk sizes differ
# (gate-sized next to k-sized: separate launches inside the one call)
CASES = [(2, (4096, 1024, 1024), 4096), (4, (4096, 1024, 1024), 4096), (8, (4096, 1024, 1024), 4096),
         (16, (4096, 1024, 1024), 4096), (11, (1032, 256, 520), 333), (3, (24, 8, 16), 100),
         (5, (14336, 1024), 4096), (24, (4096, 1024, 1024), 4096), (32, (14336, 14336), 4096),
         (37, (1032, 256, 520), 333)]


@pytest.mark.parametrize("B,Ns,Z", CASES)
def test_multi_equals_single_calls(cuda, B, Ns, Z):
    from leankv_amd import kernels

    print("multi case B=%d Ns=%s Z=%d" % (B, Ns, Z), flush=True)
    g = torch.Generator().manual_seed(B * 7 + Z)
    ws = [_weight(N, Z, g, cuda) for N in Ns]
    x = _x(B, Z, B + Z, cuda)
    ts = [_quantile_t(x, q) for q in (0.0, 0.3, 0.5)[:len(Ns)]]
    got = kernels.sparse_gemm_batched_multi(x, ws, ts)
    for w, t, y in zip(ws, ts, got):
        assert torch.equal(y, kernels.sparse_gemm_batched(x, w, t))
    # and the semantics themselves, on the first product
    ref = torch.stack([torch.from_numpy(ot.sparse_gemv(x[b].cpu().numpy(), ws[0].cpu().numpy(), ts[0]))
                       for b in range(B)]).float().numpy()
    assert ot.rel_err(got[0].float().cpu().numpy(), ref) < 1e-3


@pytest.mark.parametrize("B,N,Z,q", [(4, 14336, 4096, 0.0), (16, 14336, 4096, 0.0), (11, 1032, 333, 0.4),
                                     (3, 24, 100, 0.3), (8, 2048, 1000, 0.5), (32, 14336, 4096, 0.0),
                                     (21, 1032, 333, 0.4)])
def test_swiglu_epilogue_equals_torch_on_single_calls(cuda, B, N, Z, q):
    from leankv_amd import kernels

    print("swiglu case B=%d N=%d Z=%d" % (B, N, Z), flush=True)
    g = torch.Generator().manual_seed(N + Z)
    wg, wu = _weight(N, Z, g, cuda), _weight(N, Z, g, cuda)
    x = _x(B, Z, N, cuda)
    tg, tu = _quantile_t(x, q), _quantile_t(x, q / 2)
    (h,) = kernels.sparse_gemm_batched_multi(x, [wg, wu], [tg, tu], kernels.EPI_SWIGLU)
    ref = F.silu(kernels.sparse_gemm_batched(x, wg, tg)) * kernels.sparse_gemm_batched(x, wu, tu)
    assert torch.equal(h, ref)


def test_swiglu_epilogue_every_fp16_gate_value(cuda):
    """All 63488 finite fp16 gate values through the epilogue: x = identity rows make each product one weight
    exactly (fp32 sum of one fp16 term), so the kernel's SwiGLU meets torch's F.silu(g) * u on every input."""
    from leankv_amd import kernels

    B, Z, N = 16, 16, 4096
    vals = torch.from_numpy(np.arange(65536, dtype=np.uint16).view(np.float16))
    vals = torch.where(torch.isfinite(vals), vals, torch.zeros_like(vals))  # 16 x 4096 slots, non-finite -> 0
    gate = vals.view(B, N)
    up = (torch.randn(B, N, generator=torch.Generator().manual_seed(3)) * 4).to(torch.float16)
    # W[n][z] = value for batch row z: the column-major storage A[z][n] is then gate[z][n]
    wg = gate.to(cuda).contiguous().t()
    wu = up.to(cuda).contiguous().t()
    assert wg.shape == (N, Z) and wg.t().is_contiguous()
    x = torch.eye(B, Z, dtype=torch.float16, device=cuda)
    (h,) = kernels.sparse_gemm_batched_multi(x, [wg, wu], [0.0, 0.0], kernels.EPI_SWIGLU)
    assert torch.equal(kernels.sparse_gemm_batched(x, wg, 0.0), gate.to(cuda))  # products are the values
    assert torch.equal(h, F.silu(gate.to(cuda)) * up.to(cuda))


@pytest.mark.parametrize("B,N,Z", [(4, 4096, 4096), (16, 4096, 14336), (11, 1032, 333), (3, 24, 100),
                                   (32, 4096, 14336)])
def test_residual_epilogue_equals_torch_add(cuda, B, N, Z):
    from leankv_amd import kernels

    print("residual case B=%d N=%d Z=%d" % (B, N, Z), flush=True)
    g = torch.Generator().manual_seed(N * 3 + Z)
    w = _weight(N, Z, g, cuda)
    x = _x(B, Z, Z, cuda)
    res = (torch.randn(B, N, generator=g) * 2).to(torch.float16).to(cuda)
    t = _quantile_t(x, 0.4)
    ref = res + kernels.sparse_gemm_batched(x, w, t)
    (y,) = kernels.sparse_gemm_batched_multi(x, [w], [t], kernels.EPI_RESIDUAL, res)
    assert torch.equal(y, ref)
    inplace = res.clone()
    kernels.sparse_gemm_batched_multi_out(x, [w], [t], [inplace], kernels.EPI_RESIDUAL, inplace)
    assert torch.equal(inplace, ref)


# q|k|v at the Mistral shape on both kernels, q and k only, products whose chunk sizes differ (separate
# launches: v must stay unrotated), one chunk with an odd number of heads (a reduce block of one head)
@pytest.mark.parametrize("B,Ns,Z", [(4, (4096, 1024, 1024), 4096), (16, (4096, 1024, 1024), 4096),
                                    (8, (512, 256), 1000), (5, (14336, 1024, 1024), 4096),
                                    (3, (384, 128, 256), 100), (32, (4096, 1024, 1024), 4096)])
def test_rope_epilogue_equals_rope_f16_on_single_calls(cuda, B, Ns, Z):
    from leankv_amd import kernels

    print("rope case B=%d Ns=%s Z=%d" % (B, Ns, Z), flush=True)
    g = torch.Generator().manual_seed(Z + len(Ns))
    ws = [_weight(N, Z, g, cuda) for N in Ns]
    x = _x(B, Z, B * 3 + Z, cuda)
    pos = torch.arange(0, 4096, 37, dtype=torch.float32)[B % 7]
    inv = 1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))
    ang = torch.cat([pos * inv, pos * inv])
    cos, sin = ang.cos().half().to(cuda), ang.sin().half().to(cuda)
    got = kernels.sparse_gemm_batched_multi(x, ws, [0.0] * len(Ns), kernels.EPI_ROPE, cos=cos, sin=sin)
    ref = [kernels.sparse_gemm_batched(x, w, 0.0) for w in ws]
    kernels.rope_f16_(ref[0].view(B, -1, 128), ref[1].view(B, -1, 128), cos, sin)
    for y, r in zip(got, ref):
        assert torch.equal(y, r)


@pytest.mark.parametrize("B,N,Z", [(4, 4096, 4096), (16, 4096, 14336), (3, 8192, 512), (11, 1032, 333),
                                   (5, 24, 100), (2, 64, 0), (32, 4096, 14336)])
def test_residual_rmsnorm_equals_residual_epilogue_then_rms_norm(cuda, B, N, Z):
    """The product, the fp16 residual add and the next RMSNorm with one launch after the product: x_out equals
    the residual epilogue's output and y_out lkv_rmsnorm of it, bit for bit (also in place, x_out = residual;
    Z = 0: the residual itself normalised)."""
    from leankv_amd import kernels

    print("residual+norm case B=%d N=%d Z=%d" % (B, N, Z), flush=True)
    g = torch.Generator().manual_seed(N + 7 * Z)
    w = _weight(N, Z, g, cuda)
    x = _x(B, Z, N + Z, cuda)
    res = (torch.randn(B, N, generator=g) * 2).to(torch.float16).to(cuda)
    nw = (1 + 0.1 * torch.randn(N, generator=g)).to(torch.float16).to(cuda)
    eps = 1e-5
    (ref_x,) = kernels.sparse_gemm_batched_multi(x, [w], [0.0], kernels.EPI_RESIDUAL, res)
    ref_y = kernels.rms_norm(ref_x, nw, eps)
    xo, yo = torch.empty_like(res), torch.empty_like(res)
    kernels.sparse_gemm_batched_residual_rmsnorm_out(x, w, 0.0, res, nw, eps, xo, yo)
    assert torch.equal(xo, ref_x) and torch.equal(yo, ref_y)
    inplace = res.clone()
    kernels.sparse_gemm_batched_residual_rmsnorm_out(x, w, 0.0, inplace, nw, eps, inplace, yo)
    assert torch.equal(inplace, ref_x) and torch.equal(yo, ref_y)


@pytest.mark.parametrize("bits,pos,hot_cap,cap", [(3, 70, 64, 200), (3, 10, 64, 200), (4, 100, 64, 200),
                                                  (2, 64, 64, 200), (1, 130, 32, 98), (3, 300, 64, 200),
                                                  (3, -1, 64, 200)])
def test_evict_and_ring_write_equal_cache_append(cuda, bits, pos, hot_cap, cap):
    """tq_cache_append's two halves, split for the batched decode step: lkv_tq_cache_evict for every layer in one
    launch, then the q/k/v launch writing the new token into the ring (lkv_sparse_gemm_batched_qkv_rope) --
    codes, norms and rings equal tq_cache_append on the same k and v, bit for bit, and q, k, v equal the RoPE
    epilogue's; positions before the window fills, at and after it, past the cold store (no eviction), and a
    negative one (no ring slot: the caches stay as they were)."""
    from leankv_amd import kernels
    from leankv_amd.turboquant.codebook import get_codebook_tensors

    print("evict+ring case bits=%d pos=%d hot=%d cap=%d" % (bits, pos, hot_cap, cap), flush=True)
    B, Hq, Hkv, Z, L = 4, 8, 2, 512, 3
    g = torch.Generator().manual_seed(pos + bits)
    rb = kernels.packed_row_bytes(bits)
    bounds = get_codebook_tensors(128, bits, device=cuda)[1][1:-1].contiguous()
    x = _x(B, Z, pos, cuda)
    pos_dev = torch.tensor([pos], dtype=torch.int32, device=cuda)
    ang = torch.arange(128, dtype=torch.float32) * 0.01 * pos
    cos, sin = ang.cos().half().to(cuda), ang.sin().half().to(cuda)
    caches = []
    for li in range(L):
        ws = [_weight(N, Z, g, cuda) for N in (Hq * 128, Hkv * 128, Hkv * 128)]
        hot = [(torch.randn(B * Hkv, hot_cap, 128, generator=g) * 0.3).half().to(cuda) for _ in range(2)]
        codes = [torch.randint(0, 256, (B * Hkv, cap, rb), generator=g, dtype=torch.uint8).to(cuda) for _ in range(2)]
        norms = [torch.rand(B * Hkv, cap, generator=g).to(cuda) for _ in range(2)]
        Pi = [torch.linalg.qr(torch.randn(128, 128, generator=g))[0].contiguous().to(cuda) for _ in range(2)]
        caches.append((ws, hot, codes, norms, Pi))
    # reference: the RoPE epilogue's q/k/v, then tq_cache_append per layer
    ref = []
    for ws, hot, codes, norms, Pi in caches:
        q, k, v = kernels.sparse_gemm_batched_multi(x, ws, [0.0] * 3, kernels.EPI_ROPE, cos=cos, sin=sin)
        kh, vh, kc, vc = hot[0].clone(), hot[1].clone(), codes[0].clone(), codes[1].clone()
        kn, vn = norms[0].clone(), norms[1].clone()
        kernels.tq_cache_append(k.view(B * Hkv, 128), v.view(B * Hkv, 128), kh, vh, kc, kn, vc, vn, Pi[0], Pi[1],
                                bounds, bits, pos_dev)
        ref.append((q, k, v, kh, vh, kc, kn, vc, vn))
    # split: one evict launch for every layer, then the ring-writing q/k/v launch per layer
    got = [(hot[0].clone(), hot[1].clone(), codes[0].clone(), norms[0].clone(), codes[1].clone(), norms[1].clone())
           for ws, hot, codes, norms, Pi in caches]
    kernels.tq_cache_evict([(gc[2], gc[3], gc[4], gc[5], gc[0], gc[1], c[4][0], c[4][1]) for gc, c in zip(got, caches)],
                           bounds, bits, pos_dev)
    for li, ((ws, hot, codes, norms, Pi), gc) in enumerate(zip(caches, got)):
        outs = [torch.empty(B, w.shape[0], dtype=torch.float16, device=cuda) for w in ws]
        kernels.sparse_gemm_batched_qkv_rope_out(x, ws, cos, sin, outs, gc[0], gc[1], pos_dev)
        q, k, v, kh, vh, kc, kn, vc, vn = ref[li]
        assert torch.equal(outs[0], q) and torch.equal(outs[1], k) and torch.equal(outs[2], v), li
        assert torch.equal(gc[0], kh) and torch.equal(gc[1], vh), li
        assert torch.equal(gc[2], kc) and torch.equal(gc[4], vc), li
        assert torch.equal(gc[3], kn) and torch.equal(gc[5], vn), li
        if pos < 0:
            _, hot, codes, norms, _ = caches[li]
            assert torch.equal(kh, hot[0]) and torch.equal(vh, hot[1]) and torch.equal(kc, codes[0]), li
            assert torch.equal(vc, codes[1]) and torch.equal(kn, norms[0]) and torch.equal(vn, norms[1]), li


def test_empty_sizes(cuda):
    """Z = 0: every product is an empty sum (0; SwiGLU of zeros is 0, the residual add returns the residual);
    B = 0 touches nothing; a zero-column product beside others is skipped."""
    from leankv_amd import kernels

    g = torch.Generator().manual_seed(1)
    x0 = torch.empty(3, 0, dtype=torch.float16, device=cuda)
    w0 = [torch.empty(0, N, dtype=torch.float16, device=cuda).t() for N in (64, 64)]
    outs = [torch.full((3, 64), 7.0, dtype=torch.float16, device=cuda) for _ in range(2)]
    kernels.sparse_gemm_batched_multi_out(x0, w0, [0.0, 0.0], outs)
    assert all(torch.count_nonzero(o) == 0 for o in outs)
    (h,) = kernels.sparse_gemm_batched_multi(x0, w0, [0.0, 0.0], kernels.EPI_SWIGLU)
    assert torch.count_nonzero(h) == 0
    res = torch.randn(3, 64, generator=g).to(torch.float16).to(cuda)
    (y,) = kernels.sparse_gemm_batched_multi(x0, w0[:1], [0.0], kernels.EPI_RESIDUAL, res)
    assert torch.equal(y, res)
    xe = torch.empty(0, 256, dtype=torch.float16, device=cuda)
    assert kernels.sparse_gemm_batched_multi(xe, [_weight(64, 256, g, cuda)], [0.0])[0].shape == (0, 64)
    x = _x(4, 256, 5, cuda)
    wa, wz, wb = _weight(64, 256, g, cuda), _weight(0, 256, g, cuda), _weight(128, 256, g, cuda)
    ya, yz, yb = kernels.sparse_gemm_batched_multi(x, [wa, wz, wb], [0.0, 0.0, 0.0])
    assert yz.shape == (4, 0)
    assert torch.equal(ya, kernels.sparse_gemm_batched(x, wa, 0.0))
    assert torch.equal(yb, kernels.sparse_gemm_batched(x, wb, 0.0))


class _Attn(nn.Module):
    def __init__(self, H, Nq, Nkv):
        super().__init__()
        self.q_proj, self.k_proj, self.v_proj = (nn.Linear(H, n, bias=False) for n in (Nq, Nkv, Nkv))


class _MLP(nn.Module):
    """HF MistralMLP's forward (modeling_mistral.py:46-47)."""

    def __init__(self, H, I):
        super().__init__()
        self.gate_proj, self.up_proj = nn.Linear(H, I, bias=False), nn.Linear(H, I, bias=False)
        self.down_proj = nn.Linear(I, H, bias=False)
        self.act_fn = nn.SiLU()

    def forward(self, x):
        return self.down_proj(self.act_fn(self.gate_proj(x)) * self.up_proj(x))


@pytest.mark.parametrize("B", [4, 16, 32])
def test_patched_qkv_and_mlp_rows(cuda, B):
    """The TEAL patches at B > 1 decode rows (Mistral-7B shapes): q_proj runs the three dense products in one
    launch and k_proj / v_proj hand back theirs, each equal to its own batched call (threshold 0); the fused
    MLP runs gate/up + SwiGLU as one launch, then down: equal to the batched calls followed by torch's SwiGLU,
    and within 1e-2 of the fp32 product."""
    from leankv_amd import kernels
    from leankv_amd.teal.patching import _maybe_patch_mlp, _maybe_patch_qkv, _patch_linear_with_kernel

    print("patched rows case B=%d" % B, flush=True)
    torch.manual_seed(11)
    attn = _Attn(4096, 4096, 1024).half().to(cuda)
    mlp = _MLP(4096, 14336).half().to(cuda)
    for m in (attn.q_proj, attn.k_proj, attn.v_proj, mlp.gate_proj, mlp.up_proj, mlp.down_proj):
        nn.init.normal_(m.weight, std=0.02)
    W32 = {n: p.detach().float().clone() for n, p in mlp.named_parameters()}
    for m in (attn.q_proj, attn.k_proj, attn.v_proj, mlp.gate_proj, mlp.up_proj, mlp.down_proj):
        _patch_linear_with_kernel(m, 0.05)
    _maybe_patch_qkv(attn)
    _maybe_patch_mlp(mlp)
    x = _x(B, 4096, 40 + B, cuda).view(B, 1, 4096)
    with torch.no_grad():
        yq, yk, yv = attn.q_proj(x), attn.k_proj(x), attn.v_proj(x)
        x2 = x.view(B, 4096)
        for y, p in ((yq, attn.q_proj), (yk, attn.k_proj), (yv, attn.v_proj)):
            assert y.shape == (B, 1, p.weight.shape[0])
            assert torch.equal(y.view(B, -1), kernels.sparse_gemm_batched(x2, p.weight, 0.0))
        h = mlp(x)
        a = F.silu(kernels.sparse_gemm_batched(x2, mlp.gate_proj.weight, 0.0)) * \
            kernels.sparse_gemm_batched(x2, mlp.up_proj.weight, 0.0)
        assert torch.equal(h.view(B, -1), mlp.down_proj(a.view(B, 1, -1)).view(B, -1))
        xf = x2.float()
        ref = (F.silu(xf @ W32["gate_proj.weight"].t()) * (xf @ W32["up_proj.weight"].t())) @ W32["down_proj.weight"].t()
    assert ot.rel_err(h.view(B, -1).float().cpu().numpy(), ref.cpu().numpy()) < 1e-2

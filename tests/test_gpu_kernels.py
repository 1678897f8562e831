"""GPU parity tests: HIP kernels (through the C ABI) vs the CPU oracle.

Tolerances (stated by the north star): GEMV / attention outputs within 1e-2
relative (fp16 storage, fp32 accumulate) -- measured as ||a - r|| / ||r|| and
max|a - r| / max|r|; quantized codes and packed bytes bit-exact, except that a
coordinate j whose fp64 rotated value lies within TIE_ULPS * 2^-24 * S_j of a
decision boundary, S_j = sum_k |u_k Pi_jk| (the scale of the fp32 rounding
error of the 128-term rotation, which two correct summation orders may
distribute differently), may round to the neighbouring code; such flips are
counted against a budget.
"""

import math

import numpy as np
import pytest
import torch

from oracle import teal as ot
from oracle import turboquant as oq
from tierule import _codes_match, _rotation_fp64

pytestmark = pytest.mark.gpu

RTOL = 1e-2


def _seeded_gemv(N, Z, seed=0, q=0.4):
    g = torch.Generator().manual_seed(seed)
    W = (torch.randn(N, Z, generator=g) * 0.02).to(torch.float16)
    lap = torch.distributions.Laplace(0.0, 0.05)
    torch.manual_seed(seed)
    x = lap.sample((Z,)).to(torch.float16)
    k = int(q * Z)
    t = torch.kthvalue(x.float().abs(), k).values.item() if k > 0 else 0.0
    return W, x, t


def _gemv(x, W, t, dev):
    from leankv_amd import kernels

    wc = W.to(dev).t().contiguous().t()
    return kernels.sparse_gemv(x.to(dev), wc, t).cpu()


# ----------------------------------------------------------------- TEAL GEMV
def test_sparse_gemv_config1(cuda):
    """Config 1 (single sparse GEMV): W[4096, 14336] ~N(0,.02), x ~Laplace(0,.05), t = 40% quantile."""
    W, x, t = _seeded_gemv(4096, 14336)
    y = _gemv(x, W, t, cuda)
    ref = ot.sparse_gemv(x.numpy(), W.numpy(), t)
    assert ot.rel_err(y.numpy(), ref) < 1e-3
    assert ot.max_rel_err(y.numpy(), ref) < RTOL
    # exactly the intended sparsity: 40% of activations dropped
    # at least the intended 40% dropped (fp16 ties at the threshold drop more)
    assert int((x.float().abs() <= t).sum()) >= int(0.4 * 14336)


@pytest.mark.parametrize("N,Z,q", [(8, 1, 0.0), (24, 1000, 0.5), (1032, 333, 0.3), (4096, 4096, 0.4),
                                   (1024, 4096, 0.4), (14336, 4096, 0.4), (520, 70000, 0.9), (2048, 257, 0.0)])
def test_sparse_gemv_shapes(cuda, N, Z, q):
    W, x, t = _seeded_gemv(N, Z, seed=N + Z, q=q)
    y = _gemv(x, W, t, cuda)
    ref = ot.sparse_gemv(x.numpy(), W.numpy(), t)
    assert ot.rel_err(y.numpy(), ref) < 1e-3
    assert ot.max_rel_err(y.numpy(), ref) < RTOL


def test_sparse_gemv_all_dropped_and_all_kept(cuda):
    W, x, _ = _seeded_gemv(1024, 4096, seed=5)
    y0 = _gemv(x, W, 1e4, cuda)
    assert torch.count_nonzero(y0) == 0
    yd = _gemv(x, W, -1.0, cuda)  # every row kept: dense matvec
    ref = W.double() @ x.double()
    assert ot.rel_err(yd.numpy(), ref.numpy()) < 1e-3


def _batched_case(B, N, Z, q, seed, dev):
    """B Laplace activation rows (each its own mask) against one weight; threshold = the q-quantile of row 0."""
    from leankv_amd import kernels

    g = torch.Generator().manual_seed(seed)
    W = (torch.randn(N, Z, generator=g) * 0.02).to(torch.float16)
    torch.manual_seed(seed)
    X = torch.distributions.Laplace(0.0, 0.05).sample((B, Z)).to(torch.float16)
    k = int(q * Z)
    t = torch.kthvalue(X[0].float().abs(), k).values.item() if k > 0 else 0.0
    wc = W.to(dev).t().contiguous().t()
    Y = kernels.sparse_gemm_batched(X.to(dev), wc, t).cpu()
    ref = np.stack([ot.sparse_gemv(X[b].numpy(), W.numpy(), t) for b in range(B)])
    return Y, ref, X, W, t, wc


# B in 1 .. 40 (the v_dot2 kernel's groups of up to 8 rows below 8 rows, the matrix-core kernel's groups
# of 16 from 8 on and of 32 (two MFMA tiles) from 17 on, a partial last group), single-chunk and
# many-chunk shapes, a ragged N on both kernels, dense (q = 0) and 90 % sparse rows.
@pytest.mark.parametrize("B,N,Z,q", [(2, 4096, 14336, 0.4), (4, 1024, 4096, 0.4), (8, 14336, 4096, 0.4),
                                     (3, 1032, 333, 0.3), (13, 2048, 1000, 0.5), (1, 520, 7000, 0.9),
                                     (5, 24, 257, 0.0), (16, 4096, 4096, 0.4), (24, 1024, 3000, 0.0),
                                     (11, 4096, 14336, 0.4), (9, 1032, 333, 0.3), (8, 24, 100, 0.5),
                                     (24, 4096, 4096, 0.4), (32, 1032, 333, 0.3), (17, 14336, 4096, 0.0),
                                     (40, 1024, 3000, 0.0)])
def test_sparse_gemm_batched(cuda, B, N, Z, q):
    Y, ref, X, W, t, wc = _batched_case(B, N, Z, q, seed=B * 100 + N % 97, dev=cuda)
    assert ot.rel_err(Y.numpy(), ref) < 1e-3
    assert ot.max_rel_err(Y.numpy(), ref) < RTOL


def test_sparse_gemm_batched_rows_equal_single_gemv(cuda):
    """Each output row is that row's own sparse GEMV (fp32 accumulation, up to summation order); a row
    whose activations all fall at or below the threshold gives exactly zero; the other rows keep their
    values (not their last bits: the union of the masks sets the summation order); the reference's
    wrapper (batched_sparse_gemm) routes here."""
    from leankv_amd import kernels
    from leankv_amd.teal.kernels.sparse_gemv import batched_sparse_gemm

    Y, ref, X, W, t, wc = _batched_case(6, 4096, 14336, 0.4, seed=77, dev=cuda)
    for b in range(6):
        yb = kernels.sparse_gemv(X[b].to(cuda), wc, t).cpu()
        assert ot.rel_err(Y[b].numpy(), yb.numpy()) < 1e-3
    Xz = X.clone()
    Xz[2] = 0
    Yz = kernels.sparse_gemm_batched(Xz.to(cuda), wc, t).cpu()
    assert torch.count_nonzero(Yz[2]) == 0
    for b in (0, 1, 3, 4, 5):
        assert ot.rel_err(Yz[b].numpy(), Y[b].numpy()) < 1e-3
    assert torch.equal(batched_sparse_gemm(X.to(cuda), wc, t, 5).cpu(), Y)


def test_sparse_gemv_deterministic_and_reusable_workspace(cuda):
    W, x, t = _seeded_gemv(4096, 14336, seed=9)
    a = _gemv(x, W, t, cuda)
    W2, x2, t2 = _seeded_gemv(1024, 4096, seed=10)
    _gemv(x2, W2, t2, cuda)  # a different shape in between reuses the workspace
    b = _gemv(x, W, t, cuda)
    assert torch.equal(a, b)


def test_gateup_swiglu_config2(cuda):
    """Config 2 (fused MLP): x[4096] ~N(0,1) at 40%, Wg/Wu [14336, 4096], then down at 40% of |h|."""
    from leankv_amd import kernels

    g = torch.Generator().manual_seed(0)
    Wg = (torch.randn(14336, 4096, generator=g) * 0.02).half()
    Wu = (torch.randn(14336, 4096, generator=g) * 0.02).half()
    Wd = (torch.randn(4096, 14336, generator=g) * 0.02).half()
    x = torch.randn(4096, generator=g).half()
    tx = ot.threshold_for_sparsity(x.float(), 0.4)
    h = kernels.sparse_gateup_swiglu(x.to(cuda), Wg.to(cuda).t().contiguous().t(),
                                     Wu.to(cuda).t().contiguous().t(), tx, tx).cpu()
    href = ot.gateup_swiglu(x.numpy(), Wg.numpy(), Wu.numpy(), tx, tx)
    assert ot.rel_err(h.numpy(), href) < 2e-3
    assert ot.max_rel_err(h.numpy(), href) < RTOL
    th = ot.threshold_for_sparsity(torch.from_numpy(href.astype(np.float32)), 0.4)
    y = kernels.sparse_gemv(torch.from_numpy(href).to(cuda), Wd.to(cuda).t().contiguous().t(), th).cpu()
    yref = ot.sparse_gemv(href, Wd.numpy(), th)
    assert ot.rel_err(y.numpy(), yref) < 1e-3


def test_gateup_distinct_thresholds(cuda):
    from leankv_amd import kernels

    g = torch.Generator().manual_seed(1)
    Wg = (torch.randn(1024, 512, generator=g) * 0.05).half()
    Wu = (torch.randn(1024, 512, generator=g) * 0.05).half()
    x = torch.randn(512, generator=g).half()
    h = kernels.sparse_gateup_swiglu(x.to(cuda), Wg.to(cuda).t().contiguous().t(),
                                     Wu.to(cuda).t().contiguous().t(), 0.3, 0.9).cpu()
    href = ot.gateup_swiglu(x.numpy(), Wg.numpy(), Wu.numpy(), 0.3, 0.9)
    assert ot.max_rel_err(h.numpy(), href) < RTOL


def test_sparse_gemv_partials_reduce_to_the_full_op(cuda):
    """Split-K partials, summed over chunks in chunk order and rounded, equal the full op bit for bit."""
    from leankv_amd import kernels

    g = torch.Generator().manual_seed(11)
    N, Z = 1024, 4096
    Wg = (torch.randn(N, Z, generator=g) * 0.02).half().to(cuda).t().contiguous().t()
    Wu = (torch.randn(N, Z, generator=g) * 0.02).half().to(cuda).t().contiguous().t()
    x = torch.randn(Z, generator=g).half().to(cuda)
    p1 = kernels.sparse_gemv_partials(x, Wg, 0.5)
    assert p1.shape[:2] == (1, N // 256) and p1.shape[2] > 1

    def reduce(p):  # p: [slabs, chunks, 256]
        acc = torch.zeros(p.shape[0], p.shape[2], dtype=torch.float32, device=cuda)
        for c in range(p.shape[1]):  # chunk order, from 0, like the kernels
            acc = acc + p[:, c]
        return acc.reshape(-1)

    assert torch.equal(reduce(p1[0]).half(), kernels.sparse_gemv(x, Wg, 0.5))
    p2 = kernels.sparse_gemv_partials(x, Wg, 0.4, Wu, 0.7)
    assert torch.equal(p2[0], kernels.sparse_gemv_partials(x, Wg, 0.4)[0])
    h = kernels.sparse_gateup_swiglu(x, Wg, Wu, 0.4, 0.7)
    gsum, usum = reduce(p2[0]).cpu().numpy(), reduce(p2[1]).cpu().numpy()
    ref = ot.silu_f16(gsum.astype(np.float16)).astype(np.float32) * usum.astype(np.float16).astype(np.float32)
    ref = ref.astype(np.float16)
    # same sums; SwiGLU's exp may differ by an ulp between numpy and the device, nothing more
    assert ot.max_rel_err(h.cpu().numpy(), ref) < 2e-3
    assert int((h.cpu().numpy() != ref).sum()) <= N // 100


@pytest.mark.parametrize("M,Z", [(1, 4096), (3, 512), (2, 14336)])
def test_rms_norm_matches_hf_rounding(cuda, M, Z):
    """lkv_rmsnorm vs HF MistralRMSNorm in fp64 (modeling_mistral.py:190-197): every element within one
    fp16 ulp of the fp64-exact RMSNorm, the fp16 product with the weight as HF rounds it."""
    from leankv_amd import kernels

    g = torch.Generator().manual_seed(M * Z)
    x = (torch.randn(M, Z, generator=g) * 3).half()
    w = (1 + 0.1 * torch.randn(Z, generator=g)).half()
    y = kernels.rms_norm(x.to(cuda), w.to(cuda), 1e-5).cpu()
    x64 = x.double()
    u = (x64 * torch.rsqrt(x64.pow(2).mean(-1, keepdim=True) + 1e-5)).half()  # exact rstd, fp16 cast
    ref = (w.double() * u.double()).half()
    ulp = torch.finfo(torch.float16).eps * ref.double().abs().clamp_min(2 ** -14)
    assert ((y.double() - ref.double()).abs() <= 2 * ulp).all()
    assert (y != ref).float().mean() < 0.02  # almost all bit-equal; the rest one rounding step apart


@pytest.mark.parametrize("B,Hq,Hkv,pos", [(1, 32, 8, 0), (4, 32, 8, 777), (16, 32, 8, 4095), (3, 8, 2, 12345)])
def test_rope_f16_equals_hf_apply_rotary_pos_emb(cuda, B, Hq, Hkv, pos):
    """lkv_rope_f16 (in place, q and k in one launch) vs transformers' own apply_rotary_pos_emb on the same fp16
    tensors and the model's rotary factors at `pos` (modeling_mistral.py:51-81), bit for bit; a Llama-scaled
    rotary embedding too."""
    from transformers import LlamaConfig, MistralConfig
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
    from transformers.models.mistral.modeling_mistral import MistralRotaryEmbedding, apply_rotary_pos_emb

    from leankv_amd import kernels

    cfgs = [(MistralRotaryEmbedding, MistralConfig(hidden_size=Hq * 128, num_attention_heads=Hq,
                                                   num_key_value_heads=Hkv, rope_theta=1e6)),
            (LlamaRotaryEmbedding, LlamaConfig(hidden_size=Hq * 128, num_attention_heads=Hq, num_key_value_heads=Hkv,
                                               max_position_embeddings=131072,
                                               rope_scaling={"rope_type": "llama3", "factor": 8.0,
                                                             "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                                                             "original_max_position_embeddings": 8192}))]
    g = torch.Generator().manual_seed(B * 1000 + pos)
    for cls, cfg in cfgs:
        rot = cls(config=cfg).to(cuda)
        dummy = torch.zeros(1, 1, 128, device=cuda, dtype=torch.float16)
        cos, sin = rot(dummy, torch.tensor([[pos]], device=cuda))  # [1, 1, 128] fp16
        q = (torch.randn(B, Hq, 1, 128, generator=g) * 4).half().to(cuda)
        k = (torch.randn(B, Hkv, 1, 128, generator=g) * 4).half().to(cuda)
        q_ref, k_ref = apply_rotary_pos_emb(q, k, cos, sin)
        qk, kk = q.reshape(B, Hq, 128).clone(), k.reshape(B, Hkv, 128).clone()
        kernels.rope_f16_(qk, kk, cos.reshape(-1).contiguous(), sin.reshape(-1).contiguous())
        assert torch.equal(qk, q_ref.reshape(B, Hq, 128)), cls.__name__
        assert torch.equal(kk, k_ref.reshape(B, Hkv, 128)), cls.__name__


# ----------------------------------------------------------------- TurboQuant
def _kv(shape, seed, outliers=(0, 31, 64, 127)):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    x[..., list(outliers)] *= 10
    return x.half()


def _quantize_check(x, Pi, b, bits, p, n):
    """GPU codes p and norms n vs the oracle.  fp16 input: the norm is an fp32 sum rounded to fp16, so where the
    kernel's and torch's summation orders round to neighbouring fp16 values (a norm tie) the unit vector differs
    by fp16 ulps; such rows are charged to the budget and checked against the oracle run with the kernel's
    norm.  Returns (#code flips, #norm-tie rows)."""
    p_ref, n_ref, _ = oq.quantize(x, Pi, b, bits)
    if x.dtype == torch.float16:
        same = (n == n_ref).numpy()
        if not same.all():
            nm, nr = n[~same].float(), n_ref[~same].float()
            ulp = torch.finfo(torch.float16).eps * nr.abs()
            assert ((nm - nr).abs() <= ulp * 1.0001).all(), "fp16 norms more than one rounding step apart"
            exact = x[~same].double().norm(dim=-1)
            assert ((exact - nr.double()).abs() <= ulp.double()).all()
            assert ((exact - nm.double()).abs() <= ulp.double()).all()
    else:
        torch.testing.assert_close(n.float(), n_ref.float(), rtol=2e-6, atol=0)
        same = np.ones(n.shape, dtype=bool)
    y64, S = _rotation_fp64(x, Pi)
    flips = _codes_match(p[same], p_ref[same], y64[same], S[same], b, bits)
    ties = int((~same).sum())
    if ties:
        xt = x[torch.from_numpy(~same)]
        n_tie = n[torch.from_numpy(~same)]  # the oracle's steps with the kernel's norm
        u = xt / (n_tie.unsqueeze(-1) + 1e-10)
        idx = torch.searchsorted(b[1:-1].contiguous(), torch.matmul(u.float(), Pi.T).contiguous())
        p_tie = oq.pack_indices(idx.numpy(), bits)
        y64t, St = _rotation_fp64(xt, Pi, norms=n_tie)
        flips += _codes_match(p[~same], p_tie, y64t, St, b, bits)
    return flips, ties


@pytest.mark.parametrize("in_dtype", [torch.float32, torch.float16])
def test_tq_quantize_config3(cuda, in_dtype):
    """Config 3 (TurboQuant quantize): K,V [8, 4096, 128] ~N(0,1), channels {0,31,64,127} x10, Pi seeds 42/43."""
    from leankv_amd import kernels

    c, b = oq.codebook_tensors(3)
    flips = ties = 0
    for seed, pseed in ((0, 42), (1, 43)):
        x = _kv((8, 4096, 128), seed).to(in_dtype)
        Pi = oq.rotation_matrix(128, pseed)
        p, n = kernels.tq_quantize(x.to(cuda), Pi.to(cuda), b[1:-1].to(cuda), 3)
        p, n = p.cpu().numpy(), n.cpu()
        assert p.shape == (8, 4096, 64) and n.dtype == in_dtype
        f, t = _quantize_check(x, Pi, b, 3, p, n)
        flips, ties = flips + f, ties + t
    print("config 3 %s: %d near-tie code flips in 8.4M coordinates, %d norm-tie rows of 65536" % (in_dtype, flips, ties))
    # measured: 3 flips (fp32 and fp16 input), 8 norm-tie rows (fp16)
    assert flips + ties <= 24, (flips, ties)


@pytest.mark.parametrize("bits", [1, 2, 4])
def test_tq_quantize_other_bits(cuda, bits):
    from leankv_amd import kernels

    c, b = oq.codebook_tensors(bits)
    x = _kv((3, 77, 128), 7).float()
    Pi = oq.rotation_matrix(128, 50)
    p, n = kernels.tq_quantize(x.to(cuda), Pi.to(cuda), b[1:-1].to(cuda), bits)
    flips, _ = _quantize_check(x, Pi, b, bits, p.cpu().numpy(), n.cpu())
    assert flips <= 2


def test_tq_quantize_zero_vector_and_ragged_rows(cuda):
    from leankv_amd import kernels

    c, b = oq.codebook_tensors(3)
    x = torch.randn(37, 128)
    x[5] = 0
    Pi = oq.rotation_matrix(128, 42)
    p, n = kernels.tq_quantize(x.to(cuda), Pi.to(cuda), b[1:-1].to(cuda), 3)
    assert _quantize_check(x, Pi, b, 3, p.cpu().numpy(), n.cpu())[0] <= 2
    assert n[5].item() == 0
    # y = 0 -> code = #(boundaries < 0) = 3 in every coordinate
    assert (oq.unpack_indices(p.cpu().numpy()[5], 3, 128) == 3).all()


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_tq_quantize_rotated_bit_exact(cuda, bits):
    from leankv_amd import kernels

    c, b = oq.codebook_tensors(bits)
    g = torch.Generator().manual_seed(bits)
    y = torch.randn(4099, 128, generator=g) * 0.09
    y[0, : (1 << bits) - 1] = b[1:-1]  # exactly on the boundaries -> lower code
    p = kernels.tq_quantize_rotated(y.to(cuda), b[1:-1].to(cuda), bits).cpu().numpy()
    idx = torch.searchsorted(b[1:-1].contiguous(), y)
    assert np.array_equal(p, oq.pack_indices(idx.numpy(), bits))


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_tq_dequantize(cuda, bits):
    from leankv_amd import kernels

    c, b = oq.codebook_tensors(bits)
    x = _kv((4, 300, 128), 3).float()
    Pi = oq.rotation_matrix(128, 44)
    p_ref, n_ref, _ = oq.quantize(x, Pi, b, bits)
    ref = oq.dequantize(p_ref, n_ref, Pi, c, bits)
    out = kernels.tq_dequantize(torch.from_numpy(p_ref).to(cuda), n_ref.to(cuda), Pi.to(cuda), c.to(cuda), bits,
                                out_dtype=torch.float32).cpu()
    torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)
    out16 = kernels.tq_dequantize(torch.from_numpy(p_ref).to(cuda), n_ref.to(cuda), Pi.to(cuda), c.to(cuda), bits,
                                  out_dtype=torch.float16).cpu()
    torch.testing.assert_close(out16, ref.half(), rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("transpose", [False, True])
def test_tq_rotate(cuda, transpose):
    from leankv_amd import kernels

    x = torch.randn(333, 128)
    Pi = oq.rotation_matrix(128, 45)
    ref = x.double() @ (Pi.double() if transpose else Pi.double().T)
    y = kernels.tq_rotate(x.to(cuda), Pi.to(cuda), transpose).cpu()
    torch.testing.assert_close(y.double(), ref, rtol=1e-5, atol=1e-5)
    yh = kernels.tq_rotate(x.half().to(cuda), Pi.to(cuda), transpose).cpu()
    torch.testing.assert_close(yh.double(), x.half().double() @ (Pi.double() if transpose else Pi.double().T),
                               rtol=1e-5, atol=1e-5)


# ----------------------------------------------------------- TurboQuantProd (QJL)
def _prod_tables(mb, seed=42):
    c, b = oq.codebook_tensors(mb)
    return oq.rotation_matrix(128, seed), oq.qjl_matrix(128, seed + 1000), c, b


def test_tq_prod_matches_reference_golden(cuda):
    """TurboQuantProd on the GPU reproduces the reference's recorded outputs (tests/golden/make_qjl_golden.py)."""
    import json
    import os

    from leankv_amd.turboquant.quantizer import TurboQuantProd

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qjl_prod_cases.json")
    for c in json.load(open(path)):
        print("golden case bits=%d %s" % (c["bits"], c["dtype"]), flush=True)
        tq = TurboQuantProd(128, bits=c["bits"], device=cuda, seed=42)
        x = torch.tensor(c["x"]).to(getattr(torch, c["dtype"])).to(cuda)
        q = tq.quantize(x)
        assert q.mse_bits == c["mse_bits"] and q.norms.dtype == x.dtype
        assert np.array_equal(q.mse_indices.cpu().numpy(), np.array(c["mse_indices"], np.uint8))
        assert np.array_equal(q.qjl_signs.cpu().numpy(), np.array(c["qjl_signs"], np.uint8))
        torch.testing.assert_close(q.norms.float().cpu(), torch.tensor(c["norms"]), rtol=2e-6, atol=0)
        torch.testing.assert_close(q.residual_norms.cpu(), torch.tensor(c["residual_norms"]), rtol=1e-5, atol=0)
        out = tq.dequantize(q).cpu()
        assert out.dtype == torch.float32
        torch.testing.assert_close(out, torch.tensor(c["dequantized"]), rtol=1e-5, atol=1e-5)


def _prod_case(x, mb, cuda, seed=42):
    """GPU quantize of x vs (a) the separate MSE / rotate kernels, bit for bit, and (b) the oracle, with
    near-tie codes and signs counted; returns (#code flips, #sign flips)."""
    from leankv_amd import kernels

    Pi, S, c, b = _prod_tables(mb, seed)
    xd = x.to(cuda)
    codes, norms, signs, rn = kernels.tq_prod_quantize(xd, Pi.to(cuda), b[1:-1].to(cuda), c.to(cuda), S.to(cuda), mb)
    # (a) the fused kernel == quantize, dequantize and rotate run one after another
    c2, n2 = kernels.tq_quantize(xd, Pi.to(cuda), b[1:-1].to(cuda), mb)
    assert torch.equal(codes, c2) and torch.equal(norms, n2)
    xh = kernels.tq_dequantize(codes, norms, Pi.to(cuda), c.to(cuda), mb, out_dtype=torch.float32)
    r = xd.float() - xh
    proj = kernels.tq_rotate(r, S.to(cuda), False)
    assert np.array_equal(signs.cpu().numpy(), oq.pack_signs(proj.cpu().numpy()))
    torch.testing.assert_close(rn, r.norm(dim=-1), rtol=1e-5, atol=1e-30)
    # (b) the oracle
    codes, norms, signs, rn = codes.cpu().numpy(), norms.cpu(), signs.cpu().numpy(), rn.cpu()
    p_ref, n_ref, s_ref, rn_ref, proj_ref = oq.prod_quantize(x, Pi, b, c, S, mb)
    if x.dtype == torch.float16:
        same = (norms == n_ref).numpy()  # an fp16 norm can round the other way (see the config-3 test)
        assert (~same).sum() <= 1e-3 * same.size
    else:
        torch.testing.assert_close(norms, n_ref, rtol=2e-6, atol=0)
        same = np.ones(norms.shape, dtype=bool)
    y64, S = _rotation_fp64(x, Pi)
    flips = _codes_match(codes[same], p_ref[same], y64[same], S[same], b, mb)
    ok = same & (oq.unpack_indices(codes, mb, 128) == oq.unpack_indices(p_ref, mb, 128)).all(-1)
    torch.testing.assert_close(rn[ok], rn_ref[ok], rtol=1e-5, atol=1e-30)
    sg = oq.unpack_signs(signs[ok])
    sr = oq.unpack_signs(s_ref[ok])
    band = 1e-5 * x.float().norm(dim=-1).numpy()[ok][:, None]
    sdiff = sg != sr
    assert not (sdiff & (np.abs(proj_ref.double().numpy()[ok]) >= band)).any(), "sign flip away from zero"
    return flips, int(sdiff.sum())


@pytest.mark.parametrize("mb", [1, 2, 3, 4])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_tq_prod_quantize(cuda, mb, dtype):
    x = _kv((4, 1000, 128), 20 + mb).to(dtype)
    flips, sflips = _prod_case(x, mb, cuda)
    assert flips <= 8 and sflips <= 8, (flips, sflips)


def test_tq_prod_quantize_ragged_zero_and_empty(cuda):
    from leankv_amd import kernels

    x = torch.randn(37, 128)
    x[5] = 0
    _prod_case(x, 2, cuda)
    Pi, S, c, b = _prod_tables(2)
    codes, norms, signs, rn = kernels.tq_prod_quantize(x.to(cuda), Pi.to(cuda), b[1:-1].to(cuda), c.to(cuda),
                                                       S.to(cuda), 2)
    # a zero vector: norm 0, every code = #(boundaries < 0), x_hat = 0, residual 0, no sign bit set
    assert norms[5].item() == 0 and rn[5].item() == 0 and int(signs[5].sum()) == 0
    assert (oq.unpack_indices(codes.cpu().numpy()[5], 2, 128) == int((b[1:-1] < 0).sum())).all()
    e = kernels.tq_prod_quantize(torch.empty(0, 128, device=cuda), Pi.to(cuda), b[1:-1].to(cuda), c.to(cuda),
                                 S.to(cuda), 2)
    assert e[0].shape == (0, 32) and e[2].shape == (0, 16)


@pytest.mark.parametrize("mb", [1, 2, 3, 4])
def test_tq_prod_dequantize(cuda, mb):
    from leankv_amd import kernels

    Pi, S, c, b = _prod_tables(mb, 7)
    x = _kv((3, 333, 128), 30 + mb).float()
    p, n, s, rn, _ = oq.prod_quantize(x, Pi, b, c, S, mb)
    ref = oq.prod_dequantize(p, n, s, rn, Pi, c, S, mb)
    scale = math.sqrt(math.pi / 2) / 128
    args = (torch.from_numpy(p).to(cuda), n.to(cuda), torch.from_numpy(s).to(cuda), rn.to(cuda), Pi.to(cuda),
            c.to(cuda), S.to(cuda), mb, scale)
    out = kernels.tq_prod_dequantize(*args).cpu()
    torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)
    out16 = kernels.tq_prod_dequantize(*args, out_dtype=torch.float16).cpu()
    torch.testing.assert_close(out16, ref.half(), rtol=2e-3, atol=2e-3)
    # fp16 norms (an fp16 input's quantization) read as their fp32 values
    out_h = kernels.tq_prod_dequantize(args[0], n.half().to(cuda), *args[2:]).cpu()
    ref_h = oq.prod_dequantize(p, n.half(), s, rn, Pi, c, S, mb)
    torch.testing.assert_close(out_h, ref_h, rtol=1e-5, atol=1e-5)


def test_wrappers_keep_converted_operands_alive(cuda):
    """Non-contiguous Pi / S views (a QR factor is column-major) are copied by the wrappers; each copy
    must stay alive until the launch, or the next copy reuses its memory.  Results equal those of
    contiguous operands bit for bit."""
    from leankv_amd import kernels

    Pi, S, c, b = _prod_tables(2)
    Pn = Pi.t().contiguous().t().to(cuda)  # column-major views
    Sn = S.t().contiguous().t().to(cuda)
    Pc, Sc = Pi.contiguous().to(cuda), S.contiguous().to(cuda)
    assert not Pn.is_contiguous() and not Sn.is_contiguous()
    x = _kv((2, 300, 128), 50).to(cuda)
    a = kernels.tq_prod_quantize(x, Pn, b[1:-1], c, Sn, 2)
    r = kernels.tq_prod_quantize(x, Pc, b[1:-1].to(cuda), c.to(cuda), Sc, 2)
    assert all(torch.equal(u, v) for u, v in zip(a, r))
    scale = math.sqrt(math.pi / 2) / 128
    d1 = kernels.tq_prod_dequantize(*r, Pn, c, Sn, 2, scale)
    d2 = kernels.tq_prod_dequantize(*r, Pc, c.to(cuda), Sc, 2, scale)
    assert torch.equal(d1, d2)


def test_tq_prod_full_size(cuda):
    """Config-3 shape (K and V fp16 [8, 4096, 128], 4 channels x10): the fused kernel equals the separate
    kernels bit for bit, and the sketch halves the inner-product error of the MSE part alone."""
    from leankv_amd.turboquant.quantizer import TurboQuantProd

    x = _kv((8, 4096, 128), 40).to(cuda)
    flips, sflips = _prod_case(x[:1].cpu(), 2, cuda)  # oracle on one head (4096 vectors)
    assert flips <= 8 and sflips <= 8
    tq = TurboQuantProd(128, bits=3, device=cuda, seed=42)
    q = tq.quantize(x)
    from leankv_amd import kernels

    m = tq.mse_quantizer
    c2, n2 = kernels.tq_quantize(x, m.Pi, m.decision_boundaries, 2)
    assert torch.equal(q.mse_indices, c2) and torch.equal(q.norms, n2)
    xh = kernels.tq_dequantize(c2, n2, m.Pi, m.centroids, 2, out_dtype=torch.float32)
    proj = kernels.tq_rotate(x.float() - xh, tq.S, False)
    assert np.array_equal(q.qjl_signs.cpu().numpy(), oq.pack_signs(proj.cpu().numpy()))
    # inner products with random queries: the QJL-corrected estimate has no systematic shrinkage
    g = torch.Generator(device=cuda).manual_seed(1)
    y = torch.randn(64, 128, generator=g, device=cuda)
    xf = x.float().reshape(-1, 128)
    est = tq.dequantize(q).reshape(-1, 128)
    true = y @ xf.T
    err_prod = (y @ est.T - true)
    err_mse = (y @ xh.reshape(-1, 128).T - true)
    assert abs(err_prod.mean().item()) < 0.02 * true.std().item()
    # the MSE estimate is shrunk toward zero (slope < 1); the corrected one is not
    slope_mse = float((err_mse.flatten() * true.flatten()).sum() / (true.flatten() ** 2).sum())
    slope_prod = float((err_prod.flatten() * true.flatten()).sum() / (true.flatten() ** 2).sum())
    assert slope_mse < -0.05 and abs(slope_prod) < 0.02, (slope_mse, slope_prod)


def test_tq_cache_append_matches_reference_cache(cuda):
    """Static ring append == TurboQuantCache.update hot/cold semantics (cache.py:84-159)."""
    from leankv_amd import kernels

    c, b = oq.codebook_tensors(3)
    PiK, PiV = oq.rotation_matrix(128, 42), oq.rotation_matrix(128, 43)
    B, H, hot, cap, steps = 2, 3, 8, 64, 30
    ref = oq.CacheRef(PiK, PiV, c, b, 3, hot=hot)
    kh = torch.zeros(B, H, hot, 128, dtype=torch.float16, device=cuda)
    vh = torch.zeros_like(kh)
    kc = torch.zeros(B, H, cap, 64, dtype=torch.uint8, device=cuda)
    vc = torch.zeros_like(kc)
    kn = torch.zeros(B, H, cap, device=cuda)
    vn = torch.zeros_like(kn)
    pos = torch.zeros(1, dtype=torch.int32, device=cuda)
    PiKd, PiVd, bd = PiK.to(cuda), PiV.to(cuda), b[1:-1].contiguous().to(cuda)
    g = torch.Generator().manual_seed(0)
    ks, vs = [], []
    for s in range(steps):
        k = torch.randn(B, H, 1, 128, generator=g).half()
        v = torch.randn(B, H, 1, 128, generator=g).half()
        ks.append(k)
        vs.append(v)
        ref.update(k, v)
        kernels.tq_cache_append(k.to(cuda), v.to(cuda), kh, vh, kc, kn, vc, vn, PiKd, PiVd, bd, 3, pos)
        pos += 1
    ncold = steps - hot
    pk, nk, pv, nv = ref.cold_arrays()
    assert pk.shape[2] == ncold
    allk, allv = torch.cat(ks, dim=2), torch.cat(vs, dim=2)
    for got, want, nrm_g, nrm_w, Pi, src in ((kc, pk, kn, nk, PiK, allk), (vc, pv, vn, nv, PiV, allv)):
        y64, S = _rotation_fp64(src[:, :, :ncold].float(), Pi)
        assert _codes_match(got[:, :, :ncold].cpu().numpy(), want, y64, S, b, 3) <= 2
        torch.testing.assert_close(nrm_g[:, :, :ncold].cpu(), nrm_w.float(), rtol=2e-6, atol=0)
    # the bulk quantizer (one wave per 16-vector tile) gives the append path's
    # codes and norms bit for bit: both run the same per-output MFMA chain
    for got, nrm_g, Pi, src in ((kc, kn, PiKd, allk), (vc, vn, PiVd, allv)):
        pq, nq = kernels.tq_quantize(src[:, :, :ncold].float().contiguous().to(cuda), Pi, bd, 3)
        assert torch.equal(pq, got[:, :, :ncold])
        assert torch.equal(nq, nrm_g[:, :, :ncold])
    # rows beyond the cold length were never written
    assert int(kc[:, :, ncold:].count_nonzero()) == 0
    # hot ring holds the last `hot` tokens at slot p % hot
    hk = kh.cpu()
    for j in range(hot):
        p = steps - hot + j
        assert torch.equal(hk[:, :, p % hot], ref.hot_k[:, :, j])


# ----------------------------------------------------------------- attention
# packed row bytes per bit width (quantizer.py:38-62: 8 / 4 / 2 codes per byte)
_ROW_BYTES = {1: 16, 2: 32, 3: 64, 4: 64}


def _attn_case(B, Hq, Hkv, L, hot, seed, dev, bits=3):
    """Build a cache of L tokens (cold = L - hot) with the oracle, run the HIP kernel."""
    from leankv_amd import kernels

    c, b = oq.codebook_tensors(bits)
    PiK, PiV = oq.rotation_matrix(128, 42), oq.rotation_matrix(128, 43)
    cold = max(0, L - hot)
    hot_len = L - cold
    K = _kv((B, Hkv, L, 128), seed)
    V = _kv((B, Hkv, L, 128), seed + 1000)
    q = torch.randn(B, Hq, 128, generator=torch.Generator().manual_seed(seed + 7)).half()
    cap = max(cold, 1)
    kc = torch.zeros(B, Hkv, cap, _ROW_BYTES[bits], dtype=torch.uint8)
    vc = torch.zeros_like(kc)
    kn = torch.zeros(B, Hkv, cap)
    vn = torch.zeros_like(kn)
    Kref, Vref = K.clone(), V.clone()
    if cold:
        pk, nk, _ = oq.quantize(K[:, :, :cold].float(), PiK, b, bits)
        pv, nv, _ = oq.quantize(V[:, :, :cold].float(), PiV, b, bits)
        kc[:, :, :cold] = torch.from_numpy(pk)
        vc[:, :, :cold] = torch.from_numpy(pv)
        kn[:, :, :cold] = nk
        vn[:, :, :cold] = nv
        Kref[:, :, :cold] = oq.dequantize(pk, nk, PiK, c, bits).half()
        Vref[:, :, :cold] = oq.dequantize(pv, nv, PiV, c, bits).half()
    kh = torch.zeros(B, Hkv, hot, 128, dtype=torch.float16)
    vh = torch.zeros_like(kh)
    for j in range(hot_len):
        p = cold + j
        kh[:, :, p % hot] = K[:, :, p]
        vh[:, :, p % hot] = V[:, :, p]
    seq = torch.tensor([L], dtype=torch.int32, device=dev)
    out = kernels.tq_decode_attn(q.to(dev), kc.to(dev), kn.to(dev), vc.to(dev), vn.to(dev), kh.to(dev), vh.to(dev),
                                 PiK.to(dev), PiV.to(dev), c.to(dev), bits, seq, L).cpu()
    ref = oq.decode_attention(q.unsqueeze(2), Kref, Vref).squeeze(2)
    return out, ref


@pytest.mark.parametrize("B", [1, 4, 16])
def test_decode_attn_config4(cuda, B):
    """Config 4 (packed-KV decode attention): 32 q heads over 8 kv heads, ctx 4096 cold + 64-token fp16 hot tail."""
    out, ref = _attn_case(B, 32, 8, 4096 + 64, 64, seed=B, dev=cuda)
    assert ot.rel_err(out.numpy(), ref.numpy()) < RTOL
    assert ot.max_rel_err(out.numpy(), ref.numpy()) < RTOL


@pytest.mark.parametrize("B,Hq,Hkv,L,hot", [(1, 32, 8, 1, 64), (1, 32, 8, 64, 64), (1, 32, 8, 65, 64),
                                            (2, 8, 8, 1000, 64), (1, 16, 2, 333, 16), (3, 32, 4, 4096, 64),
                                            (1, 64, 4, 2048, 64)])
def test_decode_attn_edges(cuda, B, Hq, Hkv, L, hot):
    out, ref = _attn_case(B, Hq, Hkv, L, hot, seed=L, dev=cuda)
    assert ot.rel_err(out.numpy(), ref.numpy()) < RTOL
    assert ot.max_rel_err(out.numpy(), ref.numpy()) < RTOL


# Every packing the cache stores (1 and 2 bits: 8 / 4 codes per byte, widened to nibbles in registers;
# 4 bits: the LDS table) and hot windows past one 64-slot group (128, 200, 256 slots; the window full
# and partly filled), including config 4 at 2 bits (the reference sweep's 2.5-bit setting, int() = 2).
@pytest.mark.parametrize("B,Hq,Hkv,L,hot,bits", [
    (1, 32, 8, 1000, 64, 1), (4, 32, 8, 4096 + 64, 64, 2), (2, 16, 2, 333, 16, 2), (1, 32, 8, 2100, 64, 4),
    (1, 32, 8, 1000, 128, 3), (2, 8, 4, 150, 200, 3), (1, 32, 8, 3000, 256, 2), (1, 32, 8, 130, 256, 1),
    (3, 32, 8, 700, 100, 3)])
def test_decode_attn_bits_and_hot(cuda, B, Hq, Hkv, L, hot, bits):
    print("decode attn case B=%d Hq=%d Hkv=%d L=%d hot=%d bits=%d" % (B, Hq, Hkv, L, hot, bits), flush=True)
    out, ref = _attn_case(B, Hq, Hkv, L, hot, seed=L + bits, dev=cuda, bits=bits)
    assert torch.isfinite(out).all()
    assert ot.rel_err(out.numpy(), ref.numpy()) < RTOL
    assert ot.max_rel_err(out.numpy(), ref.numpy()) < RTOL


def _prefill_case(B, Hq, Hkv, L, S, hot, seed, dev, bits=3):
    """A cache of L tokens (cold = L - hot, built with the oracle) and the newest S tokens' queries:
    the HIP prefill kernel vs causal fp64 attention over cat(dequantize(cold).fp16, hot)."""
    from leankv_amd import kernels

    c, b = oq.codebook_tensors(bits)
    PiK, PiV = oq.rotation_matrix(128, 42), oq.rotation_matrix(128, 43)
    cold = max(0, L - hot)
    K = _kv((B, Hkv, L, 128), seed)
    V = _kv((B, Hkv, L, 128), seed + 1000)
    q = torch.randn(B, Hq, S, 128, generator=torch.Generator().manual_seed(seed + 7)).half()
    cap = max(cold, 1)
    kc = torch.zeros(B, Hkv, cap, _ROW_BYTES[bits], dtype=torch.uint8)
    vc = torch.zeros_like(kc)
    kn = torch.zeros(B, Hkv, cap)
    vn = torch.zeros_like(kn)
    Kref, Vref = K.clone(), V.clone()
    if cold:
        pk, nk, _ = oq.quantize(K[:, :, :cold].float(), PiK, b, bits)
        pv, nv, _ = oq.quantize(V[:, :, :cold].float(), PiV, b, bits)
        kc[:, :, :cold] = torch.from_numpy(pk)
        vc[:, :, :cold] = torch.from_numpy(pv)
        kn[:, :, :cold] = nk
        vn[:, :, :cold] = nv
        Kref[:, :, :cold] = oq.dequantize(pk, nk, PiK, c, bits).half()
        Vref[:, :, :cold] = oq.dequantize(pv, nv, PiV, c, bits).half()
    kh = torch.full((B, Hkv, hot, 128), float("nan"), dtype=torch.float16)  # slots past the window stay NaN
    vh = torch.full_like(kh, float("nan"))
    for p in range(cold, L):
        kh[:, :, p % hot] = K[:, :, p]
        vh[:, :, p % hot] = V[:, :, p]
    out = kernels.tq_prefill_attn(q.to(dev), kc.to(dev), kn.to(dev), vc.to(dev), vn.to(dev), kh.to(dev), vh.to(dev),
                                  PiK.to(dev), PiV.to(dev), c.to(dev), bits, L).cpu()
    ref = oq.prefill_attention(q, Kref, Vref)
    return out, ref


# (B, Hq, Hkv, L, S, hot, bits): fresh prefills (S = L), chunks (S < L), all-hot and one-cold-token
# caches, a single query, 1 / 2 / 4 / 8 / 16 query heads per kv head, 4-bit codes, a 16-token window.
@pytest.mark.parametrize("B,Hq,Hkv,L,S,hot,bits", [
    (1, 8, 2, 100, 100, 64, 3), (1, 4, 4, 37, 37, 64, 3), (1, 32, 8, 200, 1, 64, 3), (2, 16, 2, 300, 77, 16, 3),
    (1, 16, 1, 130, 130, 64, 4), (1, 32, 8, 700, 700, 64, 3), (1, 2, 2, 64, 64, 64, 3), (1, 8, 4, 65, 65, 64, 3),
    (3, 8, 8, 257, 129, 64, 4), (1, 32, 4, 333, 333, 64, 3),
    (1, 32, 8, 500, 500, 64, 2), (2, 8, 2, 300, 40, 64, 1), (1, 16, 4, 700, 700, 128, 2)])
def test_prefill_attn(cuda, B, Hq, Hkv, L, S, hot, bits):
    print("prefill case B=%d Hq=%d Hkv=%d L=%d S=%d hot=%d bits=%d" % (B, Hq, Hkv, L, S, hot, bits), flush=True)
    out, ref = _prefill_case(B, Hq, Hkv, L, S, hot, seed=L + S, dev=cuda, bits=bits)
    assert torch.isfinite(out).all()
    assert ot.rel_err(out.numpy(), ref.numpy()) < RTOL
    assert ot.max_rel_err(out.numpy(), ref.numpy()) < RTOL


def test_prefill_attn_full_size(cuda):
    """Config-5 layer shape: a 4096-token prompt (4032 cold 3-bit tokens + 64 hot), 32 query / 8 kv heads.
    Reference: torch fp32 causal SDPA on the GPU over K/V dequantized by the fp64 oracle."""
    from leankv_amd import kernels

    B, Hq, Hkv, S, hot, D = 1, 32, 8, 4096, 64, 128
    cold = S - hot
    c, _ = oq.codebook_tensors(3)
    PiK, PiV = oq.rotation_matrix(D, 42), oq.rotation_matrix(D, 43)
    g = torch.Generator().manual_seed(11)
    # codes: 3-bit values in both nibbles; norms ~ those of unit-variance 128-vectors
    kc = (torch.randint(0, 8, (B, Hkv, cold, 64), generator=g) | (torch.randint(0, 8, (B, Hkv, cold, 64),
                                                                               generator=g) << 4)).to(torch.uint8)
    vc = (torch.randint(0, 8, (B, Hkv, cold, 64), generator=g) | (torch.randint(0, 8, (B, Hkv, cold, 64),
                                                                               generator=g) << 4)).to(torch.uint8)
    kn = torch.rand(B, Hkv, cold, generator=g) * 4 + 9
    vn = torch.rand(B, Hkv, cold, generator=g) * 4 + 9
    kh = torch.randn(B, Hkv, hot, D, generator=g).half()
    vh = torch.randn(B, Hkv, hot, D, generator=g).half()
    q = torch.randn(B, Hq, S, D, generator=g).half()
    out = kernels.tq_prefill_attn(q.to(cuda), kc.to(cuda), kn.to(cuda), vc.to(cuda), vn.to(cuda), kh.to(cuda),
                                  vh.to(cuda), PiK.to(cuda), PiV.to(cuda), c.to(cuda), 3, S).float()
    order = [p % hot for p in range(cold, S)]
    K = torch.cat([oq.dequantize(kc.numpy(), kn, PiK, c, 3).half(), kh[:, :, order]], dim=2)
    V = torch.cat([oq.dequantize(vc.numpy(), vn, PiV, c, 3).half(), vh[:, :, order]], dim=2)
    Kd = K.float().repeat_interleave(Hq // Hkv, dim=1).contiguous().to(cuda)
    Vd = V.float().repeat_interleave(Hq // Hkv, dim=1).contiguous().to(cuda)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float().to(cuda), Kd, Vd, is_causal=True)
    assert torch.isfinite(out).all()
    err = float((out - ref).norm() / ref.norm())
    assert err < RTOL, err
    assert float((out - ref).abs().max() / ref.abs().max()) < RTOL


def _paged_case(lens, Hq, Hkv, ps, seed, dev):
    """A shuffled page pool holding sequences of the given lengths; the HIP kernel vs fp64 attention over
    each sequence's gathered K/V."""
    from leankv_amd import kernels

    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    npages = [-(-n // ps) for n in lens]
    max_pages = sum(npages) + 3
    perm = torch.randperm(max_pages, generator=g).tolist()
    pool = torch.randn(max_pages, 2, ps, Hkv, 128, generator=g).half()
    indptr, indices, last = [0], [], []
    for b in range(B):
        mine = perm[indptr[-1]:indptr[-1] + npages[b]]
        indices += mine
        indptr.append(indptr[-1] + npages[b])
        r = lens[b] % ps
        last.append(r if r else ps)
    q = torch.randn(B, Hq, 128, generator=g).half()
    out = kernels.paged_decode_attn(q.to(dev), pool.to(dev), torch.tensor(indptr, dtype=torch.int32, device=dev),
                                    torch.tensor(indices or [0], dtype=torch.int32, device=dev),
                                    torch.tensor(last, dtype=torch.int32, device=dev), max(lens)).cpu()
    refs = []
    for b in range(B):
        pg = torch.tensor(indices[indptr[b]:indptr[b + 1]], dtype=torch.long)
        k = pool[pg, 0].reshape(-1, Hkv, 128)[: lens[b]].permute(1, 0, 2).unsqueeze(0)
        v = pool[pg, 1].reshape(-1, Hkv, 128)[: lens[b]].permute(1, 0, 2).unsqueeze(0)
        refs.append(oq.decode_attention(q[b:b + 1].unsqueeze(2), k, v).squeeze(2))
    return out, torch.cat(refs)


# (sequence lengths, Hq, Hkv, page size): one token, page boundaries, ragged batches, 4096-token contexts,
# 1-token pages, 64-token pages, 1 / 4 / 16 query heads per kv head.
@pytest.mark.parametrize("lens,Hq,Hkv,ps", [([1], 32, 8, 16), ([16, 17, 33], 32, 8, 16), ([4096], 32, 8, 16),
                                            ([300, 1, 4096, 77, 129], 8, 2, 16), ([50, 51], 4, 4, 1),
                                            ([1000, 999], 16, 1, 64), ([2049] * 16, 32, 8, 16)])
def test_paged_decode_attn(cuda, lens, Hq, Hkv, ps):
    """The fp16 page-pool attention of the dense fp16 baseline (OwnDenseEngine) vs fp64 attention."""
    out, ref = _paged_case(lens, Hq, Hkv, ps, seed=sum(lens) + ps, dev=cuda)
    assert torch.isfinite(out).all()
    assert ot.rel_err(out.numpy(), ref.numpy()) < RTOL
    assert ot.max_rel_err(out.numpy(), ref.numpy()) < RTOL


def _paged_tq_case(lens, Hq, Hkv, hot, ps, bits, seed, dev):
    """Sequences of the given lengths in a paged packed cache built with the oracle (cold codes in pages
    scattered over a pool whose other rows hold random codes and norms, fp16 hot rings); the HIP kernel
    vs fp64 attention over each sequence's cat(dequantize(cold).fp16, hot)."""
    from leankv_amd import kernels

    c, bnd = oq.codebook_tensors(bits)
    PiK, PiV = oq.rotation_matrix(128, 42), oq.rotation_matrix(128, 43)
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    colds = [max(0, n - hot) for n in lens]
    npages = [-(-cl // ps) for cl in colds]
    max_pages = sum(npages) + 3
    perm = torch.randperm(max_pages, generator=g).tolist()
    mask = 0x77 if bits == 3 else 0xFF
    rb = _ROW_BYTES[bits]
    kc = torch.randint(0, 256, (max_pages, Hkv, ps, rb), generator=g, dtype=torch.uint8) & mask
    vc = torch.randint(0, 256, (max_pages, Hkv, ps, rb), generator=g, dtype=torch.uint8) & mask
    kn = torch.rand(max_pages, Hkv, ps, generator=g) * 50 + 50  # rows no sequence owns: large, visible if read
    vn = torch.rand(max_pages, Hkv, ps, generator=g) * 50 + 50
    kh = torch.randn(B, Hkv, hot, 128, generator=g).half()
    vh = torch.randn(B, Hkv, hot, 128, generator=g).half()
    q = torch.randn(B, Hq, 128, generator=g).half()
    indptr, indices, refs = [0], [], []
    for b, n in enumerate(lens):
        mine = perm[indptr[-1]:indptr[-1] + npages[b]]
        indices += mine
        indptr.append(indptr[-1] + npages[b])
        K = _kv((Hkv, n, 128), seed + 17 * b)
        V = _kv((Hkv, n, 128), seed + 17 * b + 5)
        cl = colds[b]
        Kref, Vref = K.clone(), V.clone()
        if cl:
            pk, nk, _ = oq.quantize(K[:, :cl].float(), PiK, bnd, bits)
            pv, nv, _ = oq.quantize(V[:, :cl].float(), PiV, bnd, bits)
            pg = torch.tensor([mine[t // ps] for t in range(cl)])
            sl = torch.tensor([t % ps for t in range(cl)])
            kc[pg, :, sl] = torch.from_numpy(pk).transpose(0, 1)
            vc[pg, :, sl] = torch.from_numpy(pv).transpose(0, 1)
            kn[pg, :, sl] = nk.t()
            vn[pg, :, sl] = nv.t()
            Kref[:, :cl] = oq.dequantize(pk, nk, PiK, c, bits).half()
            Vref[:, :cl] = oq.dequantize(pv, nv, PiV, c, bits).half()
        for p in range(cl, n):
            kh[b, :, p % hot] = K[:, p]
            vh[b, :, p % hot] = V[:, p]
        refs.append(oq.decode_attention(q[b:b + 1].unsqueeze(2), Kref.unsqueeze(0), Vref.unsqueeze(0)).squeeze(2))
    print("paged packed case lens=%s Hq=%d Hkv=%d hot=%d ps=%d bits=%d" % (lens, Hq, Hkv, hot, ps, bits), flush=True)
    i32 = dict(dtype=torch.int32, device=dev)
    out = kernels.tq_paged_decode_attn(q.to(dev), kc.to(dev), kn.to(dev), vc.to(dev), vn.to(dev), kh.to(dev),
                                       vh.to(dev), PiK.to(dev), PiV.to(dev), c.to(dev), bits,
                                       torch.tensor(indptr, **i32), torch.tensor(indices or [0], **i32),
                                       torch.tensor(lens, **i32), max(lens)).cpu()
    return out, torch.cat(refs)


# (lengths, Hq, Hkv, hot window, page size, bits): config 4 through pages; ragged batches with hot-only,
# window-boundary and page-boundary sequences; 32 / 64 / 128-token pages; 4-bit codes; 1 / 8 query heads
# per kv head; a 9000-token sequence in a 32-sequence batch, so that a split's pages hit the LDS table
# cap and the split count grows past the target.
@pytest.mark.parametrize("lens,Hq,Hkv,hot,ps,bits", [
    ([4096 + 64] * 16, 32, 8, 64, 16, 3),
    ([1, 64, 65, 1000, 4160, 333, 17, 129], 32, 8, 64, 16, 3),
    ([80, 81, 2000], 32, 4, 16, 32, 3),
    ([700, 1, 3000], 8, 8, 64, 64, 4),
    ([5000, 129, 4097], 64, 8, 64, 128, 3),
    ([9000] + [100] * 31, 8, 8, 64, 16, 3),
    ([300, 4160, 65], 32, 8, 64, 16, 2),
    ([129, 1000], 16, 4, 128, 32, 1),
    ([2000, 5, 256], 32, 8, 256, 16, 3),
])
def test_tq_paged_decode_attn(cuda, lens, Hq, Hkv, hot, ps, bits):
    out, ref = _paged_tq_case(lens, Hq, Hkv, hot, ps, bits, seed=sum(lens) % 1000 + ps, dev=cuda)
    assert torch.isfinite(out).all()
    assert ot.rel_err(out.numpy(), ref.numpy()) < RTOL
    assert ot.max_rel_err(out.numpy(), ref.numpy()) < RTOL


def test_paged_tq_cache_matches_dense_cache(cuda):
    """PagedTurboQuantCache vs TurboQuantCache on the same appends (a 300-token prefill, then 70 decode
    tokens, 2 layers, 3 sequences): every sequence's cold codes and norms equal the dense cache's bit for
    bit, and decode attention on the pages agrees with the dense kernel and with fp64 attention."""
    from leankv_amd.turboquant.cache import TurboQuantCache
    from leankv_amd.turboquant.paged_tq_cache import PagedTurboQuantCache

    g = torch.Generator().manual_seed(21)
    paged = PagedTurboQuantCache(num_layers=2, num_kv_heads=2, num_q_heads=8, page_size=16, max_pages=128,
                                 max_batch_size=4, device=cuda)
    dense = TurboQuantCache(num_layers=2, device=cuda, fused_attention=False, max_seq_len=512)
    for S in [300] + [1] * 70:
        for li in range(2):
            k = (torch.randn(3, 2, S, 128, generator=g) * 2).half().to(cuda)
            v = torch.randn(3, 2, S, 128, generator=g).half().to(cuda)
            kp, vp = paged.update(k, v, li)
            kd, vd = dense.update(k, v, li)
            if S > 1:
                assert torch.equal(kp, kd) and torch.equal(vp, vd)
    q = torch.randn(3, 8, 128, generator=g).half().to(cuda)
    for li in range(2):
        n = dense._seq_lengths[li]
        cl = n - 64
        for b in range(3):
            k_c, k_n, v_c, v_n = paged.cold_arrays(li, b)
            assert torch.equal(k_c, dense._k_codes[li][b, :, :cl]) and torch.equal(v_c, dense._v_codes[li][b, :, :cl])
            assert torch.equal(k_n, dense._k_norms[li][b, :, :cl]) and torch.equal(v_n, dense._v_norms[li][b, :, :cl])
        out = paged.decode_attention(li, q).cpu()
        seq = torch.tensor([n], dtype=torch.int32, device=cuda)
        from leankv_amd import kernels

        out_d = kernels.tq_decode_attn(q, dense._k_codes[li], dense._k_norms[li], dense._v_codes[li],
                                       dense._v_norms[li], dense._k_hot[li], dense._v_hot[li], dense.PiK[li],
                                       dense.PiV[li], dense.centroids, 3, seq, n).cpu()
        assert ot.rel_err(out.numpy(), out_d.numpy()) < 2e-3
        k, v = paged.gather(li, 3)
        ref = oq.decode_attention(q.cpu().unsqueeze(2), k.cpu(), v.cpu()).squeeze(2)
        assert ot.rel_err(out.numpy(), ref.numpy()) < RTOL


def test_paged_tq_cache_ragged_free_and_reuse(cuda):
    """Sequences appended one by one to different lengths, one freed and its pages reused by a new
    sequence: decode attention of each equals fp64 attention over its own gathered K/V."""
    from leankv_amd.turboquant.paged_tq_cache import PagedTurboQuantCache

    g = torch.Generator().manual_seed(8)
    c = PagedTurboQuantCache(num_layers=1, num_kv_heads=4, num_q_heads=16, page_size=32, max_pages=40,
                             max_batch_size=3, hot_buffer_size=32, device=cuda)

    def add(b, S):
        c.append(0, b, torch.randn(4, S, 128, generator=g).half().to(cuda),
                 torch.randn(4, S, 128, generator=g).half().to(cuda))

    for b, S in ((0, 500), (1, 20), (2, 33)):
        add(b, S)
    used = c.get_pages_used()
    assert used == -(-(500 - 32) // 32) + 0 + 1
    c.free_sequence(0)
    assert c.get_pages_used() == used - 15
    add(0, 700)  # reuses the freed pages
    for _ in range(5):
        for b in range(3):
            add(b, 1)
    q = torch.randn(3, 16, 128, generator=g).half().to(cuda)
    out = c.decode_attention(0, q).cpu()
    k, v = c.gather(0, 3)
    for b, n in enumerate((705, 25, 38)):
        ref = oq.decode_attention(q[b:b + 1].cpu().unsqueeze(2), k[b:b + 1, :, :n].cpu(),
                                  v[b:b + 1, :, :n].cpu()).squeeze(2)
        assert ot.rel_err(out[b:b + 1].numpy(), ref.numpy()) < RTOL
    with pytest.raises(RuntimeError, match="out of pages"):
        add(1, 40 * 32)


# Large batches (many (batch, kv head) pairs, few splits each): hot-only,
# boundary and short cold ranges, a 16-token window, 16 query heads per kv head.
@pytest.mark.parametrize("B,Hq,Hkv,L,hot", [(16, 32, 8, 1, 64), (16, 32, 8, 65, 64), (16, 32, 8, 700, 64),
                                            (32, 16, 4, 333, 16), (16, 128, 8, 300, 64), (64, 8, 2, 200, 64)])
def test_decode_attn_large_batch(cuda, B, Hq, Hkv, L, hot):
    out, ref = _attn_case(B, Hq, Hkv, L, hot, seed=L + B, dev=cuda)
    assert ot.rel_err(out.numpy(), ref.numpy()) < RTOL
    assert ot.max_rel_err(out.numpy(), ref.numpy()) < RTOL

"""CPU tests: pin the oracle (and the host-side codebook / rotation) before trusting it.

Each check is chosen so that a plausible mistake in the restatement -- a wrong
shift, a transposed rotation, '>=' for '>', a dropped norm -- fails one of them.
"""

import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import teal as ot
from oracle import turboquant as oq

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ------------------------------------------------------------------ codebook
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_codebook_golden_self_consistent(bits):
    cb = oq.load_codebook(bits)
    c = np.array(cb["centroids"])
    b = np.array(cb["boundaries"])
    assert len(c) == 2 ** bits and len(b) == 2 ** bits + 1
    assert b[0] == -1.0 and b[-1] == 1.0
    assert np.all(np.diff(c) > 0)
    # boundaries are midpoints of adjacent centroids (codebook.py:104-108)
    assert np.array_equal(b[1:-1], (c[:-1] + c[1:]) / 2.0)
    # float32 hex in the fixture is the rounding of the float64 list
    hexes = ["%08x" % v for v in np.asarray(c, np.float32).view(np.uint32)]
    assert hexes == cb["centroids_f32_hex"]
    # symmetric density -> symmetric codebook
    np.testing.assert_allclose(c, -c[::-1], atol=1e-9)


@pytest.mark.parametrize("bits", [1, 2, 3])
def test_codebook_lloyd_conditions(bits):
    """Each centroid is the conditional mean of its cell (converged to ~1e-6)."""
    from scipy import integrate, special

    cb = oq.load_codebook(bits)
    c, b = np.array(cb["centroids"]), np.array(cb["boundaries"])
    d = 128
    lc = special.gammaln(d / 2) - 0.5 * math.log(math.pi) - special.gammaln((d - 1) / 2)
    f = lambda x: math.exp(lc + (d - 3) / 2 * math.log(max(1 - x * x, 1e-300)))
    tot = integrate.quad(f, -1, 1)[0]
    assert abs(tot - 1) < 1e-8
    mse = 0.0
    for i in range(len(c)):
        num = integrate.quad(lambda x: x * f(x), b[i], b[i + 1])[0]
        den = integrate.quad(f, b[i], b[i + 1])[0]
        assert abs(num / den - c[i]) < 1e-5
        mse += integrate.quad(lambda x: (x - c[i]) ** 2 * f(x), b[i], b[i + 1])[0]
    assert abs(mse - cb["mse_per_coord"]) < 1e-9 * max(1.0, mse) + 1e-12


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_shipped_codebook_equals_reference_solver(bits):
    """The package's own solver output (shipped JSON) equals the reference's run."""
    g = oq.load_codebook(bits)
    here = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    with open(os.path.join(here, "leankv_amd", "turboquant", "codebooks", "codebook_d128_b%d.json" % bits)) as f:
        s = json.load(f)
    assert s["centroids"] == g["centroids"]
    assert s["boundaries"] == g["boundaries"]


def test_codebook_solver_reproduces_reference_b2():
    """Re-run the package solver (not the shipped file) for bits=2 and compare bits."""
    from leankv_amd.turboquant.codebook import compute_lloyd_max_codebook

    cb = compute_lloyd_max_codebook(128, 2)
    g = oq.load_codebook(2)
    assert cb["centroids"] == g["centroids"]
    assert cb["boundaries"] == g["boundaries"]


# ------------------------------------------------------------------ rotation
@pytest.mark.parametrize("seed", [42, 43, 105])
def test_rotation_is_the_unique_qr_factor(seed):
    Q = oq.rotation_matrix(128, seed).double()
    g = torch.Generator().manual_seed(seed)
    G = torch.randn(128, 128, generator=g, dtype=torch.float32).double()
    I = torch.eye(128, dtype=torch.float64)
    assert torch.allclose(Q.T @ Q, I, atol=1e-5)
    R = Q.T @ G  # must be upper triangular with positive diagonal
    assert torch.allclose(torch.tril(R, -1), torch.zeros_like(R), atol=1e-4)
    assert bool((torch.diag(R) > 0).all())


def test_product_rotation_matches_oracle():
    from leankv_amd.turboquant.rotation import generate_rotation_matrix

    for seed in (42, 43, 44):
        assert torch.equal(generate_rotation_matrix(128, "cpu", torch.float32, seed), oq.rotation_matrix(128, seed))


def test_rotation_memo_hands_out_copies():
    """Each (d, seed) is factorised once per process: later calls, and the caches' one-copy list, must
    still equal the oracle after a caller has written into an earlier result."""
    from leankv_amd.turboquant.cache import TurboQuantCache
    from leankv_amd.turboquant.rotation import generate_rotation_matrices, generate_rotation_matrix

    first = generate_rotation_matrix(128, "cpu", torch.float32, 42)
    first.zero_()
    assert torch.equal(generate_rotation_matrix(128, "cpu", torch.float32, 42), oq.rotation_matrix(128, 42))
    many = generate_rotation_matrices(128, [44, 42, 43], "cpu")
    for m, seed in zip(many, (44, 42, 43)):
        assert m.is_contiguous() and torch.equal(m, oq.rotation_matrix(128, seed))
    c = TurboQuantCache(bits=3, num_layers=3, device="cpu", seed=7)
    for i in range(3):
        assert torch.equal(c.PiK[i], oq.rotation_matrix(128, 7 + 2 * i))
        assert torch.equal(c.PiV[i], oq.rotation_matrix(128, 8 + 2 * i))


# --------------------------------------------------------------- pack/unpack
def _brute_pack(idx, bits):
    width = 1 if bits == 1 else (2 if bits == 2 else 4)
    per = 8 // width
    out = []
    for row in idx.reshape(-1, idx.shape[-1]):
        row = list(row) + [0] * ((-len(row)) % per)
        bs = []
        for j in range(0, len(row), per):
            v = 0
            for e in range(per):
                v |= int(row[j + e]) << (width * e)
            bs.append(v)
        out.append(bs)
    return np.array(out, dtype=np.uint8).reshape(idx.shape[:-1] + (-1,))


@pytest.mark.parametrize("bits,d", [(1, 128), (2, 128), (3, 128), (4, 128), (3, 7), (2, 5), (1, 9)])
def test_pack_matches_brute_force_and_round_trips(bits, d):
    rng = np.random.default_rng(bits * 100 + d)
    idx = rng.integers(0, 2 ** bits, size=(3, 5, d))
    p = oq.pack_indices(idx, bits)
    assert np.array_equal(p, _brute_pack(idx, bits))
    assert np.array_equal(oq.unpack_indices(p, bits, d), idx)


def test_pack_nibble_layout_3bit():
    """byte j = c[2j] | c[2j+1] << 4 (quantizer.py:46-61)."""
    idx = np.array([[1, 2, 7, 0, 5, 6]])
    assert list(oq.pack_indices(idx, 3)[0]) == [0x21, 0x07, 0x65]


def test_product_pack_helpers_match_oracle():
    from leankv_amd.turboquant.quantizer import _pack_indices, _unpack_indices

    rng = np.random.default_rng(0)
    for bits in (1, 2, 3, 4):
        idx = rng.integers(0, 2 ** bits, size=(4, 128))
        p = _pack_indices(torch.from_numpy(idx), bits).numpy()
        assert np.array_equal(p, oq.pack_indices(idx, bits))
        assert np.array_equal(_unpack_indices(torch.from_numpy(p), bits, 128).numpy(), idx)


# ------------------------------------------------------------------ TurboQuantProd / QJL
def _qjl_cases():
    return json.load(open(os.path.join(GOLDEN, "qjl_prod_cases.json")))


def test_qjl_oracle_matches_reference_golden():
    """The reference's TurboQuantProd on seeded inputs (make_qjl_golden.py), bit for bit."""
    import hashlib

    S = oq.qjl_matrix(128, 42 + 1000)
    Pi = oq.rotation_matrix(128, 42)
    for c in _qjl_cases():
        assert hashlib.sha256(S.numpy().tobytes()).hexdigest() == c["S_sha256"]
        assert S[0].tolist() == c["S_row0"]
        assert c["qjl_scale"] == math.sqrt(math.pi / 2) / 128
        mb = c["mse_bits"]
        assert mb == c["bits"] - 1
        cen, b = oq.codebook_tensors(mb)
        x = torch.tensor(c["x"]).to(getattr(torch, c["dtype"]))
        codes, norms, signs, rn, _ = oq.prod_quantize(x, Pi, b, cen, S, mb)
        assert np.array_equal(codes, np.array(c["mse_indices"], np.uint8))
        assert np.array_equal(signs, np.array(c["qjl_signs"], np.uint8))
        assert torch.equal(rn, torch.tensor(c["residual_norms"]))
        assert torch.equal(norms.float(), torch.tensor(c["norms"]))
        out = oq.prod_dequantize(codes, norms, signs, rn, Pi, cen, S, mb)
        assert torch.equal(out, torch.tensor(c["dequantized"]))


def _brute_signs(proj):
    out = []
    for row in np.asarray(proj).reshape(-1, proj.shape[-1]):
        bs = []
        for j in range(0, len(row), 8):
            v = 0
            for i in range(8):
                if j + i < len(row) and row[j + i] > 0:
                    v |= 1 << i
            bs.append(v)
        out.append(bs)
    return np.array(out, dtype=np.uint8).reshape(proj.shape[:-1] + (-1,))


@pytest.mark.parametrize("d", [128, 13, 8])
def test_qjl_sign_packing_brute_force(d):
    rng = np.random.default_rng(d)
    proj = rng.standard_normal((3, 4, d)).astype(np.float32)
    proj[0, 0, :3] = 0.0  # exactly zero packs as a 0 bit ('> 0')
    p = oq.pack_signs(proj)
    assert np.array_equal(p, _brute_signs(proj))
    s = oq.unpack_signs(p, d)
    assert np.array_equal(s, np.where(proj > 0, 1.0, -1.0).astype(np.float32))


def test_qjl_estimator_is_unbiased():
    """E_S[(sign(S r) @ S) * sqrt(pi/2)/d * ||r||] = r: pins the scale constant and the sign convention."""
    g = torch.Generator().manual_seed(5)
    d, draws = 128, 2000
    r = torch.randn(3, d, generator=g)
    acc = torch.zeros(3, d, dtype=torch.float64)
    for k in range(0, draws, 250):
        S = torch.randn(250, d, d, generator=g)
        proj = torch.einsum("kij,bj->kbi", S, r)
        s = torch.from_numpy(oq.unpack_signs(oq.pack_signs(proj.numpy()), d))
        est = torch.einsum("kbi,kij->kbj", s, S) * (math.sqrt(math.pi / 2) / d * r.norm(dim=-1)).unsqueeze(-1)
        acc += est.double().sum(0)
    mean = acc / draws
    rel = (mean - r.double()).norm(dim=-1) / r.double().norm(dim=-1)
    assert (rel < 0.06).all(), rel  # expected ~0.025 at 2000 draws; sqrt(2/pi) or a flipped sign gives >= 0.36


def test_prod_host_helpers_and_constructor():
    from leankv_amd.turboquant.quantizer import TurboQuantProd

    tq = TurboQuantProd(128, bits=3, device="cpu", seed=7)
    assert tq.mse_quantizer.bits == 2 and torch.equal(tq.S, oq.qjl_matrix(128, 1007))
    assert torch.equal(tq.mse_quantizer.Pi, oq.rotation_matrix(128, 7))
    assert tq.qjl_scale == math.sqrt(math.pi / 2) / 128
    proj = torch.randn(5, 128)
    proj[0, :4] = 0
    p = tq._pack_qjl_signs(proj)
    assert np.array_equal(p.numpy(), oq.pack_signs(proj.numpy()))
    assert np.array_equal(tq._unpack_qjl_signs(p).numpy(), oq.unpack_signs(p.numpy()))
    with pytest.raises(AssertionError, match="at least 2 bits"):
        TurboQuantProd(128, bits=1, device="cpu")


# ------------------------------------------------------------------ quantize
def test_quantize_codes_are_boundary_counts():
    """searchsorted(right=False) == number of decision boundaries strictly below y."""
    torch.manual_seed(0)
    c, b = oq.codebook_tensors(3)
    Pi = oq.rotation_matrix(128, 42)
    x = torch.randn(64, 128)
    x[:, [0, 31, 64, 127]] *= 10
    packed, norms, y = oq.quantize(x, Pi, b, 3)
    inner = b[1:-1].numpy()
    brute = (y.numpy()[..., None] > inner).sum(-1)
    assert np.array_equal(oq.unpack_indices(packed, 3, 128), brute)
    # ties go to the lower code: y exactly on a boundary
    yb = torch.tensor([[float(inner[2])] * 128])
    assert int(torch.searchsorted(b[1:-1].contiguous(), yb)[0, 0]) == 2
    np.testing.assert_allclose(norms.numpy(), np.linalg.norm(x.double().numpy(), axis=-1), rtol=1e-6)


def test_quantize_rotation_direction():
    """y = u @ Pi^T, not u @ Pi: a basis vector maps to a ROW of Pi."""
    Pi = oq.rotation_matrix(128, 42)
    e = torch.zeros(1, 128)
    e[0, 5] = 3.0
    _, n, y = oq.quantize(e, Pi, oq.codebook_tensors(3)[1], 3)
    assert torch.allclose(y[0], Pi[:, 5], atol=1e-7)
    assert abs(n.item() - 3.0) < 1e-7


def test_dequantize_inverts_rotation():
    c, b = oq.codebook_tensors(4)
    Pi = oq.rotation_matrix(128, 7)
    torch.manual_seed(1)
    x = torch.randn(32, 128)
    p, n, _ = oq.quantize(x, Pi, b, 4)
    xh = oq.dequantize(p, n, Pi, c, 4)
    rel = ((xh - x).norm(dim=-1) / x.norm(dim=-1)).mean().item()
    # 4-bit Lloyd-Max MSE per coordinate * d = relative squared error
    assert rel ** 2 < 3 * oq.load_codebook(4)["mse_total"]


def test_cache_ref_hot_cold_split():
    c, b = oq.codebook_tensors(3)
    PiK, PiV = oq.rotation_matrix(128, 42), oq.rotation_matrix(128, 43)
    ref = oq.CacheRef(PiK, PiV, c, b, 3, hot=64)
    torch.manual_seed(2)
    k = torch.randn(1, 2, 100, 128, dtype=torch.float16)
    K, V = ref.update(k, k)
    assert K.shape == (1, 2, 100, 128)
    assert ref.hot_k.shape[2] == 64
    assert torch.equal(K[:, :, 36:], k[:, :, 36:])  # hot tokens are exact fp16
    K2, _ = ref.update(k[:, :, :1], k[:, :, :1])
    assert K2.shape[2] == 101 and ref.hot_k.shape[2] == 64


# ------------------------------------------------------------------ TEAL
def test_keep_mask_strict_and_fp32_threshold():
    x = np.array([0.5, -0.5, 0.25, 0.0], dtype=np.float16)
    assert list(ot.keep_mask(x, 0.25)) == [True, True, False, False]
    # The Triton kernel compares in fp32 (sparse_gemv.py:82): fp16(0.04) =
    # 0.040008544921875 lies above fp32(0.04) and is kept, although a compare
    # in fp16 (t rounded to the same value) would drop it.
    t = 0.04
    x16 = np.float16(t)
    assert float(x16) > float(np.float32(t))
    assert ot.keep_mask(np.array([x16]), t)[0]
    below = np.nextafter(x16, np.float16(0))
    assert not ot.keep_mask(np.array([below]), t)[0]


def test_sparse_gemv_closed_forms():
    rng = np.random.default_rng(0)
    W = (rng.standard_normal((24, 40)) * 0.02).astype(np.float16)
    x = rng.laplace(0, 0.05, 40).astype(np.float16)
    dense = W.astype(np.float64) @ x.astype(np.float64)
    assert np.allclose(ot.sparse_gemv(x, W, -1.0), dense)
    assert np.all(ot.sparse_gemv(x, W, 10.0) == 0)
    t = float(np.sort(np.abs(x.astype(np.float32)))[15])
    m = np.abs(x.astype(np.float32)) > t
    brute = np.zeros(24)
    for z in range(40):
        if m[z]:
            brute += W[:, z].astype(np.float64) * float(x[z])
    assert np.allclose(ot.sparse_gemv(x, W, t), brute, rtol=0, atol=1e-12)
    assert m.sum() == 40 - 16  # distinct magnitudes: exactly 16 dropped


def test_threshold_for_sparsity_drops_exactly_k():
    torch.manual_seed(0)
    x = torch.randn(14336, dtype=torch.float64)
    t = ot.threshold_for_sparsity(x, 0.4)
    k = int(0.4 * x.numel())
    assert int((x.abs() <= t).sum()) == k
    from leankv_amd.teal.sparse_fns import compute_threshold_for_sparsity

    assert compute_threshold_for_sparsity(x, 0.4) == t
    assert compute_threshold_for_sparsity(x, 0.0) == 0.0
    assert compute_threshold_for_sparsity(x, 1.0) == x.abs().max().item()


def test_swiglu_chain_rounding():
    g = np.array([0.0, 1.0, -3.0], dtype=np.float16)
    s = ot.silu_f16(g)
    assert s[0] == 0 and abs(float(s[1]) - 0.7310586) < 1e-3
    rng = np.random.default_rng(3)
    Wg = (rng.standard_normal((16, 32)) * 0.1).astype(np.float16)
    Wu = (rng.standard_normal((16, 32)) * 0.1).astype(np.float16)
    x = rng.standard_normal(32).astype(np.float16)
    h = ot.gateup_swiglu(x, Wg, Wu, -1.0, -1.0)
    g64 = Wg.astype(np.float64) @ x.astype(np.float64)
    u64 = Wu.astype(np.float64) @ x.astype(np.float64)
    ref = g64 / (1 + np.exp(-g64)) * u64
    assert np.allclose(h.astype(np.float64), ref, rtol=5e-3, atol=1e-3)


def test_attention_oracle_closed_form():
    """One kv head, all keys equal -> uniform softmax -> mean of values."""
    q = torch.randn(1, 4, 1, 128)
    K = torch.ones(1, 1, 10, 128)
    V = torch.arange(10, dtype=torch.float32).view(1, 1, 10, 1).expand(1, 1, 10, 128)
    o = oq.decode_attention(q, K, V)
    assert torch.allclose(o, torch.full_like(o, 4.5, dtype=torch.float64))


def test_prefill_oracle_pins():
    """Causal prefill oracle: S = 1 is the decode oracle; S = L is torch's fp64 causal SDPA (top-left
    alignment is exact there); a chunk (S < L) matches a brute-force loop over the visible keys."""
    g = torch.Generator().manual_seed(5)
    q = torch.randn(2, 4, 6, 16, generator=g)
    K = torch.randn(2, 2, 9, 16, generator=g)
    V = torch.randn(2, 2, 9, 16, generator=g)
    assert torch.allclose(oq.prefill_attention(q[:, :, -1:], K, V), oq.decode_attention(q[:, :, -1:], K, V),
                          rtol=0, atol=1e-14)
    Ks, Vs = K[:, :, :6], V[:, :, :6]
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.double(), Ks.double().repeat_interleave(2, dim=1), Vs.double().repeat_interleave(2, dim=1), is_causal=True)
    assert torch.allclose(oq.prefill_attention(q, Ks, Vs), ref, rtol=0, atol=1e-12)
    out = oq.prefill_attention(q[:, :, :4], K, V)  # 4 queries at positions 5..8
    for b in range(2):
        for h in range(4):
            for i in range(4):
                pos = 9 - 4 + i
                k, v = K[b, h // 2, : pos + 1].double(), V[b, h // 2, : pos + 1].double()
                w = [math.exp(float(q[b, h, i].double() @ k[t]) / 4.0) for t in range(pos + 1)]
                o = sum(wt * v[t] for t, wt in enumerate(w)) / sum(w)
                assert torch.allclose(out[b, h, i], o, rtol=0, atol=1e-12)


def test_reference_model_matches_hf_mistral_without_compression():
    """The oracle decoder (no TEAL, hot window larger than the sequence) equals HF Mistral in fp32."""
    from transformers import MistralConfig, MistralForCausalLM

    from oracle.model import RefModel

    cfg = MistralConfig(vocab_size=300, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                        num_attention_heads=2, num_key_value_heads=1, head_dim=128, max_position_embeddings=512,
                        rope_theta=1e6, rms_norm_eps=1e-5)
    torch.manual_seed(0)
    m = MistralForCausalLM(cfg).float().eval()
    with torch.no_grad():
        for p in m.parameters():
            if p.dim() == 2:
                p.normal_(0, 0.05)
    ref = RefModel(m.state_dict(), cfg, None, hot=10_000)
    ids = torch.randint(0, 300, (20,))
    with torch.no_grad():
        hf_pref = m(ids.view(1, -1)).logits[0, -1]
    lg = ref.forward(ids)
    assert torch.allclose(lg, hf_pref, rtol=2e-2, atol=2e-2 * hf_pref.abs().max().item())
    # one decode step after the prompt
    nxt = torch.tensor([7])
    with torch.no_grad():
        hf_dec = m(torch.cat([ids, nxt]).view(1, -1)).logits[0, -1]
    lg2 = ref.forward(nxt)
    assert (lg2 - hf_dec).norm() / hf_dec.norm() < 2e-2

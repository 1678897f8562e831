"""Parity of the fused decode engine at the timed shape (config 5: Mistral-7B-v0.3, hidden 4096, ffn 14336,
32/8 heads, vocab 32768, head_dim 128) with a 1024-token prompt, and for the TEAL-on layer step also the
bench's own 4096-token context, so every kernel instantiation the bench times (the decode-mode attention
split with its 16-split plan at 4096 tokens among them) runs here at its own size:

  * TEAL off, 2 layers: the engine's teacher-forced logits vs oracle.model.RefModel (fp64 projections,
    the reference's TurboQuant cache semantics: cache.py:84-189), within 2e-2 relative per step.
  * TEAL on, 2 layers: one decode layer step of the engine, every fused launch checked against the
    oracle on the very input it consumed (read back from the step's workspace through
    lkv_decode_workspace_layout): the 3-segment q|k|v GEMV with its three thresholds
    (patching.py:169-177), RoPE and the ring write, the packed-KV attention (cache.py:169-189 +
    sdpa_attention.py:79-105), o_proj, the gate|up GEMV (two thresholds) and down with the SwiGLU
    prologue (modeling_mistral.py:46-47), and both residual adds (bit-exact).
  * TEAL on, all 32 layers: the engine vs the HF-patched path (apply_teal + TurboQuantCache + the
    leankv_tq attention, the reference's call path combined.py:57-126) fed the same tokens: logits and
    tokens identical, caches bit-identical.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import teal as ot
from oracle import turboquant as oq
from oracle.model import RefModel

pytestmark = pytest.mark.gpu

PROMPT, STEPS = 1024, 8
MAXLEN = PROMPT + STEPS + 8
SPARSITY = (0.3, 0.5)  # per-projection TEAL sparsity drawn from U[0.3, 0.5] (the config-5 decoder)
RTOL = 2e-2      # model logits vs the fp64 oracle (fp16 activations, fp32 sums)
GEMV_TOL = 1e-3  # one projection vs fp64 on the same input (fp32 accumulate, fp16 output)


def _model(cuda, layers, seed):
    from leankv_amd.engine import random_mistral

    return random_mistral(device=cuda, seed=seed, num_hidden_layers=layers)


def _thresholds(model, seed, context=PROMPT):
    """Thresholds at the decode's context: the quantiles of the last 256 positions of a calibration prompt as
    long as the decode's (bench.py calibrates the same way)."""
    from leankv_amd.teal.calibrate import calibrate_thresholds, uniform_random_sparsity

    g = torch.Generator().manual_seed(seed + 100)
    calib = [torch.randint(0, model.config.vocab_size, (1, context), generator=g)]
    with torch.no_grad():
        return calibrate_thresholds(model, calib, uniform_random_sparsity(*SPARSITY, seed),
                                    positions=slice(-256, None))


def _prompt(model, seed, n=PROMPT):
    g = torch.Generator().manual_seed(seed + 200)
    return torch.randint(0, model.config.vocab_size, (n,), generator=g)


def _patch(model, th, maxlen=MAXLEN, bits=3):
    from leankv_amd.teal.patching import apply_teal
    from leankv_amd.turboquant.attention import use_on
    from leankv_amd.turboquant.cache import TurboQuantCache

    if th is not None:
        apply_teal(model, thresholds=th, use_triton=True)
    cache = TurboQuantCache(bits=bits, head_dim=128, num_layers=model.config.num_hidden_layers,
                            device=model.device, max_seq_len=maxlen, fused_attention=True)
    use_on(model, cache)
    return cache


def _prefill(model, cache, prompt):
    with torch.no_grad():
        out = model(prompt.view(1, -1).to(model.device), past_key_values=cache, use_cache=True)
    return torch.argmax(out.logits[0, -1])


def test_config5_engine_matches_reference_teal_off(cuda):
    """2 full-width layers, TEAL off: engine logits vs the fp64 oracle decoder, teacher forced."""
    from leankv_amd.engine import LeanKVEngine

    model = _model(cuda, 2, seed=11)
    prompt = _prompt(model, 11)
    ref = RefModel({k: v.detach().float().cpu() for k, v in model.state_dict().items()}, model.config, None)
    cache = _patch(model, None)
    first = _prefill(model, cache, prompt)
    ref.forward(prompt)
    eng = LeanKVEngine(model, cache, MAXLEN)
    eng.start(first, PROMPT)
    errs = []
    with torch.no_grad():
        for i in range(STEPS):
            if i == 1:
                eng.capture()
            fed = int(eng.tok)
            eng.step()
            r = ref.forward(torch.tensor([fed]))
            errs.append(ot.rel_err(eng.logits.float().cpu().numpy(), r.numpy()))
    print("config-5 engine (TEAL off) vs oracle: rel err per step", ["%.2e" % e for e in errs])
    assert max(errs) < RTOL
    assert int(eng.pos64) == PROMPT + STEPS


def _sum_chunks(ws, off, n, nchunk):
    """fp16 outputs of a [slab][chunk][256] partial area: chunks summed in order from 0 (the kernels' order)."""
    slabs = (n + 255) // 256
    p = ws[off: off + slabs * nchunk * 256 * 4].view(torch.float32).view(slabs, nchunk, 256)
    s = torch.zeros(slabs, 256, dtype=torch.float32, device=ws.device)
    for c in range(nchunk):
        s = s + p[:, c]
    return s.reshape(-1)[:n].half()


def _np16(t):
    return t.detach().cpu().numpy().astype(np.float16)


def _w16(mod):
    return mod.weight.detach().cpu().numpy().astype(np.float16)


@pytest.mark.parametrize("context,bits", [(1024, 3), (4096, 3), (4096, 2), (1024, 1)])
def test_config5_engine_layer_step_matches_oracle_teal_on(cuda, context, bits):
    """2 full-width layers, TEAL on: every fused launch of one engine layer step vs the oracle on its input, at
    a 1024-token context and at the bench's 4096 (where the attention split runs its 16-split plan), 3-bit
    codes and the reference's 2- and 1-bit packings (configs/mistral7b.yaml sweeps bit widths), with
    thresholds calibrated at that context: every projection keeps a fraction of its inputs inside the band
    its configured sparsity sets."""
    from leankv_amd import _lib
    from leankv_amd.engine import LeanKVEngine
    from leankv_amd.kernels import rms_norm

    print("config-5 layer step case: context %d, %d-bit codes" % (context, bits), flush=True)
    PROMPT = context
    maxlen = PROMPT + STEPS + 8
    model = _model(cuda, 2, seed=12)
    th = _thresholds(model, 12, PROMPT)
    prompt = _prompt(model, 12, PROMPT)
    cache = _patch(model, th, maxlen, bits)
    first = _prefill(model, cache, prompt)
    eng = LeanKVEngine(model, cache, maxlen)
    eng.start(first, PROMPT)
    lib = _lib.load()
    st = _lib.stream_handle(cuda)
    ws, nb = eng.ws, eng.ws.numel()
    dims = ctypes.byref(eng.dims)
    lay = _lib.DecodeLayout()
    _lib.check(lib.lkv_decode_workspace_layout(dims, ctypes.byref(lay)), "layout")
    with torch.no_grad():
        _lib.check(lib.lkv_decode_begin(dims, model.model.embed_tokens.weight.data_ptr(), eng.tok.data_ptr(),
                                        eng.pos64.data_ptr(), eng.x.data_ptr(), ws.data_ptr(), nb, st), "begin")
        _lib.check(lib.lkv_decode_evict(dims, eng.layer_table, len(eng.layer_structs), ws.data_ptr(), nb, st), "evict")
        x0 = eng.x.clone()
        _lib.check(lib.lkv_decode_layer_step(dims, ctypes.byref(eng.layer_structs[0]), eng.x.data_ptr(),
                                             ws.data_ptr(), nb, st), "layer_step")
        x1 = eng.x.clone()
        torch.cuda.synchronize()
    layer = model.model.layers[0]
    at, mlp = layer.self_attn, layer.mlp
    t = th[0]
    nq, nkv, hidden, ffn = 4096, 1024, 4096, 14336
    report = {}

    def gemv_check(name, x16, y16, mod, thr):
        ref = ot.sparse_gemv(x16, _w16(mod), thr)
        err = ot.rel_err(_np16(y16).astype(np.float64), ref)
        kept = float(ot.keep_mask(x16, thr).mean())
        report[name] = (err, kept)
        assert err < GEMV_TOL, (name, err)
        # the configured band: sparsity in [0.3, 0.5] keeps 50-70 % of a projection's inputs over the
        # calibration positions; one decode token's inputs scatter around that by a few percent
        assert 1 - SPARSITY[1] - 0.06 < kept < 1 - SPARSITY[0] + 0.06, (name, kept)

    # 1. q|k|v: one launch, three thresholds, input = RMSNorm(x0) (lkv_rmsnorm = the prologue's arithmetic)
    h1 = rms_norm(x0.view(1, -1), layer.input_layernorm.weight, model.config.rms_norm_eps).view(-1)
    h1n = _np16(h1)
    q = _sum_chunks(ws, lay.part_q, nq, lay.chunks_qkv)
    k = _sum_chunks(ws, lay.part_k, nkv, lay.chunks_qkv)
    v = _sum_chunks(ws, lay.part_v, nkv, lay.chunks_qkv)
    gemv_check("q_proj", h1n, q, at.q_proj, t["q_proj"])
    gemv_check("k_proj", h1n, k, at.k_proj, t["k_proj"])
    gemv_check("v_proj", h1n, v, at.v_proj, t["v_proj"])
    # 2. RoPE at position PROMPT with HF's fp16 rounding (modeling_mistral.py apply_rotary_pos_emb), bit-exact;
    #    the new key / value land in ring slot PROMPT % 64
    cos, sin = eng.cos[PROMPT].float(), eng.sin[PROMPT].float()

    def rope(a):  # a fp16 [H, 128]
        a = a.float()
        rh = torch.cat([-a[:, 64:], a[:, :64]], dim=1)
        return ((a * cos).half().float() + (rh * sin).half().float()).half()

    q_rope = ws[lay.q_rope: lay.q_rope + nq * 2].view(torch.float16).view(32, 128)
    assert torch.equal(q_rope, rope(q.view(32, 128)))
    slot = PROMPT % 64
    assert torch.equal(cache._k_hot[0][0, :, slot], rope(k.view(8, 128)))
    assert torch.equal(cache._v_hot[0][0, :, slot], v.view(8, 128))
    # 3. attention over the cache as the step left it: cold codes dequantized by the oracle + the hot ring
    L = PROMPT + 1
    cold = L - 64
    cb, _ = oq.codebook_tensors(bits)
    Kc = oq.dequantize(cache._k_codes[0][:, :, :cold].cpu().numpy(), cache._k_norms[0][:, :, :cold].cpu(),
                       oq.rotation_matrix(128, 42), cb, bits).half()
    Vc = oq.dequantize(cache._v_codes[0][:, :, :cold].cpu().numpy(), cache._v_norms[0][:, :, :cold].cpu(),
                       oq.rotation_matrix(128, 43), cb, bits).half()
    order = [p % 64 for p in range(cold, L)]
    Kf = torch.cat([Kc, cache._k_hot[0][:, :, order].cpu()], dim=2)
    Vf = torch.cat([Vc, cache._v_hot[0][:, :, order].cpu()], dim=2)
    a_ref = oq.decode_attention(q_rope.cpu().view(1, 32, 1, 128), Kf, Vf).view(-1)
    attn = ws[lay.attn_out: lay.attn_out + nq * 2].view(torch.float16)
    err_attn = ot.rel_err(attn.float().cpu().numpy(), a_ref.numpy())
    report["attention"] = (err_attn, 1.0)
    assert err_attn < RTOL, err_attn
    # 4. o_proj on the attention output, then the fp16 residual add (bit-exact)
    o = _sum_chunks(ws, lay.part_o, hidden, lay.chunks_o)
    gemv_check("o_proj", _np16(attn), o, at.o_proj, t["o_proj"])
    x_mid = (x0.float() + o.float()).half()
    # 5. gate|up: one launch, two thresholds, input = RMSNorm(x_mid)
    h2 = rms_norm(x_mid.view(1, -1), layer.post_attention_layernorm.weight, model.config.rms_norm_eps).view(-1)
    h2n = _np16(h2)
    g = _sum_chunks(ws, lay.part_gate, ffn, lay.chunks_gateup)
    u = _sum_chunks(ws, lay.part_up, ffn, lay.chunks_gateup)
    gemv_check("gate_proj", h2n, g, mlp.gate_proj, t["gate_proj"])
    gemv_check("up_proj", h2n, u, mlp.up_proj, t["up_proj"])
    # 6. down on SwiGLU(g, u) with HF's fp16 rounding, then the residual add (bit-exact)
    s = (g.float() / (1 + torch.exp(-g.float()))).half().float()
    h = (s * u.float()).half()
    d = _sum_chunks(ws, lay.part_down, hidden, lay.chunks_down)
    gemv_check("down_proj", _np16(h), d, mlp.down_proj, t["down_proj"])
    assert torch.equal(x1, (x_mid.float() + d.float()).half())
    print("config-5 layer step vs oracle (rel err, kept fraction):",
          {k_: ("%.1e" % e, "%.3f" % kf) for k_, (e, kf) in report.items()})


def _hip_rmsnorm_and_lm_head(model, lm_head_cm):
    """HF path with the engine's RMSNorm arithmetic (lkv_rmsnorm) and a dense lm_head through the same GEMV kernel
    as the engine's head (threshold 0), so both paths compute every value identically."""
    from leankv_amd.kernels import rms_norm, sparse_gemv

    for m in model.modules():
        if type(m).__name__.endswith("RMSNorm"):
            m.forward = (lambda x, m=m: rms_norm(x, m.weight, m.variance_epsilon))
    head = model.lm_head
    dense = head.forward

    def fwd(h):
        if h.shape[-2] == 1 and h.shape[0] == 1:
            return sparse_gemv(h.reshape(-1), lm_head_cm.t(), 0.0).view(1, 1, -1)
        return dense(h)

    head.forward = fwd


def test_config5_engine_matches_hf_path_32_layers(cuda):
    """All 32 layers, TEAL on: engine vs the HF-patched path on the engine's tokens, identical results."""
    from leankv_amd.engine import LeanKVEngine
    from leankv_amd.turboquant.cache import TurboQuantCache

    model = _model(cuda, 32, seed=13)
    th = _thresholds(model, 13)
    prompt = _prompt(model, 13)
    cache = _patch(model, th)
    cache2 = TurboQuantCache(bits=3, head_dim=128, num_layers=32, device=cuda, max_seq_len=MAXLEN,
                             fused_attention=True)
    first = _prefill(model, cache, prompt)
    first2 = _prefill(model, cache2, prompt)
    assert int(first) == int(first2)
    eng = LeanKVEngine(model, cache2, MAXLEN)
    _hip_rmsnorm_and_lm_head(model, eng.lm_head_cm)
    eng.start(first, PROMPT)
    with torch.no_grad():
        for i in range(STEPS):
            if i == 1:
                eng.capture()
            fed = int(eng.tok)
            eng.step()
            hf = model(torch.tensor([[fed]], device=cuda), past_key_values=cache, use_cache=True).logits[0, -1]
            assert torch.equal(eng.logits, hf.half()), "step %d: logits differ" % i
            assert int(eng.tok) == int(torch.argmax(hf)), i
    assert int(eng.pos64) == PROMPT + STEPS
    for li in range(32):
        for a, b in ((cache._k_codes, cache2._k_codes), (cache._v_codes, cache2._v_codes),
                     (cache._k_norms, cache2._k_norms), (cache._v_norms, cache2._v_norms),
                     (cache._k_hot, cache2._k_hot), (cache._v_hot, cache2._v_hot)):
            assert torch.equal(a[li], b[li]), li

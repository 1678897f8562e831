"""GPU integration parity: HF-patched model and the graph-captured engine vs the CPU reference decoder.

A small random-init Mistral (head_dim 128, GQA) runs a prompt long enough to
push tokens out of the 64-token fp16 window, then greedy decode steps.  The
reference semantics (TEAL thresholds at single-token decode, fp32 quantize of
flushed tokens, attention over dequant(cold).fp16 ++ hot) are computed on the
CPU by oracle.model.RefModel, fed the same tokens (teacher forcing), and every
step's logits must agree within 2e-2 relative (fp16 activations, fp32 sums;
a TEAL mask bit may flip where an activation sits within an ulp of its
threshold, which moves logits by a few 1e-3).
"""

import numpy as np
import pytest
import torch

from oracle.model import RefModel
from oracle import teal as ot

pytestmark = pytest.mark.gpu

TINY = dict(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=128, max_position_embeddings=1024)
PROMPT, STEPS, MAXLEN = 100, 40, 160
RTOL = 2e-2


def _setup(cuda, seed=0):
    from leankv_amd.engine import random_mistral
    from leankv_amd.teal.calibrate import calibrate_thresholds, uniform_random_sparsity

    model = random_mistral(device=cuda, seed=seed, **TINY)
    g = torch.Generator().manual_seed(seed + 1)
    calib = [torch.randint(0, TINY["vocab_size"], (1, 64), generator=g)]
    th = calibrate_thresholds(model, calib, uniform_random_sparsity(0.3, 0.5, seed))
    prompt = torch.randint(0, TINY["vocab_size"], (PROMPT,), generator=g)
    state = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    return model, th, prompt, state


def _apply(model, th, max_len=MAXLEN):
    from leankv_amd.teal.patching import apply_teal
    from leankv_amd.turboquant.attention import use_on
    from leankv_amd.turboquant.cache import TurboQuantCache

    if th is not None:
        apply_teal(model, thresholds=th, use_triton=True)
    cache = TurboQuantCache(bits=3, head_dim=128, num_layers=model.config.num_hidden_layers, device=model.device,
                            max_seq_len=max_len, fused_attention=True)
    use_on(model, cache)
    return cache


def test_hf_path_turboquant_matches_reference(cuda):
    """TEAL off: the HF path with TurboQuantCache + packed-KV attention vs the CPU reference, per step."""
    model, _, prompt, state = _setup(cuda)
    ref = RefModel(state, model.config, None)
    cache = _apply(model, None)
    with torch.no_grad():
        out = model(prompt.view(1, -1).to(cuda), past_key_values=cache, use_cache=True)
    lg = out.logits[0, -1].float().cpu()
    errs = [ot.rel_err(lg.numpy(), ref.forward(prompt).numpy())]
    tok = int(torch.argmax(lg))
    for _ in range(STEPS):
        with torch.no_grad():
            out = model(torch.tensor([[tok]], device=cuda), past_key_values=cache, use_cache=True)
        lg = out.logits[0, -1].float().cpu()
        errs.append(ot.rel_err(lg.numpy(), ref.forward(torch.tensor([tok])).numpy()))
        tok = int(torch.argmax(lg))
    print("max step rel err", max(errs))
    assert max(errs) < RTOL
    assert cache.get_seq_length(0) == PROMPT + STEPS


def test_hf_path_teal_projections_match_reference(cuda):
    """TEAL on: every patched projection / fused MLP call at decode equals the oracle on its own input.

    (Model-level logits are not compared with TEAL on: one activation within an
    ulp of its threshold flips a mask bit and moves that projection's output by
    a few percent, so two correct implementations that round intermediate
    activations differently legitimately diverge.)"""
    model, th, prompt, _ = _setup(cuda, seed=2)
    cache = _apply(model, th)
    calls = []

    def grab(name, mod, li):
        def hook(m, args, out):
            if args[0].shape[-2] == 1:
                calls.append((name, li, args[0].detach().float().cpu().reshape(-1), out.detach().float().cpu().reshape(-1)))
        return mod.register_forward_hook(hook)

    hs = []
    for li, layer in enumerate(model.model.layers):
        for pn in ("q_proj", "k_proj", "v_proj", "o_proj"):
            hs.append(grab(pn, getattr(layer.self_attn, pn), li))
        hs.append(grab("down_proj", layer.mlp.down_proj, li))
        hs.append(grab("mlp", layer.mlp, li))
    with torch.no_grad():
        out = model(prompt.view(1, -1).to(cuda), past_key_values=cache, use_cache=True)
        tok = int(torch.argmax(out.logits[0, -1]))
        for _ in range(6):
            out = model(torch.tensor([[tok]], device=cuda), past_key_values=cache, use_cache=True)
            tok = int(torch.argmax(out.logits[0, -1]))
    for h in hs:
        h.remove()
    assert len(calls) == 6 * 6 * 2
    last_down_in = {}
    for name, li, x, y in calls:
        layer = model.model.layers[li]
        if name == "mlp":
            # fused gate/up + SwiGLU: its output is the input the down projection received
            wg = layer.mlp.gate_proj.weight.detach().float().cpu().numpy().astype(np.float16)
            wu = layer.mlp.up_proj.weight.detach().float().cpu().numpy().astype(np.float16)
            h = ot.gateup_swiglu(x.numpy().astype(np.float16), wg, wu, th[li]["gate_proj"], th[li]["up_proj"])
            err = ot.rel_err(last_down_in[li].numpy(), h)
        else:
            mod = getattr(layer.self_attn, name) if name != "down_proj" else layer.mlp.down_proj
            w = mod.weight.detach().float().cpu().numpy().astype(np.float16)
            err = ot.rel_err(y.numpy(), ot.sparse_gemv(x.numpy().astype(np.float16), w, th[li][name]))
            if name == "down_proj":
                last_down_in[li] = x
        assert err < RTOL, (name, li, err)


def test_engine_matches_reference_teal_off(cuda):
    """Fused decode step (TEAL off: every projection dense through the same kernels) vs the CPU reference."""
    from leankv_amd.engine import LeanKVEngine

    model, _, prompt, state = _setup(cuda, seed=4)
    ref = RefModel(state, model.config, None)
    cache = _apply(model, None)
    with torch.no_grad():
        out = model(prompt.view(1, -1).to(cuda), past_key_values=cache, use_cache=True)
    ref.forward(prompt)
    eng = LeanKVEngine(model, cache, MAXLEN)
    eng.start(torch.argmax(out.logits[0, -1]), PROMPT)
    errs = []
    with torch.no_grad():
        for i in range(STEPS):
            if i == 1:
                eng.capture()
            fed = int(eng.tok)
            eng.step()
            r = ref.forward(torch.tensor([fed]))
            errs.append(ot.rel_err(eng.logits.float().cpu().numpy(), r.numpy()))
    print("engine (TEAL off) vs reference: max step rel err %.3e" % max(errs))
    assert max(errs) < RTOL
    assert int(eng.pos64) == PROMPT + STEPS


def _hip_rmsnorm(model):
    """Route every RMSNorm module of the HF path through lkv_rmsnorm.

    TEAL thresholds are fp16 quantile values, so activations exactly at a
    threshold are common; a one-ulp difference in the RMSNorm output (torch's
    reduction order vs the fused GEMV prologue's) then flips a mask bit, which
    moves that projection by a few percent.  With the same RMSNorm arithmetic
    on both sides the comparison below is exact up to the lm_head rounding."""
    from leankv_amd.kernels import rms_norm

    for m in model.modules():
        if type(m).__name__.endswith("RMSNorm"):
            m.forward = (lambda x, m=m: rms_norm(x, m.weight, m.variance_epsilon))


def test_engine_matches_hf_path(cuda):
    """Fused decode step vs the HF-patched path (TEAL on), both fed the engine's tokens: the same
    projections (TEAL masks included), RoPE, cache append, attention, SwiGLU and residual adds;
    only lm_head differs (torch dense GEMM there, the sparse GEMV kernel at threshold 0 here)."""
    from leankv_amd.engine import LeanKVEngine

    model, th, prompt, _ = _setup(cuda, seed=3)
    _hip_rmsnorm(model)
    cache = _apply(model, th)
    cache2 = _apply_cache_only(model)
    with torch.no_grad():
        out = model(prompt.view(1, -1).to(cuda), past_key_values=cache, use_cache=True)
        out2 = model(prompt.view(1, -1).to(cuda), past_key_values=cache2, use_cache=True)
    assert torch.equal(out.logits, out2.logits)
    first = torch.argmax(out.logits[0, -1])
    eng = LeanKVEngine(model, cache2, MAXLEN)
    eng.start(first, PROMPT)
    errs, same, fed_all = [], [], []
    with torch.no_grad():
        for i in range(STEPS):
            if i == 1:
                eng.capture()
            fed = int(eng.tok)
            fed_all.append(fed)
            eng.step()
            hf = model(torch.tensor([[fed]], device=cuda), past_key_values=cache, use_cache=True).logits[0, -1]
            errs.append(float((eng.logits.float() - hf.float()).norm() / hf.float().norm()))
            same.append(int(eng.tok) == int(torch.argmax(hf)))
    print("engine vs hf: rel err max %.3e median %.3e, token agreement %d/%d"
          % (max(errs), float(np.median(errs)), sum(same), len(same)))
    assert max(errs) < 1e-3
    assert all(same)
    assert int(eng.pos64) == PROMPT + STEPS
    # the device token history holds every step's token (step at position p -> hist[p])
    assert eng.hist[PROMPT:PROMPT + STEPS].tolist() == fed_all[1:] + [int(eng.tok)]
    # the caches the two paths built are identical
    for li in range(model.config.num_hidden_layers):
        for a, b in ((cache._k_codes, cache2._k_codes), (cache._v_codes, cache2._v_codes),
                     (cache._k_norms, cache2._k_norms), (cache._k_hot, cache2._k_hot), (cache._v_hot, cache2._v_hot)):
            assert torch.equal(a[li], b[li]), li


def _apply_cache_only(model, max_len=MAXLEN):
    from leankv_amd.turboquant.cache import TurboQuantCache

    return TurboQuantCache(bits=3, head_dim=128, num_layers=model.config.num_hidden_layers, device=model.device,
                           max_seq_len=max_len, fused_attention=True)


def test_engine_graph_replays_equal_eager(cuda):
    """Replaying the captured step reproduces eager steps bit for bit (no stale workspace state)."""
    from leankv_amd.engine import LeanKVEngine

    model, th, prompt, _ = _setup(cuda, seed=5)
    cache = _apply(model, th)
    with torch.no_grad():
        out = model(prompt.view(1, -1).to(cuda), past_key_values=cache, use_cache=True)
    first = torch.argmax(out.logits[0, -1])
    # snapshot cache buffers so the same steps can run twice
    snap = [[t.clone() for t in lst] for lst in (cache._k_codes, cache._v_codes, cache._k_norms, cache._v_norms,
                                                 cache._k_hot, cache._v_hot)]
    eng = LeanKVEngine(model, cache, MAXLEN)
    eng.start(first, PROMPT)
    eager = []
    with torch.no_grad():
        for _ in range(6):
            eng.step()
            eager.append(eng.logits.clone())
        for lst, saved in zip((cache._k_codes, cache._v_codes, cache._k_norms, cache._v_norms, cache._k_hot,
                               cache._v_hot), snap):
            for t, s in zip(lst, saved):
                t.copy_(s)
        eng.start(first, PROMPT)
        eng.capture()
        for i in range(6):
            eng.step()
            torch.cuda.synchronize()
            assert torch.equal(eng.logits, eager[i]), "replay %d differs" % i
            _ = torch.zeros(1000, device=cuda).sum()  # eager work between replays


def test_dense_engine_matches_hf(cuda):
    """Dense graph engine vs HF's own fp16 forward with a DynamicCache, teacher-forced logits."""
    from transformers import DynamicCache

    from leankv_amd.engine import DenseEngine, random_mistral

    model = random_mistral(device=cuda, seed=7, **TINY)
    g = torch.Generator().manual_seed(8)
    prompt = torch.randint(0, TINY["vocab_size"], (1, PROMPT), generator=g).to(cuda)
    with torch.no_grad():
        cache = DynamicCache(config=model.config)
        out = model(prompt, past_key_values=cache, use_cache=True)
        first = torch.argmax(out.logits[0, -1])
        eng = DenseEngine(model, MAXLEN)
        n = eng.load_cache(cache)
        eng.start(first, n)
        eng.step()
        eng.capture()
        tok = first
        errs = []
        for i in range(6):
            if i > 0:
                eng.step()
            hf = model(tok.view(1, 1), past_key_values=cache, use_cache=True).logits[0, -1].float()
            errs.append(float((eng.logits.float() - hf).norm() / hf.norm()))
            tok = eng.tok.clone()
    assert max(errs) < 1e-2, errs


def test_engine_refuses_steps_past_max_len(cuda):
    """The engine tracks the position on the host: a step at max_len raises instead of overwriting the last
    RoPE row and ring slot (the device position is clamped there)."""
    from leankv_amd._lib import LeanKVError
    from leankv_amd.engine import LeanKVEngine

    model, _, prompt, _ = _setup(cuda, seed=6)
    cache = _apply(model, None)
    with torch.no_grad():
        out = model(prompt.view(1, -1).to(cuda), past_key_values=cache, use_cache=True)
    eng = LeanKVEngine(model, cache, PROMPT + 2)
    with pytest.raises(LeanKVError):
        eng.step()  # not started
    with pytest.raises(LeanKVError):
        eng.start(torch.argmax(out.logits[0, -1]), PROMPT + 2)
    eng.start(torch.argmax(out.logits[0, -1]), PROMPT)
    with pytest.raises(LeanKVError):
        eng.generate(3)
    assert len(eng.generate(2)) == 2
    with pytest.raises(LeanKVError):
        eng.step()
    assert int(eng.pos64) == PROMPT + 2


@pytest.mark.parametrize("over", [dict(num_attention_heads=4, num_key_value_heads=2),
                                  dict(num_attention_heads=8, num_key_value_heads=1),
                                  dict(num_attention_heads=20, num_key_value_heads=5, hidden_size=2560,
                                       intermediate_size=2560)], ids=["G2", "G8", "G4-10chunks"])
def test_own_dense_engine_matches_hf_and_oracle(cuda, over):
    """The dense baseline on this library's kernels (every threshold 0, fp16 paged KV) vs HF's own fp16
    forward with a DynamicCache and vs the CPU oracle without compression, teacher-forced logits.  G2:
    the split kernel sums the projection partials and appends the token itself (the splits of 128
    tokens put the new token in the first, then the second split); G8 (more than 4 query heads per kv
    head): the epilogue kernel and the general paged attention; G4-10chunks: hidden 2560 gives the
    q|k|v GEMV 10 row chunks of 256, more than the split prologue's 8 preloaded partials, so its
    general partial-sum path runs."""
    from transformers import DynamicCache

    from leankv_amd.engine import OwnDenseEngine, random_mistral

    cfg = dict(TINY, **over)
    model = random_mistral(device=cuda, seed=9, **cfg)
    state = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    ref = RefModel(state, model.config, None, hot=1 << 20)
    g = torch.Generator().manual_seed(10)
    prompt = torch.randint(0, TINY["vocab_size"], (1, PROMPT - 3), generator=g)  # not a whole number of pages
    with torch.no_grad():
        cache = DynamicCache(config=model.config)
        out = model(prompt.to(cuda), past_key_values=cache, use_cache=True)
        ref.forward(prompt[0])
        first = torch.argmax(out.logits[0, -1])
        eng = OwnDenseEngine(model, MAXLEN)
        n = eng.load_cache(cache)
        eng.start(first, n)
        errs_hf, errs_ref = [], []
        for i in range(STEPS):
            if i == 1:
                eng.capture()
            fed = eng.tok.clone()
            eng.step()
            hf = model(fed.view(1, 1), past_key_values=cache, use_cache=True).logits[0, -1].float()
            errs_hf.append(float((eng.logits.float() - hf).norm() / hf.norm()))
            errs_ref.append(ot.rel_err(eng.logits.float().cpu().numpy(), ref.forward(fed.cpu()).numpy()))
    print("own dense engine: vs HF max %.2e, vs oracle max %.2e" % (max(errs_hf), max(errs_ref)))
    assert max(errs_hf) < 1e-2, errs_hf
    assert max(errs_ref) < RTOL, errs_ref
    assert int(eng.pos64) == n + STEPS

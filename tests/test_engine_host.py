"""Host-side checks of the engine helpers (CPU only)."""

import math

import torch

TINY = dict(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=128, max_position_embeddings=8192)


def test_random_mistral_keeps_fp32_rope_frequencies():
    """fp16 parameters, fp32 rotary inverse frequencies (as from_pretrained(torch_dtype=float16) builds them):
    the fp16 RoPE table at a long-context position equals the fp32 closed form rounded once to fp16."""
    from leankv_amd.engine import MISTRAL_7B, random_mistral

    m = random_mistral(device="cpu", seed=0, **TINY)
    assert m.model.layers[0].self_attn.q_proj.weight.dtype == torch.float16
    assert m.model.rotary_emb.inv_freq.dtype == torch.float32
    assert m.config.sliding_window is None and MISTRAL_7B["sliding_window"] is None  # Mistral-7B-v0.3
    pos = torch.tensor([[4000]])
    cos, sin = m.model.rotary_emb(torch.zeros(1, 1, 128, dtype=torch.float16), pos)
    inv = [1.0 / (1e6 ** (2 * i / 128)) for i in range(64)]
    want = torch.tensor([math.cos(4000 * f) for f in inv] * 2).half()
    assert (cos[0, 0].float() - want.float()).abs().max() <= 2 ** -10  # one fp16 rounding (+ fp32 angle error)
    assert torch.get_default_dtype() == torch.float32


def test_apply_teal_installs_the_fused_qkv_and_mlp_patches():
    """With every projection patched, apply_teal fuses q|k|v and gate|up + SwiGLU (transformers' own SiLU module
    counts as SiLU); a zero threshold keeps that projection dense and its group unfused; remove_teal undoes it."""
    from leankv_amd.engine import random_mistral
    from leankv_amd.teal.patching import PROJ_NAMES, apply_teal, remove_teal

    m = random_mistral(device="cpu", seed=1, **TINY)
    th = {li: {p: 0.1 for p in PROJ_NAMES} for li in range(2)}
    th[1]["k_proj"] = 0.0
    th[1]["up_proj"] = 0.0
    apply_teal(m, thresholds=th, use_triton=True)
    l0, l1 = m.model.layers
    assert l0.self_attn._teal_qkv_fused and l0.mlp._teal_fused
    assert not hasattr(l1.self_attn, "_teal_qkv_fused") and not hasattr(l1.mlp, "_teal_fused")
    assert l0.self_attn.q_proj.weight.t().is_contiguous()  # column-major relayout of patched projections
    remove_teal(m)
    assert not hasattr(l0.self_attn, "_teal_qkv_fused") and not hasattr(l0.mlp, "_teal_fused")
    assert l0.self_attn.k_proj.forward.__func__ is torch.nn.Linear.forward
    assert l0.mlp.forward.__func__ is type(l0.mlp).forward


def test_optimize_model_paged_cache_raises_as_without_flashinfer():
    """use_paged_cache=True asks for the reference's FlashInfer fp16 pool, which is not built: RuntimeError,
    as the reference raises where FlashInfer is absent (leankv/combined.py:98-102)."""
    import pytest

    from leankv_amd.combined import optimize_model
    from leankv_amd.engine import random_mistral

    m = random_mistral(device="cpu", seed=2, **TINY)
    with pytest.raises(RuntimeError, match="FlashInfer"):
        optimize_model(m, use_paged_cache=True, page_size=16, max_pages=8)


def test_multi_row_projection_dispatch_rule():
    """Which multi-row decode products the patched projections send to the batched kernel (dense, threshold
    0) rather than torch's GEMM: 2-8 rows, or up to 32 unless the weight has more than twice as many outputs as
    inputs (gate / up); one row is the sparse GEMV's and prefill-sized inputs stay on torch."""
    from leankv_amd.teal.patching import _skinny_dense

    assert not _skinny_dense(1, 4096, 14336)
    assert all(_skinny_dense(r, 14336, 4096) for r in range(2, 9))
    assert not _skinny_dense(9, 14336, 4096) and not _skinny_dense(32, 14336, 4096)
    assert _skinny_dense(16, 4096, 4096) and _skinny_dense(32, 6144, 4096)
    assert _skinny_dense(32, 4096, 14336) and not _skinny_dense(33, 4096, 14336)
    assert not _skinny_dense(4096, 4096, 4096)
    # the fused gate/up + SwiGLU takes 2-32 rows as one grouped launch, whatever the projection rule says
    from leankv_amd.teal.patching import _skinny_gateup

    assert [r for r in range(0, 40) if _skinny_gateup(r)] == list(range(2, 33))


def _fast_path_on(m, bits=3, hot=64, n=10, B=1):
    """A TEAL-patched model behind GenerateFastPath and a fused cache whose host state says n tokens are held."""
    from leankv_amd.engine import enable_generate_fast_path
    from leankv_amd.teal.patching import PROJ_NAMES, apply_teal
    from leankv_amd.turboquant.cache import TurboQuantCache

    L = m.config.num_hidden_layers
    apply_teal(m, thresholds={li: {p: 0.1 for p in PROJ_NAMES} for li in range(L)}, use_triton=True)
    fp = enable_generate_fast_path(m)
    cache = TurboQuantCache(bits=bits, num_layers=L, hot_buffer_size=hot, device="cpu", max_seq_len=256,
                            fused_attention=True)
    for li in range(L):
        cache._alloc(li, B, m.config.num_key_value_heads, 256)
        cache._seq_lengths[li] = n
    return fp, cache


def test_generate_fast_path_eligibility_follows_the_step_checks():
    """The fast path takes a single-token call only where the fused kernels accept the model: fp16 tensors,
    no projection bias and the dimensions lkv_decode_* accept (asked of the library itself); anything else
    falls back to the model's own forward instead of failing mid-decode or reading bf16 as fp16."""
    from leankv_amd.engine import random_mistral

    ids = torch.zeros(1, 1, dtype=torch.long)
    fp, cache = _fast_path_on(random_mistral(device="cpu", seed=3, **TINY))
    assert fp._eligible(ids, cache, {}) == "one"
    fp2, cache2 = _fast_path_on(random_mistral(device="cpu", seed=3, **TINY), B=2)
    assert fp2._eligible(torch.zeros(2, 1, dtype=torch.long), cache2, {}) == "batch"

    # bf16 weights: neither engine (raw fp16 pointers), at B = 1 or B > 1
    m = random_mistral(device="cpu", seed=3, **TINY).to(torch.bfloat16)
    fp, cache = _fast_path_on(m)
    assert fp._eligible(ids, cache, {}) is None and "bfloat16" in fp._model_reason()
    fp, cache = _fast_path_on(random_mistral(device="cpu", seed=3, **TINY).to(torch.bfloat16), B=2)
    assert fp._eligible(torch.zeros(2, 1, dtype=torch.long), cache, {}) is None

    # a vocabulary the step's lm_head GEMV does not tile (Mistral fine-tunes with 32002 tokens)
    fp, cache = _fast_path_on(random_mistral(device="cpu", seed=3, **dict(TINY, vocab_size=514)))
    assert fp._model_reason() is None
    assert fp._eligible(ids, cache, {}) is None and "vocab" in fp._step_reason(cache)

    # more query heads per kv head than the step holds
    fp, cache = _fast_path_on(random_mistral(device="cpu", seed=3, **dict(
        TINY, hidden_size=2048, num_attention_heads=16, num_key_value_heads=1)))
    assert fp._eligible(ids, cache, {}) is None and "n_heads" in fp._step_reason(cache)

    # a window wider than the step's ring, and code widths the step is not built for
    fp, cache = _fast_path_on(random_mistral(device="cpu", seed=3, **TINY), hot=320, n=10)
    assert fp._eligible(ids, cache, {}) is None and "hot_cap" in fp._step_reason(cache)


def test_generate_fast_path_refuses_projection_bias():
    from leankv_amd.engine import random_mistral

    m = random_mistral(device="cpu", seed=4, **TINY)
    lin = m.model.layers[1].self_attn.o_proj
    lin.bias = torch.nn.Parameter(torch.zeros(lin.out_features, dtype=torch.float16))
    fp, cache = _fast_path_on(m)
    assert fp._eligible(torch.zeros(1, 1, dtype=torch.long), cache, {}) is None
    assert "bias" in fp._model_reason()


def test_cache_storage_generation_moves_with_its_buffers():
    """Decode engines hold raw pointers to a cache's buffers; the cache's storage generation changes exactly
    when those buffers are replaced (allocation, growth, reset), and the fast path keys its engines on it."""
    from leankv_amd.turboquant.cache import TurboQuantCache

    c = TurboQuantCache(bits=3, num_layers=2, device="cpu", max_seq_len=8)
    g0 = c.storage_generation
    c._alloc(0, 1, 2, 8)
    g1 = c.storage_generation
    assert g1 > g0
    c._ensure_cap(0, 8)  # fits: nothing replaced
    assert c.storage_generation == g1
    c._ensure_cap(0, 9)  # grows: codes and norms replaced
    assert c.storage_generation > g1 and c.cold_capacity(0) == 16
    g2 = c.storage_generation
    c.reset()
    assert c.storage_generation > g2 and c._k_codes[0] is None


def test_generate_fast_path_asks_again_after_a_dtype_change():
    """The eligibility answer is kept per model state: a model converted to bf16 after the fast path was
    installed (and asked once) stops being eligible instead of reusing the fp16 answer."""
    from leankv_amd.engine import random_mistral

    fp, cache = _fast_path_on(random_mistral(device="cpu", seed=7, **TINY))
    ids = torch.zeros(1, 1, dtype=torch.long)
    assert fp._eligible(ids, cache, {}) == "one"
    fp.model.to(torch.bfloat16)
    assert fp._eligible(ids, cache, {}) is None and "bfloat16" in fp._model_reason()

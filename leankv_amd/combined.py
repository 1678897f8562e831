"""Unified API: TEAL + TurboQuant on a HuggingFace decoder.

Drop-in for leankv/combined.py: TEALConfig / TurboQuantConfig (:32-42),
load_model (:45-54), optimize_model (:57-126), reset_optimizations (:129-132).

Differences, all in the direction of the fast path:
  * optimize_model patches the projections with the HIP sparse GEMV
    (``use_kernels=True``; the reference used the hook path here) and, when
    TurboQuant is on, selects the "leankv_tq" attention implementation so
    decode attention reads the packed cache directly.
  * with TEAL and TurboQuant both on, generate's single-token decode calls run
    the fused decode step replayed as a HIP graph (fast_decode=True, the
    default; see engine.GenerateFastPath).
  * use_paged_cache=True asks for the reference's FlashInfer fp16 page pool
    (leankv/turboquant/paged_cache.py), which HF generate never calls and
    which is not built here; it raises RuntimeError, as the reference does
    where FlashInfer is not installed (combined.py:98-102).  The paged
    TurboQuant layout is leankv_amd.turboquant.paged_tq_cache.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from .teal.patching import apply_teal, remove_teal
from .turboquant.cache import TurboQuantCache


@dataclass
class TEALConfig:
    sparsity: Optional[float] = None
    thresholds_path: Optional[str] = None


@dataclass
class TurboQuantConfig:
    bits: int = 3
    head_dim: int = 128
    num_layers: int = 32


def load_model(model_name: str, dtype=torch.float16, device_map="cuda"):
    """Load a HuggingFace model + tokenizer by name (needs the checkpoint locally or a hub)."""
    from transformers import AutoModelForCausalLM, AutoTokenizer

    print("Loading %s..." % model_name)
    model = AutoModelForCausalLM.from_pretrained(model_name, torch_dtype=dtype, device_map=device_map)
    tok = AutoTokenizer.from_pretrained(model_name)
    tok.pad_token = tok.pad_token or tok.eos_token
    return model, tok


def optimize_model(model, teal_sparsity: Optional[float] = None, teal_thresholds_path: Optional[str] = None,
                   turboquant_bits: Optional[int] = None, use_paged_cache: bool = False, page_size: int = 16,
                   max_pages: int = 2048, use_kernels: bool = True, max_seq_len: int = 4096,
                   fast_decode: bool = True):
    """Apply TEAL and/or TurboQuant; returns (model, cache or None).

    fast_decode (not in the reference): with both TEAL and TurboQuant on the HIP kernels, single-token
    decode calls of generate run the fused, graph-replayed decode step (engine.GenerateFastPath) when the
    call is one it serves; every other call runs the patched HF forward."""
    if teal_sparsity is not None or teal_thresholds_path is not None:
        apply_teal(model, sparsity=teal_sparsity, thresholds_path=teal_thresholds_path, use_triton=use_kernels)
        label = teal_thresholds_path or "%.0f%%" % (100 * teal_sparsity)
        print("[LeanKV] TEAL enabled (sparsity=%s)" % label)
    cfg = model.config
    head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
    cache = None
    if use_paged_cache:
        raise RuntimeError("use_paged_cache: the FlashInfer fp16 paged cache is not part of leankv_amd; "
                           "use leankv_amd.turboquant.paged_tq_cache.PagedTurboQuantCache for paged 3/4-bit KV")
    elif turboquant_bits is not None:
        cache = TurboQuantCache(bits=turboquant_bits, head_dim=head_dim, num_layers=cfg.num_hidden_layers,
                                device=model.device, dtype=torch.float16, max_seq_len=max_seq_len,
                                fused_attention=use_kernels)
        if cache.fused_attention:
            from .turboquant.attention import use_on

            use_on(model, cache)
        print("[LeanKV] TurboQuant enabled (bits=%d, head_dim=%d)" % (turboquant_bits, head_dim))
    teal_on = teal_sparsity is not None or teal_thresholds_path is not None
    if fast_decode and use_kernels and teal_on and cache is not None and cache.fused_attention:
        from .engine import enable_generate_fast_path

        enable_generate_fast_path(model)
    return model, cache


def reset_optimizations(model):
    from .engine import disable_generate_fast_path

    disable_generate_fast_path(model)
    remove_teal(model)
    print("[LeanKV] All optimizations removed.")

"""HF attention implementation "leankv_tq": packed-KV attention on HIP.

The reference returns dequantized fp16 K/V from TurboQuantCache.update and lets
HF run SDPA on them (leankv/turboquant/cache.py:124-127;
transformers/integrations/sdpa_attention.py:79-105).  With this function
registered (transformers AttentionInterface) and selected as the model's
attention implementation, attention over a TurboQuantCache whose update was
deferred reads the packed store: a single-token decode step runs the split-K
decode kernel, a several-token update (prefill or chunk) the causal prefill
kernel.  HF builds no mask for a custom implementation (masking_utils
_preprocess_mask_arguments), so causality is positional: query i of S sees
keys up to position kv_len - S + i, as HF's causal mask with the cache offset.
Calls with an explicit mask or a sliding window shorter than the cache, a
plain fp16 cache, or no cache, go to HF's SDPA on the reference's K/V.
"""

from __future__ import annotations

from .cache import active_cache

NAME = "leankv_tq"


def leankv_tq_attention(module, query, key, value, attention_mask, dropout: float = 0.0, scaling=None, **kwargs):
    layer_idx = getattr(module, "layer_idx", None)
    cache = active_cache()
    if cache is not None and layer_idx is not None and layer_idx < cache.num_layers:
        if query.shape[2] == 1 and cache._fused_pending[layer_idx]:
            out = cache.decode_attention(layer_idx, query, scaling)  # [B, Hq, 1, D]
            return out.transpose(1, 2).contiguous().to(query.dtype), None
        if cache._prefill_pending[layer_idx]:
            window = kwargs.get("sliding_window")
            if (attention_mask is None and not dropout
                    and (window is None or cache._pending_len[layer_idx] <= window)):
                out = cache.prefill_attention(layer_idx, query, scaling)  # [B, Hq, S, D]
                return out.transpose(1, 2).contiguous().to(query.dtype), None
            key, value = cache.take_full_cache(layer_idx)
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                                  **kwargs)


_REGISTERED = False


def register() -> str:
    """Register "leankv_tq" with transformers' AttentionInterface; returns the name."""
    global _REGISTERED
    if not _REGISTERED:
        from transformers import AttentionInterface

        AttentionInterface.register(NAME, leankv_tq_attention)
        _REGISTERED = True
    return NAME


def use_on(model) -> None:
    """Select the packed-KV attention for every attention module of `model`."""
    register()
    if hasattr(model, "set_attn_implementation"):
        try:
            model.set_attn_implementation(NAME)
            return
        except Exception:  # older transformers: fall back to the config field
            pass
    model.config._attn_implementation = NAME

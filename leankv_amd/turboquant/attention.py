"""HF attention implementation "leankv_tq": packed-KV attention on HIP.

The reference returns dequantized fp16 K/V from TurboQuantCache.update and lets
HF run SDPA on them (leankv/turboquant/cache.py:124-127;
transformers/integrations/sdpa_attention.py:79-105).  With this function
registered (transformers AttentionInterface) and selected as the model's
attention implementation, attention over a TurboQuantCache built with
``fused_attention=True`` reads the packed store: a single-token decode step
runs the split-K decode kernel, a several-token update (prefill or chunk) the
causal prefill kernel.  Causality there is positional: query i of S sees keys
up to position kv_len - S + i, HF's causal mask with the cache offset.

The name is also registered with HF's mask interface (masking_utils
AttentionMaskInterface): a forward whose mask is plain causal over the whole
cache (no padding in the 2-D attention mask, no sliding window reached) gets
no mask and takes the packed kernels; any other mask (left padding of a
batch, a sliding window shorter than the cache) is built as SDPA's boolean
mask and the call goes to HF's SDPA on the reference's K/V (cold dequantized
to fp16, then hot), which applies it.  So do calls on a plain fp16 cache, or
with no cache.
"""

from __future__ import annotations

import torch

from .cache import active_cache

NAME = "leankv_tq"


def _causal_mask(S: int, T: int, device) -> torch.Tensor:
    """Boolean [1, 1, S, T]: query i (position T - S + i) sees keys 0 .. T - S + i."""
    q = torch.arange(T - S, T, device=device).view(S, 1)
    k = torch.arange(T, device=device).view(1, T)
    return (k <= q).view(1, 1, S, T)


def leankv_tq_attention(module, query, key, value, attention_mask, dropout: float = 0.0, scaling=None, **kwargs):
    layer_idx = getattr(module, "layer_idx", None)
    cache = active_cache()
    if cache is not None and layer_idx is not None and layer_idx < cache.num_layers:
        pending = cache._fused_pending[layer_idx] or cache._prefill_pending[layer_idx]
        if pending:
            window = kwargs.get("sliding_window")
            fits = window is None or cache._pending_len[layer_idx] <= window
            if attention_mask is None and not dropout and fits:
                if cache._fused_pending[layer_idx] and query.shape[2] == 1:
                    out = cache.decode_attention(layer_idx, query, scaling)  # [B, Hq, 1, D]
                    return out.transpose(1, 2).contiguous().to(query.dtype), None
                if cache._prefill_pending[layer_idx]:
                    out = cache.prefill_attention(layer_idx, query, scaling)  # [B, Hq, S, D]
                    return out.transpose(1, 2).contiguous().to(query.dtype), None
            key, value = cache.take_full_cache(layer_idx)
            S, T = query.shape[2], key.shape[2]
            if attention_mask is None and S > 1 and T > S:
                # SDPA's is_causal aligns the mask top-left; a chunk after cached tokens needs the offset
                attention_mask = _causal_mask(S, T, query.device)
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                                  **kwargs)


def leankv_tq_mask(batch_size, q_length, kv_length, q_offset=0, kv_offset=0, mask_function=None,
                   attention_mask=None, local_size=None, allow_is_causal_skip=True, **kwargs):
    """HF mask-interface entry for "leankv_tq": None when the mask is plain causal over the whole cache with
    no padding (the packed kernels apply causality by position), else SDPA's boolean mask."""
    from transformers.masking_utils import causal_mask_function, sdpa_mask

    if mask_function is None:
        mask_function = causal_mask_function
    # HF's local masks (sliding window, chunked; local_size set) equal the causal mask while the cache
    # is no longer than the window; or/and overlays (use_vmap) are never plain
    plain = kv_offset == 0 and not kwargs.get("use_vmap", False) and (
        (mask_function is causal_mask_function and local_size is None)
        or (local_size is not None and kv_length <= local_size))
    if plain and (attention_mask is None or bool(attention_mask[:, -kv_length:].all())):
        return None
    return sdpa_mask(batch_size, q_length, kv_length, q_offset=q_offset, kv_offset=kv_offset,
                     mask_function=mask_function, attention_mask=attention_mask, local_size=local_size,
                     allow_is_causal_skip=False, **kwargs)


_REGISTERED = False


def register() -> str:
    """Register "leankv_tq" with transformers' attention and mask interfaces; returns the name."""
    global _REGISTERED
    if not _REGISTERED:
        from transformers import AttentionInterface
        from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS

        AttentionInterface.register(NAME, leankv_tq_attention)
        ALL_MASK_ATTENTION_FUNCTIONS.register(NAME, leankv_tq_mask)
        _REGISTERED = True
    return NAME


def use_on(model, cache=None) -> None:
    """Select the packed-KV attention for every attention module of `model`; with `cache` (a
    TurboQuantCache), also switch that cache to deferred (fused) attention."""
    register()
    if cache is not None:
        cache.fused_attention = True
    if hasattr(model, "set_attn_implementation"):
        try:
            model.set_attn_implementation(NAME)
            return
        except Exception:  # older transformers: fall back to the config field
            pass
    model.config._attn_implementation = NAME

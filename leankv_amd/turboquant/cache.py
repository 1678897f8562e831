"""TurboQuantCache: hot fp16 window + packed cold KV, on static device buffers.

Drop-in for leankv/turboquant/cache.py (constructor :35-80, update :84-127,
HF duck-typed interface :193-291, memory diagnostics :295-351).  Semantics are
the reference's: the last ``hot_buffer_size`` tokens of every layer stay fp16;
older tokens are quantized (as fp32, cache.py:141) with per-layer rotations
seeded ``seed + 2 i`` (keys) and ``seed + 2 i + 1`` (values); attention sees
cold tokens dequantized, then the hot window, in position order.

Storage is MI355X-shaped instead of a list of torch.cat'ed tensors:
  codes  uint8 [B, Hkv, cap, rb]   norms fp32 [B, Hkv, cap]    (cold, per K/V)
  hot    fp16  [B, Hkv, hot, 128]  ring: token p lives in slot p % hot
with rb the reference's packed row (64 bytes at 3 and 4 bits, 32 at 2, 16 at
1), so a decode step writes rb + 4 bytes per (head, K/V) instead of re-concatenating
the whole store, and ``cap`` grows by doubling when a sequence outgrows it.

By default update() returns the reference's full K/V -- cold dequantized to
fp16 by the HIP kernel, then hot -- so the cache works under any attention
implementation, exactly as the reference's (cache.py:17-19 builds it and hands
it to generate()).  ``fused_attention=True`` (what optimize_model and
``use_on(model, cache)`` set) defers attention to the packed-KV kernels and
requires the model to run the "leankv_tq" attention implementation
(leankv_amd.turboquant.attention): one new token appends with one HIP launch
and runs the split-K decode kernel, several tokens (a prefill or a chunk) are
appended with the bulk quantizer and run the causal prefill kernel; no
dequantized K/V is formed either way.  A deferred update that no leankv_tq
attention call consumed makes the next update raise instead of letting another
attention implementation read only the newest token.
"""

from __future__ import annotations

import math
import weakref

import torch

from .. import kernels as _k  # also registers torch.ops.leankv (the cache's kernels go through the dispatcher)
from .codebook import get_codebook_tensors
from .rotation import generate_rotation_matrices

_ACTIVE = None  # weakref to the cache whose update() ran last (read by the attention function)


def active_cache():
    return _ACTIVE() if _ACTIVE is not None else None


class TurboQuantCache:
    """Hybrid KV cache: compressed cold storage + fp16 hot window (static buffers)."""

    is_compileable = False
    layer_type = None

    def __init__(self, bits: int = 3, head_dim: int = 128, num_layers: int = 32, hot_buffer_size: int = 64,
                 device=None, dtype: torch.dtype = torch.float16, seed: int = 42, max_seq_len: int = 4096,
                 fused_attention: bool = False):
        if head_dim != _k.HEAD_DIM:
            raise ValueError("TurboQuantCache: head_dim=%d is not built (the HIP kernels take head_dim %d)"
                             % (head_dim, _k.HEAD_DIM))
        if bits not in (1, 2, 3, 4):
            raise ValueError("TurboQuantCache: bits must be 1..4")
        if hot_buffer_size < 1:
            raise ValueError("TurboQuantCache: hot_buffer_size must be at least 1")
        self.bits, self.head_dim, self.num_layers = bits, head_dim, num_layers
        self.hot_buffer_size = hot_buffer_size
        self._device = torch.device(device) if device is not None else torch.device("cuda")
        self._dtype = dtype
        self.fused_attention = bool(fused_attention)
        # the packed-KV attention kernels read every packing (1..4 bits); the
        # decode combine walks at most 256 hot slots: a larger window attends to
        # the dequantized K/V with SDPA
        self.fused_prefill = True
        self.fused_decode = hot_buffer_size <= 256
        self._seen_tokens = 0
        self._seq_lengths = [0] * num_layers
        self._init_cap = max(int(max_seq_len), 1)
        rot = generate_rotation_matrices(head_dim, [seed + j for j in range(2 * num_layers)], self._device,
                                         torch.float32)
        self.PiK, self.PiV = rot[0::2], rot[1::2]  # layer i: seeds seed + 2i, seed + 2i + 1
        self.centroids, bnd = get_codebook_tensors(head_dim, bits, self._device, torch.float32)
        self.decision_boundaries = bnd[1:-1].contiguous()
        self._row_bytes = _k.packed_row_bytes(bits)
        self._k_codes = [None] * num_layers
        self._v_codes = [None] * num_layers
        self._k_norms = [None] * num_layers
        self._v_norms = [None] * num_layers
        self._k_hot = [None] * num_layers
        self._v_hot = [None] * num_layers
        self._pos_dev = [None] * num_layers     # int32 [1]: length before the pending append
        self._len_dev = [None] * num_layers     # int32 [1]: length after it (attention input)
        self._fused_pending = [False] * num_layers   # a one-token update awaits decode_attention
        self._prefill_pending = [False] * num_layers  # a several-token update awaits prefill_attention
        self._pending_len = [0] * num_layers
        # bumped whenever a layer's device buffers are replaced (first allocation, growth, reset): decode
        # engines that hold raw pointers to them compare it to know when they must be rebuilt
        self.storage_generation = 0

    # ----------------------------------------------------------- storage
    def _alloc(self, layer: int, B: int, H: int, cap: int) -> None:
        dev = self._device
        self._k_codes[layer] = torch.zeros(B, H, cap, self._row_bytes, dtype=torch.uint8, device=dev)
        self._v_codes[layer] = torch.zeros(B, H, cap, self._row_bytes, dtype=torch.uint8, device=dev)
        self._k_norms[layer] = torch.zeros(B, H, cap, dtype=torch.float32, device=dev)
        self._v_norms[layer] = torch.zeros(B, H, cap, dtype=torch.float32, device=dev)
        self._k_hot[layer] = torch.zeros(B, H, self.hot_buffer_size, self.head_dim, dtype=torch.float16, device=dev)
        self._v_hot[layer] = torch.zeros_like(self._k_hot[layer])
        self._pos_dev[layer] = torch.zeros(1, dtype=torch.int32, device=dev)
        self._len_dev[layer] = torch.zeros(1, dtype=torch.int32, device=dev)
        self.storage_generation += 1

    def _ensure_cap(self, layer: int, cold_needed: int) -> None:
        cur = self._k_codes[layer].shape[2]
        if cold_needed <= cur:
            return
        new = cur
        while new < cold_needed:
            new *= 2
        for name in ("_k_codes", "_v_codes", "_k_norms", "_v_norms"):
            lst = getattr(self, name)
            old = lst[layer]
            shape = list(old.shape)
            shape[2] = new
            t = torch.zeros(shape, dtype=old.dtype, device=old.device)
            t[:, :, :cur] = old
            lst[layer] = t
        self.storage_generation += 1

    def _cold_len(self, n: int) -> int:
        return max(0, n - self.hot_buffer_size)

    def cold_capacity(self, layer: int) -> int:
        return 0 if self._k_codes[layer] is None else self._k_codes[layer].shape[2]

    def attn_max_len(self, layer: int) -> int:
        """Tokens the layer's store holds at its current capacity: the length bound every decode-attention
        launch over it is sized for."""
        return self.cold_capacity(layer) + self.hot_buffer_size

    # ----------------------------------------------------------- update
    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int, cache_kwargs=None):
        global _ACTIVE
        if self._fused_pending[layer_idx] or self._prefill_pending[layer_idx]:
            raise RuntimeError(
                "TurboQuantCache(fused_attention=True): layer %d's previous update was never attended by the "
                "'leankv_tq' attention implementation, so the model attended to the newest tokens only; call "
                "leankv_amd.turboquant.attention.use_on(model, cache) or build the cache with "
                "fused_attention=False" % layer_idx)
        _ACTIVE = weakref.ref(self)
        B, H, S, D = key_states.shape
        if layer_idx == 0:
            self._seen_tokens += S
        p0 = self._seq_lengths[layer_idx]
        if self._k_codes[layer_idx] is None:
            self._alloc(layer_idx, B, H, max(self._init_cap, self._cold_len(p0 + S), 1))
        k16 = key_states.to(torch.float16)
        v16 = value_states.to(torch.float16)
        T = p0 + S
        self._ensure_cap(layer_idx, self._cold_len(T))
        if S == 1:
            self._pos_dev[layer_idx].fill_(p0)
            torch.ops.leankv.tq_cache_append(
                k16.reshape(B, H, D).contiguous(), v16.reshape(B, H, D).contiguous(), self._k_hot[layer_idx],
                self._v_hot[layer_idx], self._k_codes[layer_idx], self._k_norms[layer_idx], self._v_codes[layer_idx],
                self._v_norms[layer_idx], self.PiK[layer_idx], self.PiV[layer_idx], self.decision_boundaries,
                self.bits, self._pos_dev[layer_idx])
        else:
            self._bulk_update(layer_idx, k16, v16, p0)
        self._seq_lengths[layer_idx] = T
        if self.fused_attention and S == 1 and self.fused_decode:
            self._len_dev[layer_idx].fill_(T)
            self._fused_pending[layer_idx] = True
            self._pending_len[layer_idx] = T
            return key_states, value_states
        if self.fused_attention and S > 1 and self.fused_prefill:
            self._prefill_pending[layer_idx] = True
            self._pending_len[layer_idx] = T
            return key_states, value_states
        return self._get_full_cache(layer_idx)

    def _bulk_update(self, li: int, k16: torch.Tensor, v16: torch.Tensor, p0: int) -> None:
        """Append S > 1 tokens: quantize every token that leaves the hot window, refill the ring.

        One gather of the ring slots that leave it and one scatter of the new window per layer (slot
        indices made on the device, no per-slot copies)."""
        hot = self.hot_buffer_size
        dev = self._device
        S = k16.shape[2]
        T = p0 + S
        c0, c1 = self._cold_len(p0), self._cold_len(T)
        if c1 > c0:
            # tokens [c0, c1) in position order: some still in the ring, the rest new
            fk = fv = None
            if min(c1, p0) > c0:
                slots = torch.arange(c0, min(c1, p0), device=dev) % hot
                fk = self._k_hot[li].index_select(2, slots)
                fv = self._v_hot[li].index_select(2, slots)
            if c1 > p0:
                nk, nv = k16[:, :, : c1 - p0], v16[:, :, : c1 - p0]
                fk = nk if fk is None else torch.cat([fk, nk], dim=2)
                fv = nv if fv is None else torch.cat([fv, nv], dim=2)
            pk, nk_ = torch.ops.leankv.tq_quantize(fk.float().contiguous(), self.PiK[li], self.decision_boundaries,
                                                   self.bits)
            pv, nv_ = torch.ops.leankv.tq_quantize(fv.float().contiguous(), self.PiV[li], self.decision_boundaries,
                                                   self.bits)
            self._k_codes[li][:, :, c0:c1] = pk
            self._v_codes[li][:, :, c0:c1] = pv
            self._k_norms[li][:, :, c0:c1] = nk_
            self._v_norms[li][:, :, c0:c1] = nv_
        first = max(p0, T - hot)  # the newest min(S, hot) tokens enter the ring, each in slot p % hot
        slots = torch.arange(first, T, device=dev) % hot
        self._k_hot[li].index_copy_(2, slots, k16[:, :, first - p0:])
        self._v_hot[li].index_copy_(2, slots, v16[:, :, first - p0:])

    def _get_full_cache(self, layer_idx: int):
        """cat(dequantize(cold).fp16, hot) in position order (cache.py:169-189)."""
        n = self._seq_lengths[layer_idx]
        c = self._cold_len(n)
        hot = self.hot_buffer_size
        idx = torch.arange(c, n, device=self._device) % hot  # ring slots in position order
        hk = self._k_hot[layer_idx].index_select(2, idx)
        hv = self._v_hot[layer_idx].index_select(2, idx)
        if c == 0:
            return hk.to(self._dtype), hv.to(self._dtype)
        ck = torch.ops.leankv.tq_dequantize(self._k_codes[layer_idx][:, :, :c], self._k_norms[layer_idx][:, :, :c],
                                            self.PiK[layer_idx], self.centroids, self.bits, torch.float16)
        cv = torch.ops.leankv.tq_dequantize(self._v_codes[layer_idx][:, :, :c], self._v_norms[layer_idx][:, :, :c],
                                            self.PiV[layer_idx], self.centroids, self.bits, torch.float16)
        return (torch.cat([ck, hk], dim=2).to(self._dtype), torch.cat([cv, hv], dim=2).to(self._dtype))

    # ----------------------------------------------------------- fused decode attention
    def decode_attention(self, layer_idx: int, query: torch.Tensor, scaling: float | None = None) -> torch.Tensor:
        """Attention of a single query [B, Hq, 1, D] over this layer's cache -> [B, Hq, 1, D]."""
        if not self._fused_pending[layer_idx]:
            raise RuntimeError("TurboQuantCache.decode_attention: no fused update pending for layer %d" % layer_idx)
        self._fused_pending[layer_idx] = False
        B, Hq, _, D = query.shape
        q = query.reshape(B, Hq, D).to(torch.float16).contiguous()
        # The launch is sized for the store's capacity, not the current length (the length itself is read on
        # the device): the split plan, and so the fp32 summation order, is then the same at every step and
        # the same as the graph-replayed decode engines' over this cache, which cannot change it per step.
        L = self.attn_max_len(layer_idx)
        scale = float(scaling) if scaling is not None else 1.0 / math.sqrt(D)
        out = torch.ops.leankv.tq_decode_attn(
            q, self._k_codes[layer_idx], self._k_norms[layer_idx], self._v_codes[layer_idx], self._v_norms[layer_idx],
            self._k_hot[layer_idx], self._v_hot[layer_idx], self.PiK[layer_idx], self.PiV[layer_idx], self.centroids,
            self.bits, self._len_dev[layer_idx], L, scale)
        return out.reshape(B, Hq, 1, D)

    def prefill_attention(self, layer_idx: int, query: torch.Tensor, scaling: float | None = None) -> torch.Tensor:
        """Causal attention of the newest S tokens' queries [B, Hq, S, D] over this layer's cache -> [B, Hq, S, D].

        Query i sits at position L - S + i and sees keys 0 .. L - S + i, the reference's
        SDPA over cat(dequantize(cold).fp16, hot) with HF's causal mask (cache.py:119-125)."""
        if not self._prefill_pending[layer_idx]:
            raise RuntimeError("TurboQuantCache.prefill_attention: no update pending for layer %d" % layer_idx)
        self._prefill_pending[layer_idx] = False
        D = query.shape[-1]
        q = query.to(torch.float16).contiguous()
        L = self._pending_len[layer_idx]
        scale = float(scaling) if scaling is not None else 1.0 / math.sqrt(D)
        return torch.ops.leankv.tq_prefill_attn(
            q, self._k_codes[layer_idx], self._k_norms[layer_idx], self._v_codes[layer_idx], self._v_norms[layer_idx],
            self._k_hot[layer_idx], self._v_hot[layer_idx], self.PiK[layer_idx], self.PiV[layer_idx], self.centroids,
            self.bits, L, scale)

    def take_full_cache(self, layer_idx: int):
        """The reference's K/V (cold dequantized to fp16, then hot) for a pending update whose attention
        runs elsewhere (a padding mask, a sliding window shorter than the cache)."""
        self._prefill_pending[layer_idx] = False
        self._fused_pending[layer_idx] = False
        return self._get_full_cache(layer_idx)

    # ----------------------------------------------------------- HF interface
    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self._seq_lengths[layer_idx] if layer_idx < len(self._seq_lengths) else 0

    def get_mask_sizes(self, query_length, layer_idx: int = 0):
        q = query_length if isinstance(query_length, int) else int(query_length.shape[0])
        return self.get_seq_length(layer_idx) + q, 0

    def get_query_offset(self, layer_idx: int = 0) -> int:
        """Position of the first query of the next forward (transformers' Cache contract: the cached length)."""
        return self.get_seq_length(layer_idx)

    def get_max_cache_shape(self, *args, **kwargs):
        return None

    def get_max_length(self):
        return None

    def has_previous_state(self, layer_idx=None):
        if layer_idx is not None:
            return layer_idx < len(self._seq_lengths) and self._seq_lengths[layer_idx] > 0
        return any(s > 0 for s in self._seq_lengths)

    def crop(self, max_length: int):
        pass

    def batch_repeat_interleave(self, repeats: int):
        pass

    def batch_select_indices(self, indices: torch.Tensor):
        pass

    def reorder_cache(self, beam_idx: torch.LongTensor):
        pass

    def reset(self):
        for lst in (self._k_codes, self._v_codes, self._k_norms, self._v_norms, self._k_hot, self._v_hot,
                    self._pos_dev, self._len_dev):
            for i in range(self.num_layers):
                lst[i] = None
        self._seq_lengths = [0] * self.num_layers
        self._fused_pending = [False] * self.num_layers
        self._prefill_pending = [False] * self.num_layers
        self._seen_tokens = 0
        self.storage_generation += 1

    @property
    def seen_tokens(self):
        return self._seen_tokens

    @property
    def key_cache(self):
        return [torch.empty(0, device=self._device)] * len([s for s in self._seq_lengths if s > 0])

    @property
    def value_cache(self):
        return self.key_cache

    @property
    def is_initialized(self):
        return any(s > 0 for s in self._seq_lengths)

    @property
    def is_sliding(self):
        return [False] * self.num_layers

    @property
    def max_batch_size(self):
        for k in self._k_hot:
            if k is not None:
                return k.shape[0]
        return 0

    @property
    def max_cache_len(self):
        return max(self._seq_lengths) if self._seq_lengths else 0

    def __len__(self) -> int:
        return len([s for s in self._seq_lengths if s > 0])

    def __getitem__(self, layer_idx: int):
        if self._seq_lengths[layer_idx] > 0:
            return self._get_full_cache(layer_idx)
        raise IndexError("Layer %d not in cache" % layer_idx)

    def __iter__(self):
        for i in range(self.num_layers):
            if self._seq_lengths[i] > 0:
                yield self._get_full_cache(i)

    def __bool__(self):
        return True

    def to_legacy_cache(self):
        return tuple(self._get_full_cache(i) for i in range(self.num_layers) if self._seq_lengths[i] > 0)

    # ----------------------------------------------------------- diagnostics (cache.py:295-351)
    def get_compressed_memory_bytes(self) -> int:
        """Bytes of the cold store actually holding tokens (codes + fp32 norms)."""
        total = 0
        for i, n in enumerate(self._seq_lengths):
            if self._k_codes[i] is None:
                continue
            B, H = self._k_codes[i].shape[:2]
            total += 2 * B * H * self._cold_len(n) * (self._row_bytes + 4)
        return total

    def get_hot_memory_bytes(self) -> int:
        total = 0
        for i, n in enumerate(self._seq_lengths):
            if self._k_hot[i] is None:
                continue
            B, H = self._k_hot[i].shape[:2]
            total += 2 * B * H * (n - self._cold_len(n)) * self.head_dim * 2
        return total

    def get_total_cache_bytes(self) -> int:
        return self.get_compressed_memory_bytes() + self.get_hot_memory_bytes()

    def get_fp16_equivalent_bytes(self) -> int:
        total = 0
        for i, n in enumerate(self._seq_lengths):
            if n > 0 and self._k_hot[i] is not None:
                B, H = self._k_hot[i].shape[:2]
                total += B * H * n * self.head_dim * 2
        return total * 2

    def get_compression_ratio(self) -> float:
        actual = self.get_total_cache_bytes()
        return 0.0 if actual == 0 else self.get_fp16_equivalent_bytes() / actual

    def print_memory_report(self):
        seq = max(self._seq_lengths) if self._seq_lengths else 0
        cold = self._cold_len(seq)
        print("[TurboQuantCache] seq=%d (cold=%d, hot=%d), actual=%.1f MB (cold=%.1f + hot=%.1f), "
              "FP16 equiv=%.1f MB, ratio=%.1fx" % (
                  seq, cold, seq - cold, self.get_total_cache_bytes() / 1e6, self.get_compressed_memory_bytes() / 1e6,
                  self.get_hot_memory_bytes() / 1e6, self.get_fp16_equivalent_bytes() / 1e6,
                  self.get_compression_ratio()))

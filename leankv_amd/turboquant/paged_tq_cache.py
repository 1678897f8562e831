"""Paged packed KV cache: TurboQuant codes in pages, fp16 hot rings per sequence.

No single reference counterpart: the reference's paged cache
(leankv/turboquant/paged_cache.py:32-362) holds fp16 K/V for FlashInfer, and
its TurboQuant cache (leankv/turboquant/cache.py:35-351) one dense store per
batch.  This joins the two for ragged batches:

  cold (per layer, per K / V)  codes uint8 [max_pages, Hkv, page_size, row_bytes] (64 at 3, 4 bits; 32 at 2; 16 at 1)
                               norms fp32  [max_pages, Hkv, page_size]
  hot  (per layer, per K / V)  fp16 [max_batch_size, Hkv, hot, 128], token p in slot p % hot

Pages come from a free list as a sequence's cold part grows (all layers of a
sequence share its page list, as in paged_cache.py:105-119) and return to it
when the sequence is freed.  Quantization follows TurboQuantCache
(cache.py:84-159): a token that leaves the hot window is quantized from its
fp16 value widened to fp32, with rotations seeded seed + 2 i (keys) and
seed + 2 i + 1 (values), so a sequence's codes equal the dense cache's bit for
bit.  decode_attention() runs lkv_tq_paged_decode_attn on the pages with
FlashInfer's CSR page table (indptr, page ids) and per-sequence lengths.
"""

from __future__ import annotations

import math

import torch

from .. import kernels as _k
from .codebook import get_codebook_tensors
from .rotation import generate_rotation_matrices


class PagedTurboQuantCache:
    is_compileable = False
    layer_type = None

    def __init__(self, num_layers: int = 32, num_kv_heads: int = 8, num_q_heads: int = 32, head_dim: int = 128,
                 bits: int = 3, hot_buffer_size: int = 64, page_size: int = 16, max_pages: int = 2048,
                 max_batch_size: int = 16, seed: int = 42, device=None):
        if head_dim != _k.HEAD_DIM:
            raise ValueError("PagedTurboQuantCache: head_dim must be %d for the HIP kernels" % _k.HEAD_DIM)
        if bits not in (1, 2, 3, 4):
            raise ValueError("PagedTurboQuantCache: bits must be 1..4")
        if page_size not in (16, 32, 64, 128):
            raise ValueError("PagedTurboQuantCache: page_size must be 16, 32, 64 or 128")
        if not 1 <= hot_buffer_size <= 256:
            raise ValueError("PagedTurboQuantCache: hot_buffer_size must be 1..256")
        if num_q_heads % num_kv_heads or num_q_heads // num_kv_heads > 16:
            raise ValueError("PagedTurboQuantCache: num_q_heads must be a multiple of num_kv_heads, at most 16x")
        self.num_layers, self.num_kv_heads, self.num_q_heads = num_layers, num_kv_heads, num_q_heads
        self.head_dim, self.bits, self.hot_buffer_size = head_dim, bits, hot_buffer_size
        self.page_size, self.max_pages, self.max_batch_size = page_size, max_pages, max_batch_size
        self._device = torch.device(device) if device is not None else torch.device("cuda")
        dev = self._device
        rot = generate_rotation_matrices(head_dim, [seed + j for j in range(2 * num_layers)], dev, torch.float32)
        self.PiK, self.PiV = rot[0::2], rot[1::2]  # layer i: seeds seed + 2i, seed + 2i + 1
        self.centroids, bnd = get_codebook_tensors(head_dim, bits, dev, torch.float32)
        self.decision_boundaries = bnd[1:-1].contiguous()
        L, H, ps = num_layers, num_kv_heads, page_size
        self._row_bytes = _k.packed_row_bytes(bits)  # 64 at 3 and 4 bits, 32 at 2, 16 at 1
        self.k_codes = torch.zeros(L, max_pages, H, ps, self._row_bytes, dtype=torch.uint8, device=dev)
        self.v_codes = torch.zeros_like(self.k_codes)
        self.k_norms = torch.zeros(L, max_pages, H, ps, dtype=torch.float32, device=dev)
        self.v_norms = torch.zeros_like(self.k_norms)
        self.k_hot = torch.zeros(L, max_batch_size, H, hot_buffer_size, head_dim, dtype=torch.float16, device=dev)
        self.v_hot = torch.zeros_like(self.k_hot)
        self._free_pages = list(range(max_pages))
        self._seq_pages: list[list[int]] = [[] for _ in range(max_batch_size)]
        self._lengths = [[0] * max_batch_size for _ in range(num_layers)]
        self._batch_size = 0
        self._seen_tokens = 0
        self._table = None  # (batch size, indptr, indices, lengths) cached until the next append

    # ------------------------------------------------------------------ pages
    def _ensure_pages(self, b: int, cold_tokens: int) -> None:
        pages = self._seq_pages[b]
        while len(pages) * self.page_size < cold_tokens:
            if not self._free_pages:
                raise RuntimeError("PagedTurboQuantCache: out of pages (%d used). Increase max_pages or reduce "
                                   "batch/sequence length." % self.max_pages)
            pages.append(self._free_pages.pop())

    def free_sequence(self, b: int) -> None:
        """Return sequence b's pages to the pool and empty it in every layer."""
        self._free_pages.extend(self._seq_pages[b])
        self._seq_pages[b] = []
        for lens in self._lengths:
            lens[b] = 0
        self._table = None

    # ------------------------------------------------------------------ appends
    def append(self, layer_idx: int, b: int, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        """Append S tokens [Hkv, S, 128] (or [1, Hkv, S, 128]) to sequence b of one layer."""
        if not 0 <= b < self.max_batch_size:
            raise IndexError("PagedTurboQuantCache: sequence %d outside max_batch_size %d" % (b, self.max_batch_size))
        for t in (key_states, value_states):
            lead = t.shape[:-3]
            if (t.dim() not in (3, 4) or any(n != 1 for n in lead) or t.shape[-3] != self.num_kv_heads
                    or t.shape[-1] != self.head_dim or t.shape != key_states.shape):
                raise ValueError("PagedTurboQuantCache.append: one sequence's states [Hkv, S, %d] or [1, Hkv, S, %d] "
                                 "expected, got %s" % (self.head_dim, self.head_dim, tuple(t.shape)))
        k16 = key_states.reshape(self.num_kv_heads, -1, self.head_dim).to(torch.float16)
        v16 = value_states.reshape(self.num_kv_heads, -1, self.head_dim).to(torch.float16)
        li, hot, ps, dev = layer_idx, self.hot_buffer_size, self.page_size, self._device
        S = k16.shape[1]
        p0 = self._lengths[li][b]
        T = p0 + S
        c0, c1 = max(0, p0 - hot), max(0, T - hot)
        if c1 > c0:
            # tokens [c0, c1) leave the window: those still in the ring first, then new ones
            self._ensure_pages(b, c1)
            fk, fv = [], []
            if p0 > c0:
                idx = torch.tensor([p % hot for p in range(c0, min(c1, p0))], dtype=torch.long, device=dev)
                fk.append(self.k_hot[li, b].index_select(1, idx))
                fv.append(self.v_hot[li, b].index_select(1, idx))
            if c1 > p0:
                fk.append(k16[:, : c1 - p0])
                fv.append(v16[:, : c1 - p0])
            fk = torch.cat(fk, dim=1).float().contiguous()
            fv = torch.cat(fv, dim=1).float().contiguous()
            pk, nk = _k.tq_quantize(fk, self.PiK[li], self.decision_boundaries, self.bits)
            pv, nv = _k.tq_quantize(fv, self.PiV[li], self.decision_boundaries, self.bits)
            pages = self._seq_pages[b]
            pg = torch.tensor([pages[p // ps] for p in range(c0, c1)], dtype=torch.long, device=dev)
            sl = torch.tensor([p % ps for p in range(c0, c1)], dtype=torch.long, device=dev)
            self.k_codes[li][pg, :, sl] = pk.transpose(0, 1)  # [n, Hkv, row bytes]
            self.v_codes[li][pg, :, sl] = pv.transpose(0, 1)
            self.k_norms[li][pg, :, sl] = nk.t()
            self.v_norms[li][pg, :, sl] = nv.t()
        keep = range(max(p0, T - hot), T)
        if len(keep):
            slots = torch.tensor([p % hot for p in keep], dtype=torch.long, device=dev)
            src = torch.tensor([p - p0 for p in keep], dtype=torch.long, device=dev)
            self.k_hot[li, b][:, slots] = k16.index_select(1, src)
            self.v_hot[li, b][:, slots] = v16.index_select(1, src)
        self._lengths[li][b] = T
        self._batch_size = max(self._batch_size, b + 1)
        self._table = None

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int, cache_kwargs=None):
        """Append [B, Hkv, S, 128] to sequences 0..B-1; return the full K/V in position order, cold
        dequantized to fp16 then hot ([B, Hkv, max_len, 128], zeros past a shorter sequence; the HF
        path's view, cache.py:169-189)."""
        B, _, S, _ = key_states.shape
        if layer_idx == 0:
            self._seen_tokens += S
        for b in range(B):
            self.append(layer_idx, b, key_states[b], value_states[b])
        return self.gather(layer_idx, B)

    def gather(self, layer_idx: int, batch_size: int):
        li, hot, ps = layer_idx, self.hot_buffer_size, self.page_size
        n_max = max(self._lengths[li][:batch_size]) if batch_size else 0
        D = self.head_dim
        keys = torch.zeros(batch_size, self.num_kv_heads, n_max, D, dtype=torch.float16, device=self._device)
        values = torch.zeros_like(keys)
        for b in range(batch_size):
            n = self._lengths[li][b]
            c = max(0, n - hot)
            if c:
                pages = self._seq_pages[b]
                pg = torch.tensor([pages[p // ps] for p in range(c)], dtype=torch.long, device=self._device)
                sl = torch.tensor([p % ps for p in range(c)], dtype=torch.long, device=self._device)
                kc = self.k_codes[li][pg, :, sl].transpose(0, 1).contiguous()  # [Hkv, c, row bytes]
                vc = self.v_codes[li][pg, :, sl].transpose(0, 1).contiguous()
                kn = self.k_norms[li][pg, :, sl].t().contiguous()
                vn = self.v_norms[li][pg, :, sl].t().contiguous()
                keys[b, :, :c] = _k.tq_dequantize(kc, kn, self.PiK[li], self.centroids, self.bits,
                                                  out_dtype=torch.float16)
                values[b, :, :c] = _k.tq_dequantize(vc, vn, self.PiV[li], self.centroids, self.bits,
                                                    out_dtype=torch.float16)
            if n > c:
                idx = torch.tensor([p % hot for p in range(c, n)], dtype=torch.long, device=self._device)
                keys[b, :, c:n] = self.k_hot[li, b].index_select(1, idx)
                values[b, :, c:n] = self.v_hot[li, b].index_select(1, idx)
        return keys, values

    def cold_arrays(self, layer_idx: int, b: int):
        """Sequence b's cold codes and norms in position order: (k_codes [Hkv, c, row bytes], k_norms [Hkv, c],
        v_codes, v_norms)."""
        li, ps = layer_idx, self.page_size
        c = max(0, self._lengths[li][b] - self.hot_buffer_size)
        pages = self._seq_pages[b]
        pg = torch.tensor([pages[p // ps] for p in range(c)], dtype=torch.long, device=self._device)
        sl = torch.tensor([p % ps for p in range(c)], dtype=torch.long, device=self._device)
        return (self.k_codes[li][pg, :, sl].transpose(0, 1), self.k_norms[li][pg, :, sl].t(),
                self.v_codes[li][pg, :, sl].transpose(0, 1), self.v_norms[li][pg, :, sl].t())

    # ------------------------------------------------------------------ attention
    def page_table(self, batch_size: int, layer_idx: int = 0):
        """(kv_indptr, kv_indices, seq_lens) int32 device tensors for sequences 0..batch_size-1."""
        key = (batch_size, layer_idx)
        if self._table is not None and self._table[0] == key:
            return self._table[1:]
        indptr, indices = [0], []
        for b in range(batch_size):
            indices.extend(self._seq_pages[b])
            indptr.append(len(indices))
        dev = self._device
        t = (torch.tensor(indptr, dtype=torch.int32, device=dev),
             torch.tensor(indices if indices else [0], dtype=torch.int32, device=dev),
             torch.tensor(self._lengths[layer_idx][:batch_size], dtype=torch.int32, device=dev))
        self._table = (key,) + t
        return t

    def decode_attention(self, layer_idx: int, query: torch.Tensor, scaling: float | None = None) -> torch.Tensor:
        """One query token per sequence, [B, Hq, 128] or [B, Hq, 1, 128] -> same shape, fp16."""
        shape = query.shape
        B = shape[0]
        q = query.reshape(B, self.num_q_heads, self.head_dim).to(torch.float16).contiguous()
        indptr, indices, lens = self.page_table(B, layer_idx)
        max_len = max(self._lengths[layer_idx][:B]) if B else 0
        li = layer_idx
        out = _k.tq_paged_decode_attn(q, self.k_codes[li], self.k_norms[li], self.v_codes[li], self.v_norms[li],
                                      self.k_hot[li, :B], self.v_hot[li, :B], self.PiK[li], self.PiV[li],
                                      self.centroids, self.bits, indptr, indices, lens, max_len,
                                      scaling if scaling is not None else 1.0 / math.sqrt(self.head_dim))
        return out.reshape(shape)

    # ------------------------------------------------------------------ HF interface / diagnostics
    def get_seq_length(self, layer_idx: int = 0) -> int:
        return max(self._lengths[layer_idx][: self._batch_size]) if self._batch_size else 0

    def get_mask_sizes(self, query_length: int, layer_idx: int = 0):
        return self.get_seq_length(layer_idx) + query_length, 0

    def get_max_length(self):
        return None

    def has_previous_state(self, layer_idx=None):
        return any(n > 0 for n in self._lengths[0])

    @property
    def seen_tokens(self):
        return self._seen_tokens

    @property
    def max_cache_len(self):
        return self.get_seq_length(0)

    def reset(self):
        self._free_pages = list(range(self.max_pages))
        self._seq_pages = [[] for _ in range(self.max_batch_size)]
        self._lengths = [[0] * self.max_batch_size for _ in range(self.num_layers)]
        self._batch_size = 0
        self._seen_tokens = 0
        self._table = None

    def get_pages_used(self) -> int:
        return self.max_pages - len(self._free_pages)

    def get_memory_usage_mb(self) -> float:
        """Cold bytes of the pages in use (codes + norms, K and V, every layer) plus the hot rings."""
        per_page = self.num_kv_heads * self.page_size * (self._row_bytes + 4) * 2
        hot = self.k_hot.numel() * 2 * 2
        return (self.get_pages_used() * per_page * self.num_layers + hot) / 1e6

    def __bool__(self):
        return True

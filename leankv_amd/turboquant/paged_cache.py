"""Paged fp16 KV cache with HIP batch decode attention.

Drop-in for leankv/turboquant/paged_cache.py (PagedKVCache): a preallocated
page pool kv_data[layer] = [max_pages][2 (K, V)][page_size][Hkv][128] fp16,
pages handed to sequences on demand from a free list, update() returning the
gathered dense K/V for HF's attention (:121-192), decode_attention() running
batch decode attention directly on the pages (:194-257; there FlashInfer,
here lkv_paged_decode_attn with the same CSR page table: indptr, page ids,
last-page lengths), and the HF cache / diagnostic interface (:260-362).

One difference on purpose: the reference allocates pages and advances the
sequence lengths while appending layer 0, and its other layers then compute the
write slot from the already advanced length, so their new tokens land one slot
late.  Here every layer writes token t of sequence b at page
_seq_page_indices[b][t // page_size], slot t % page_size (the layout the
decode attention and _gather_kv read), tracking how many tokens each layer has
written.
"""

from __future__ import annotations

import math

import torch

from .. import kernels as _k


class PagedKVCache:
    is_compileable = False
    layer_type = None

    def __init__(self, num_layers: int = 32, num_kv_heads: int = 8, num_q_heads: int = 32, head_dim: int = 128,
                 page_size: int = 16, max_pages: int = 2048, dtype: torch.dtype = torch.float16, device=None):
        if head_dim != _k.HEAD_DIM:
            raise ValueError("PagedKVCache: head_dim must be %d for the HIP kernels" % _k.HEAD_DIM)
        if dtype != torch.float16:
            raise ValueError("PagedKVCache: the pool is float16")
        if num_q_heads % num_kv_heads or num_q_heads // num_kv_heads > 16:
            raise ValueError("PagedKVCache: num_q_heads must be a multiple of num_kv_heads, at most 16x")
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.num_q_heads = num_q_heads
        self.head_dim = head_dim
        self.page_size = page_size
        self.max_pages = max_pages
        self._dtype = dtype
        self._device = torch.device(device) if device is not None else torch.device("cuda")
        self._seen_tokens = 0
        self.kv_data = torch.zeros(num_layers, max_pages, 2, page_size, num_kv_heads, head_dim, dtype=dtype,
                                   device=self._device)
        self._free_pages = list(range(max_pages))
        self._seq_page_indices: list[list[int]] = []
        self._seq_lengths: list[int] = []
        self._layer_lengths = [[] for _ in range(num_layers)]  # tokens each layer has written, per sequence
        self._batch_size = 0

    # ------------------------------------------------------------------ pages
    def _allocate_page(self) -> int:
        if not self._free_pages:
            raise RuntimeError("PagedKVCache: out of pages (%d used). Increase max_pages or reduce batch/sequence "
                               "length." % self.max_pages)
        return self._free_pages.pop()

    def _free_sequence_pages(self, batch_idx: int):
        self._free_pages.extend(self._seq_page_indices[batch_idx])
        self._seq_page_indices[batch_idx] = []
        self._seq_lengths[batch_idx] = 0
        for lens in self._layer_lengths:
            if batch_idx < len(lens):
                lens[batch_idx] = 0

    def _ensure_batch_size(self, batch_size: int):
        while len(self._seq_page_indices) < batch_size:
            self._seq_page_indices.append([])
            self._seq_lengths.append(0)
        for lens in self._layer_lengths:
            while len(lens) < batch_size:
                lens.append(0)
        self._batch_size = max(self._batch_size, batch_size)

    def _page_slot(self, b: int, t0: int, n: int):
        """(page ids, slots) as long device tensors for tokens t0 .. t0 + n of sequence b."""
        pages = self._seq_page_indices[b]
        ps = self.page_size
        pg = torch.tensor([pages[t // ps] for t in range(t0, t0 + n)], dtype=torch.long, device=self._device)
        sl = torch.tensor([t % ps for t in range(t0, t0 + n)], dtype=torch.long, device=self._device)
        return pg, sl

    # ------------------------------------------------------------------ cache ops
    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int, cache_kwargs=None):
        """Append key/value states [B, Hkv, S, D]; return the gathered dense K/V [B, Hkv, max_len, D]."""
        B, _, S, _ = key_states.shape
        if layer_idx == 0:
            self._seen_tokens += S
            self._ensure_batch_size(B)
            for b in range(B):
                need = -(-(self._seq_lengths[b] + S) // self.page_size)
                while len(self._seq_page_indices[b]) < need:
                    self._seq_page_indices[b].append(self._allocate_page())
                self._seq_lengths[b] += S
        lens = self._layer_lengths[layer_idx]
        layer = self.kv_data[layer_idx]
        for b in range(B):
            t0 = lens[b] if b < len(lens) else 0
            if b >= len(self._seq_lengths) or t0 + S > self._seq_lengths[b]:
                raise RuntimeError("PagedKVCache.update: layer %d appends past the pages layer 0 allocated"
                                   % layer_idx)
            pg, sl = self._page_slot(b, t0, S)
            layer[pg, 0, sl] = key_states[b].permute(1, 0, 2).to(self._dtype)  # in place: [S, Hkv, D]
            layer[pg, 1, sl] = value_states[b].permute(1, 0, 2).to(self._dtype)
            lens[b] = t0 + S
        return self._gather_kv(layer_idx, B)

    def _gather_kv(self, layer_idx: int, batch_size: int):
        """Dense [B, Hkv, max_len, D] copies of the pages (zeros past a shorter sequence), :170-192."""
        max_seq = max(self._seq_lengths[:batch_size]) if batch_size else 0
        keys = torch.zeros(batch_size, self.num_kv_heads, max_seq, self.head_dim, dtype=self._dtype,
                           device=self._device)
        values = torch.zeros_like(keys)
        layer = self.kv_data[layer_idx]
        for b in range(batch_size):
            n = self._seq_lengths[b]
            if n == 0:
                continue
            pg, sl = self._page_slot(b, 0, n)
            keys[b, :, :n] = layer[pg, 0, sl].permute(1, 0, 2)
            values[b, :, :n] = layer[pg, 1, sl].permute(1, 0, 2)
        return keys, values

    def page_table(self, batch_size: int):
        """FlashInfer's CSR page table as int32 device tensors: (indptr, indices, last_page_len)."""
        indptr, indices, last = [0], [], []
        for b in range(batch_size):
            pages = self._seq_page_indices[b]
            indices.extend(pages)
            indptr.append(indptr[-1] + len(pages))
            r = self._seq_lengths[b] % self.page_size
            last.append(r if r > 0 else self.page_size)
        dev = self._device
        return (torch.tensor(indptr, dtype=torch.int32, device=dev),
                torch.tensor(indices if indices else [0], dtype=torch.int32, device=dev),
                torch.tensor(last, dtype=torch.int32, device=dev))

    def decode_attention(self, layer_idx: int, query: torch.Tensor) -> torch.Tensor:
        """Batch decode attention on the pages: query [B, Hq, D] -> [B, Hq, D] (:194-257)."""
        B = query.shape[0]
        indptr, indices, last = self.page_table(B)
        max_len = max(self._seq_lengths[:B]) if B else 0
        return _k.paged_decode_attn(query.to(torch.float16).contiguous(), self.kv_data[layer_idx], indptr, indices,
                                    last, max_len, 1.0 / math.sqrt(self.head_dim))

    # ------------------------------------------------------------------ HF interface
    def get_seq_length(self, layer_idx: int = 0) -> int:
        if self._seq_lengths:
            return max(self._seq_lengths[: self._batch_size]) if self._batch_size > 0 else 0
        return 0

    def get_mask_sizes(self, query_length: int, layer_idx: int = 0):
        return self.get_seq_length(layer_idx) + query_length, 0

    def get_max_cache_shape(self, *args, **kwargs):
        return None

    def get_max_length(self):
        return self.max_pages * self.page_size

    def has_previous_state(self, layer_idx=None):
        return any(s > 0 for s in self._seq_lengths)

    def crop(self, max_length):
        pass

    def batch_repeat_interleave(self, repeats):
        pass

    def batch_select_indices(self, indices):
        pass

    def reorder_cache(self, beam_idx):
        pass

    def reset(self):
        self._free_pages = list(range(self.max_pages))
        self._seq_page_indices = []
        self._seq_lengths = []
        self._layer_lengths = [[] for _ in range(self.num_layers)]
        self._batch_size = 0
        self._seen_tokens = 0
        self.kv_data.zero_()

    @property
    def seen_tokens(self):
        return self._seen_tokens

    @property
    def key_cache(self):
        return [torch.empty(0, device=self._device)] * self.num_layers

    @property
    def value_cache(self):
        return [torch.empty(0, device=self._device)] * self.num_layers

    @property
    def is_initialized(self):
        return any(s > 0 for s in self._seq_lengths)

    @property
    def is_sliding(self):
        return [False] * self.num_layers

    @property
    def max_batch_size(self):
        return self._batch_size

    @property
    def max_cache_len(self):
        return max(self._seq_lengths) if self._seq_lengths else 0

    def __len__(self):
        return self.num_layers if any(s > 0 for s in self._seq_lengths) else 0

    def __getitem__(self, layer_idx):
        return self._gather_kv(layer_idx, self._batch_size)

    def __iter__(self):
        for i in range(self.num_layers):
            yield self._gather_kv(i, self._batch_size)

    def __bool__(self):
        return True

    # ------------------------------------------------------------------ diagnostics
    def get_pages_used(self) -> int:
        return self.max_pages - len(self._free_pages)

    def get_memory_usage_mb(self) -> float:
        bytes_per_page = 2 * self.page_size * self.num_kv_heads * self.head_dim * 2
        return self.get_pages_used() * bytes_per_page * self.num_layers / 1e6

    def get_total_pool_mb(self) -> float:
        return self.kv_data.numel() * self.kv_data.element_size() / 1e6

    def print_memory_report(self):
        seq_len = max(self._seq_lengths) if self._seq_lengths else 0
        print("[PagedKVCache] pages=%d/%d, pool=%.1f MB, used=%.1f MB, batch=%d, seq_len=%d"
              % (self.get_pages_used(), self.max_pages, self.get_total_pool_mb(), self.get_memory_usage_mb(),
                 self._batch_size, seq_len))

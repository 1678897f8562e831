"""CPU tests of the paged fp16 KV cache's host logic: page allocation and reuse, appends across layers,
the gathered dense K/V, FlashInfer's CSR page table, the HF cache interface, optimize_model wiring."""

import pytest
import torch

from leankv_amd.turboquant.paged_cache import PagedKVCache


def _cache(**kw):
    d = dict(num_layers=2, num_kv_heads=2, num_q_heads=4, page_size=4, max_pages=16, device="cpu")
    d.update(kw)
    return PagedKVCache(**d)


def test_appends_gather_back_exactly_for_every_layer():
    c = _cache()
    g = torch.Generator().manual_seed(0)
    K = [torch.randn(3, 2, 11, 128, generator=g).half() for _ in range(2)]
    V = [torch.randn(3, 2, 11, 128, generator=g).half() for _ in range(2)]
    for lo, hi in ((0, 5), (5, 6), (6, 11)):  # a prefill, one decode token, a chunk
        for li in range(2):
            k, v = c.update(K[li][:, :, lo:hi], V[li][:, :, lo:hi], li)
            assert torch.equal(k, K[li][:, :, :hi]) and torch.equal(v, V[li][:, :, :hi])
    assert c.get_seq_length() == 11 and c.seen_tokens == 11
    assert c.get_pages_used() == 3 * 3  # ceil(11 / 4) pages per sequence, shared by the layers
    for li in range(2):
        k, v = c[li]
        assert torch.equal(k, K[li]) and torch.equal(v, V[li])


def test_page_table_is_flashinfer_csr():
    c = _cache()
    c.update(torch.zeros(2, 2, 9, 128).half(), torch.zeros(2, 2, 9, 128).half(), 0)
    indptr, indices, last = c.page_table(2)
    assert indptr.tolist() == [0, 3, 6]
    assert indices.tolist() == c._seq_page_indices[0] + c._seq_page_indices[1]
    assert len(set(indices.tolist())) == 6
    assert last.tolist() == [1, 1]  # 9 = 2 * 4 + 1
    c.update(torch.zeros(2, 2, 3, 128).half(), torch.zeros(2, 2, 3, 128).half(), 0)
    assert c.page_table(2)[2].tolist() == [4, 4]  # 12 tokens: a full last page


def test_pages_are_freed_and_reused_and_exhaustion_raises():
    c = _cache(max_pages=4)
    c.update(torch.zeros(1, 2, 12, 128).half(), torch.zeros(1, 2, 12, 128).half(), 0)
    assert c.get_pages_used() == 3
    c._free_sequence_pages(0)
    assert c.get_pages_used() == 0 and c.get_seq_length() == 0
    c.update(torch.zeros(1, 2, 16, 128).half(), torch.zeros(1, 2, 16, 128).half(), 0)
    assert c.get_pages_used() == 4
    with pytest.raises(RuntimeError, match="out of pages"):
        c.update(torch.zeros(1, 2, 1, 128).half(), torch.zeros(1, 2, 1, 128).half(), 0)


def test_a_later_layer_cannot_run_ahead_of_layer_zero():
    c = _cache()
    with pytest.raises(RuntimeError, match="layer 1"):
        c.update(torch.zeros(1, 2, 3, 128).half(), torch.zeros(1, 2, 3, 128).half(), 1)


def test_hf_interface_and_diagnostics():
    c = _cache()
    assert bool(c) and len(c) == 0 and not c.is_initialized
    c.update(torch.zeros(1, 2, 5, 128).half(), torch.zeros(1, 2, 5, 128).half(), 0)
    assert len(c) == 2 and c.is_initialized and c.has_previous_state()
    assert c.get_mask_sizes(1) == (6, 0)
    assert c.get_max_length() == 16 * 4
    assert c.max_cache_len == 5 and c.max_batch_size == 1
    assert c.get_memory_usage_mb() == pytest.approx(2 * 2 * 4 * 2 * 128 * 2 * 2 / 1e6)
    c.reset()
    assert c.get_pages_used() == 0 and c.get_seq_length() == 0 and float(c.kv_data.abs().sum()) == 0.0


def test_optimize_model_builds_the_paged_cache():
    from transformers import MistralConfig, MistralForCausalLM

    from leankv_amd.combined import optimize_model

    cfg = MistralConfig(vocab_size=64, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                        num_attention_heads=4, num_key_value_heads=2, head_dim=128)
    model = MistralForCausalLM(cfg)
    _, cache = optimize_model(model, use_paged_cache=True, page_size=16, max_pages=8)
    assert isinstance(cache, PagedKVCache)
    assert (cache.num_layers, cache.num_kv_heads, cache.num_q_heads, cache.page_size, cache.max_pages) == (2, 2, 4,
                                                                                                          16, 8)


def test_paged_tq_cache_rejects_batched_states_in_append():
    from leankv_amd.turboquant.paged_tq_cache import PagedTurboQuantCache

    c = PagedTurboQuantCache(num_layers=1, num_kv_heads=2, num_q_heads=4, max_pages=4, max_batch_size=2,
                             device="cpu")
    with pytest.raises(ValueError, match="one sequence"):
        c.append(0, 0, torch.zeros(2, 2, 3, 128), torch.zeros(2, 2, 3, 128))  # a batch of 2, not one sequence
    with pytest.raises(ValueError, match="one sequence"):
        c.append(0, 0, torch.zeros(3, 3, 128), torch.zeros(3, 3, 128))  # 3 heads for a 2-head cache
    with pytest.raises(IndexError):
        c.append(0, 2, torch.zeros(2, 3, 128), torch.zeros(2, 3, 128))
    assert c.get_pages_used() == 0 and c.get_seq_length() == 0

"""Host-side decode bookkeeping (CPU): the held tail's descriptor, kept per tail layout and token count."""

from __future__ import annotations

import torch

from dartkv_amd import cache as C


def _cache_with_tail(tokens: int, capacity: int = 224) -> C.DartKVCache:
    cache = C.DartKVCache(C.DartKVCacheConfig(bits=2, page_size=128, promote_ratio=0.25, sink_tokens=32,
                                              hold_partial_pages=True))
    tk = torch.zeros(2, 4, capacity, 128, dtype=torch.bfloat16)
    tv = torch.zeros_like(tk)
    cache._tail_key, cache._tail_value = tk, tv
    cache._pending_key, cache._pending_value = tk.narrow(2, 0, tokens), tv.narrow(2, 0, tokens)
    return cache


def test_tail_descriptor_is_kept_while_layout_and_count_stay():
    cache = _cache_with_tail(5)
    d1, dense_ok = C.tail_segment(cache, with_dense_check=True)
    assert dense_ok and d1.tokens == 5
    assert d1.key[0] == cache._tail_key.data_ptr() and d1.value[0] == cache._tail_value.data_ptr()
    assert d1.key_bh[0] == cache._tail_key.stride(1) and d1.value_bh[0] == cache._tail_value.stride(1)
    assert C.tail_segment(cache) is d1  # nothing changed: the same descriptor

    # one more token: a descriptor with the new count at the same addresses; the old one is untouched
    cache._pending_key = cache._tail_key.narrow(2, 0, 6)
    cache._pending_value = cache._tail_value.narrow(2, 0, 6)
    d2 = C.tail_segment(cache)
    assert d2 is not d1 and d2.tokens == 6 and d1.tokens == 5
    assert (d2.key[0], d2.value[0], d2.key_bh[0]) == (d1.key[0], d1.value[0], d1.key_bh[0])

    # new tail tensors (a batch reorder, a device move): the descriptor follows their addresses
    tk, tv = cache._tail_key.clone(), cache._tail_value.clone()
    cache._tail_key, cache._tail_value = tk, tv
    cache._pending_key, cache._pending_value = tk.narrow(2, 0, 6), tv.narrow(2, 0, 6)
    d3 = C.tail_segment(cache)
    assert d3.key[0] == tk.data_ptr() and d3.value[0] == tv.data_ptr() and d3.tokens == 6


def test_no_held_tail_is_an_empty_descriptor():
    cache = C.DartKVCache(C.DartKVCacheConfig(bits=2, page_size=128))
    desc, dense_ok = C.tail_segment(cache, with_dense_check=True)
    assert desc.tokens == 0 and dense_ok
    assert C.tail_segment(cache).tokens == 0

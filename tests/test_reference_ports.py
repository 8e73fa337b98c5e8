"""The reference's own cache, quantization and attention tests, run against dartkv_amd.

Each test names the reference test it ports (reference tests/test_cache.py,
tests/test_quantization.py, tests/test_attention.py,
tests/test_fused_attention.py).  Literals, shapes, seeds and message
substrings are the reference's; tensors live on the GPU because dartkv_amd has
no CPU compute path (argument checks that fail before any device work run on
the CPU).  Differences from the reference are stated where they occur:

* the reference's CPU-only `fused_dart_attention` fallback becomes a GPU
  comparison of the fused and streamed entry points;
* Triton-gated reference tests (page runs vs per-page launches) run
  unconditionally: the HIP path is always present.
"""

from __future__ import annotations

import pytest
import torch

import dartkv_amd as dart
from dartkv_amd import DartKVCache, DartKVCacheConfig

DEV = "cuda"
gpu = pytest.mark.gpu


# ------------------------------------------------------------------ CPU -----

def test_invalid_quantization_inputs():
    """tests/test_quantization.py:26-34 (validation precedes any device work)."""
    with pytest.raises(ValueError, match="bits"):
        dart.quantize(torch.ones(2, 3), bits=3)
    with pytest.raises(ValueError, match="group_size"):
        dart.quantize(torch.ones(2, 3), group_size=0)
    with pytest.raises(TypeError, match="floating"):
        dart.quantize(torch.ones(2, 3, dtype=torch.int32))
    with pytest.raises(ValueError, match="finite"):
        dart.quantize(torch.tensor([[float("nan")]]))


def test_config_rejects_bad_values():
    """The messages of reference src/dart/cache.py:70-96."""
    for kw, exc, msg in [(dict(bits=3), ValueError, "bits"), (dict(group_size=0), ValueError, "group_size"),
                         (dict(sink_tokens=-1), ValueError, "sink_tokens"), (dict(key_bits=5), ValueError, "key_bits"),
                         (dict(value_group_size=0), ValueError, "value_group_size"),
                         (dict(page_size=0), ValueError, "page_size"), (dict(local_tokens=-1), ValueError, "local"),
                         (dict(promote_bits=8), ValueError, "promote_bits"),
                         (dict(promote_ratio=1.5), ValueError, "promote_ratio"),
                         (dict(channel_selection="x"), ValueError, "channel_selection"),
                         (dict(metadata_dtype=torch.int8), TypeError, "metadata_dtype")]:
        with pytest.raises(exc, match=msg):
            DartKVCacheConfig(**kw)


def test_empty_cache_page_table_on_host():
    """tests/test_cache.py:126-129: an empty cache has a valid empty table (no device needed)."""
    cache = DartKVCache(DartKVCacheConfig(page_size=4))
    empty = cache.page_table().validate()
    assert empty.page_ids.shape == (0, 0)
    assert cache.page_table() is empty
    assert cache.page_runs() == ()


# ------------------------------------------------------------------ GPU -----

@gpu
def test_cache_preserves_sink_and_supports_incremental_updates():
    """tests/test_cache.py:8-26."""
    torch.manual_seed(2)
    keys = torch.randn(1, 2, 5, 7, dtype=torch.float32).to(DEV)
    values = torch.randn_like(keys)
    cache = DartKVCache(DartKVCacheConfig(bits=4, group_size=4, sink_tokens=2, metadata_dtype=torch.float32))

    first_keys, first_values = cache.update(keys[..., :1, :], values[..., :1, :])
    assert cache.get_seq_length() == 1
    torch.testing.assert_close(first_keys, keys[..., :1, :])
    torch.testing.assert_close(first_values, values[..., :1, :])

    restored_keys, restored_values = cache.update(keys[..., 1:, :], values[..., 1:, :])
    assert cache.get_seq_length() == 5
    assert restored_keys.shape == keys.shape
    assert restored_values.shape == values.shape
    torch.testing.assert_close(restored_keys[..., :2, :], keys[..., :2, :])
    torch.testing.assert_close(restored_values[..., :2, :], values[..., :2, :])
    assert cache.storage_bytes < cache.dense_bytes
    assert cache.compression_ratio > 1.0


@gpu
def test_cache_rejects_incompatible_updates_and_can_clear():
    """tests/test_cache.py:29-41."""
    cache = DartKVCache()
    key = torch.zeros(1, 1, 1, 4, device=DEV)
    cache.update(key, key)
    with pytest.raises(ValueError, match="batch/head/head_dim"):
        incompatible = torch.zeros(1, 2, 1, 4, device=DEV)
        cache.update(incompatible, incompatible)
    with pytest.raises(ValueError, match="dtype"):
        cache.update(key.half(), key.half())
    cache.clear()
    assert len(cache) == 0
    with pytest.raises(RuntimeError, match="empty"):
        cache.get()


@gpu
def test_cache_rejects_mismatched_key_value_dtype():
    """tests/test_cache.py:44-49."""
    cache = DartKVCache()
    keys = torch.zeros(1, 1, 1, 4, dtype=torch.float32, device=DEV)
    values = torch.zeros_like(keys, dtype=torch.float16)
    with pytest.raises(ValueError, match="same dtype and device"):
        cache.update(keys, values)


@gpu
def test_cache_separates_key_value_axes_and_flushes_pages():
    """tests/test_cache.py:52-73."""
    torch.manual_seed(5)
    keys = torch.randn(1, 2, 9, 16).to(DEV)
    values = torch.randn_like(keys)
    cache = DartKVCache(DartKVCacheConfig(page_size=4, hold_partial_pages=True, sink_tokens=1, key_group_size=4,
                                          value_group_size=8, promote_ratio=0.25, metadata_dtype=torch.float32))
    restored_keys, restored_values = cache.update(keys, values)
    assert cache.get_seq_length() == 9
    assert cache._pending_key is None
    assert restored_keys.shape == keys.shape
    assert restored_values.shape == values.shape
    cache.update(keys[..., :3, :], values[..., :3, :])
    assert cache._pending_key is not None
    assert cache.get_seq_length() == 12
    assert cache.storage_bytes < cache.dense_bytes


@gpu
def test_page_metadata_freezes_sequence_order_and_storage_strides():
    """tests/test_cache.py:76-99."""
    torch.manual_seed(51)
    keys = torch.randn(1, 2, 11, 12).to(DEV)
    values = torch.randn_like(keys)
    cache = DartKVCache(DartKVCacheConfig(page_size=4, hold_partial_pages=True, sink_tokens=2, key_group_size=4,
                                          value_group_size=6, promote_ratio=0.25, metadata_dtype=torch.float32))
    cache.update(keys, values)
    pages = cache.page_metadata()
    assert [(page.sequence_start, page.token_count) for page in pages] == [(0, 2), (2, 4), (6, 4), (10, 1)]
    assert pages[0].key.kind == pages[0].value.kind == "dense"
    assert pages[1].key.kind == "mixed_key"
    assert pages[1].value.kind == "quantized"
    assert pages[1].key.fields[0][0] == "low_values"
    assert pages[1].key.fields[0][2][-1] == 1
    assert pages[1].value.fields[0][2][-1] == 1
    assert pages[-1].token_count == 1
    assert sum(page.token_count for page in pages) == cache.seen_tokens


@gpu
def test_page_table_tracks_kitty_style_ids_modes_and_reorder():
    """tests/test_cache.py:102-123."""
    torch.manual_seed(52)
    keys = torch.randn(2, 2, 11, 12).to(DEV)
    values = torch.randn_like(keys)
    cache = DartKVCache(DartKVCacheConfig(page_size=4, hold_partial_pages=True, sink_tokens=2, key_group_size=4,
                                          value_group_size=6, promote_ratio=0.25, metadata_dtype=torch.float32))
    cache.update(keys, values)
    table = cache.page_table().validate()
    assert table.page_ids.shape == (2, 4)
    assert table.page_ids.tolist() == [[0, 1, 2, 3], [0, 1, 2, 3]]
    assert table.sequence_ranges().tolist() == [[0, 2], [2, 6], [6, 10], [10, 11]]
    assert table.key_modes.tolist() == [0, 2, 2, 0]
    assert table.value_modes.tolist() == [0, 1, 1, 0]
    assert table.reorder(torch.tensor([1, 1])).page_ids.tolist() == [[0, 1, 2, 3], [0, 1, 2, 3]]
    assert table.to("cpu").device.type == "cpu"


@gpu
def test_empty_page_table_is_valid_and_append_refreshes_metadata():
    """tests/test_cache.py:126-134."""
    cache = DartKVCache(DartKVCacheConfig(page_size=4))
    empty = cache.page_table().validate()
    assert empty.page_ids.shape == (0, 0)
    key = torch.randn(1, 1, 5, 8, device=DEV)
    cache.update(key, key)
    table = cache.page_table().validate()
    assert table.page_count == 2
    assert table.seen_tokens == 5


@gpu
def test_page_descriptors_are_cached_and_invalidated_by_cache_lifecycle():
    """tests/test_cache.py:137-176."""
    torch.manual_seed(55)
    keys = torch.randn(2, 1, 9, 8).to(DEV)
    cache = DartKVCache(DartKVCacheConfig(page_size=4, hold_partial_pages=True, key_group_size=4, value_group_size=4,
                                          metadata_dtype=torch.float32))
    assert cache.layout_version == 0
    empty_table = cache.page_table()
    assert cache.page_table() is empty_table
    cache.update(keys[..., :8, :], keys[..., :8, :])
    assert cache.layout_version == 1
    table = cache.page_table()
    runs = cache.page_runs()
    assert cache.page_table() is table
    assert cache.page_runs() is runs
    assert table.page_count == 2
    assert len(runs) == 1 and runs[0].page_count == 2

    cache.update(keys[..., 8:, :], keys[..., 8:, :])
    assert cache.layout_version == 2
    refreshed_table = cache.page_table()
    refreshed_runs = cache.page_runs()
    assert refreshed_table is not table
    assert refreshed_runs is not runs
    assert refreshed_table.page_count == 3
    assert refreshed_runs[0].page_count == 2

    rebuilt = cache.page_table(rebuild=True)
    assert rebuilt is not refreshed_table
    cache.to("cpu")
    assert cache.layout_version == 3
    moved_table = cache.page_table()
    assert moved_table is not rebuilt
    cache.clear()
    assert cache.layout_version == 4
    assert cache.page_table().page_count == 0


@gpu
def test_custom_reordered_page_table_does_not_replace_cache_owned_run():
    """tests/test_cache.py:179-188."""
    torch.manual_seed(56)
    keys = torch.randn(2, 1, 8, 8).to(DEV)
    cache = DartKVCache(DartKVCacheConfig(page_size=4, key_group_size=4, value_group_size=4))
    cache.update(keys, keys)
    owned_runs = cache.page_runs()
    reordered = cache.page_table().reorder(torch.tensor([1, 0])).validate()
    custom_runs = cache.page_runs(page_table=reordered)
    assert custom_runs is not owned_runs
    assert cache.page_runs() is owned_runs


@gpu
def test_page_table_stacks_consecutive_uniform_pages_page_major():
    """tests/test_cache.py:191-216."""
    torch.manual_seed(53)
    keys = torch.randn(1, 2, 13, 16).to(DEV)
    values = torch.randn_like(keys)
    cache = DartKVCache(DartKVCacheConfig(page_size=4, hold_partial_pages=True, sink_tokens=1, key_group_size=4,
                                          value_group_size=8, metadata_dtype=torch.float32))
    cache.update(keys, values)
    table = cache.page_table().validate()
    runs = table.uniform_quantized_runs(cache)
    assert len(runs) == 1
    run = runs[0].validate()
    assert run.first_page_index == 1
    assert run.page_indices.tolist() == [1, 2, 3]
    assert run.sequence_starts.tolist() == [1, 5, 9]
    assert run.token_counts.tolist() == [4, 4, 4]
    assert run.key_values.shape[:4] == (3, 1, 2, 16)
    assert run.value_values.shape[:4] == (3, 1, 2, 4)
    assert run.key_scale.shape[0] == run.value_scale.shape[0] == 3
    # the run's page p holds the bytes of segment first + p
    segs = cache.iter_segments()
    for p in range(3):
        kseg, vseg = segs[1 + p]
        assert torch.equal(run.key_values[p], kseg.values) and torch.equal(run.value_values[p], vseg.values)
        assert torch.equal(run.key_scale[p], kseg.scale) and torch.equal(run.value_zero_point[p], vseg.zero_point)


@gpu
def test_page_runs_stop_at_mixed_and_pending_tail_pages():
    """tests/test_cache.py:219-232."""
    torch.manual_seed(54)
    keys = torch.randn(1, 1, 10, 8).to(DEV)
    cache = DartKVCache(DartKVCacheConfig(page_size=4, hold_partial_pages=True, promote_ratio=0.25, key_group_size=4,
                                          value_group_size=4, metadata_dtype=torch.float32))
    cache.update(keys, keys)
    table = cache.page_table().validate()
    assert table.key_modes.tolist() == [2, 2, 0]
    assert table.value_modes.tolist() == [1, 1, 0]
    assert table.uniform_quantized_runs(cache) == ()


@gpu
def test_local_tokens_preserve_kitty_style_fp16_suffix_until_next_page():
    """tests/test_cache.py:235-262."""
    torch.manual_seed(57)
    keys = torch.randn(1, 1, 13, 8).to(DEV)
    cache = DartKVCache(DartKVCacheConfig(page_size=4, local_tokens=4, key_group_size=4, value_group_size=4,
                                          metadata_dtype=torch.float32))
    cache.update(keys, keys)
    pages = cache.page_metadata()
    assert [(page.key.kind, page.token_count) for page in pages] == [("quantized", 4), ("quantized", 4), ("dense", 5)]
    assert cache.page_table().key_modes.tolist() == [1, 1, 0]
    cache.update(keys[..., :3, :], keys[..., :3, :])
    pages = cache.page_metadata()
    assert [(page.key.kind, page.token_count) for page in pages] == [
        ("quantized", 4), ("quantized", 4), ("quantized", 4), ("dense", 4)]
    restored, _ = cache.get()
    assert restored.shape[-2] == 16


@gpu
def test_cache_runs_on_gpu_and_moves_to_the_host():
    """tests/test_cache.py:308-318.  After ``to("cpu")`` the pages live in host memory; ``get()``
    dequantizes them on the GPU and returns host tensors."""
    key = torch.randn(1, 1, 3, 16, device=DEV, dtype=torch.float16)
    cache = DartKVCache(DartKVCacheConfig(bits=2, group_size=8, metadata_dtype=torch.float16))
    restored, _ = cache.update(key, key)
    assert restored.device.type == "cuda"
    cache.to("cpu")
    restored_cpu, _ = cache.get()
    assert restored_cpu.device.type == "cpu"
    assert torch.equal(restored_cpu, restored.cpu())
    table = cache.page_table().validate()
    assert table.device.type == "cpu"
    assert table.page_count == 1


@gpu
@pytest.mark.parametrize("bits,tolerance", [(2, 0.55), (4, 0.12), (8, 0.01)])
def test_round_trip_supports_non_divisible_dimension(bits, tolerance):
    """tests/test_quantization.py:7-17."""
    torch.manual_seed(1)
    source = torch.randn(2, 3, 7, dtype=torch.float32).to(DEV)
    packed = dart.quantize(source, bits=bits, group_size=4, metadata_dtype=torch.float32)
    restored = dart.dequantize(packed)
    assert restored.shape == source.shape
    assert restored.dtype == source.dtype
    assert torch.max(torch.abs(source - restored)).item() <= tolerance
    assert packed.values.dtype == torch.uint8
    assert packed.nbytes < packed.dense_nbytes


@gpu
def test_constant_group_is_stable():
    """tests/test_quantization.py:20-23."""
    source = torch.full((1, 5), 3.25, dtype=torch.float32, device=DEV)
    restored = dart.quantize(source, bits=2, group_size=8, metadata_dtype=torch.float32).dequantize()
    torch.testing.assert_close(restored, source)


@gpu
def test_quantize_axis_restores_original_layout():
    """tests/test_quantization.py:37-44."""
    torch.manual_seed(3)
    source = torch.randn(2, 3, 9, 5).to(DEV)
    packed = dart.quantize_axis(source, axis=-2, bits=2, group_size=4, metadata_dtype=torch.float32)
    restored = packed.dequantize()
    assert restored.shape == source.shape
    assert packed.scale.shape == (2, 3, 5, 3)
    assert torch.max((source - restored).abs()).item() < 0.9


@gpu
def test_mixed_key_stores_only_promoted_high_bits():
    """tests/test_quantization.py:47-60."""
    torch.manual_seed(4)
    source = torch.randn(1, 2, 17, 16).to(DEV)
    mask, indices = dart.select_key_channels(source, 0.25, strategy="magnitude")
    assert mask.shape == (1, 2, 16)
    assert indices.shape == (1, 2, 4)
    mixed = dart.quantize_key_mixed(source, group_size=8, promote_ratio=0.25, metadata_dtype=torch.float32)
    restored = mixed.dequantize()
    assert restored.shape == source.shape
    assert mixed.high_values.shape[2] == 4
    assert mixed.promote_mask.sum().item() == 8
    assert mixed.nbytes < mixed.dense_nbytes
    assert torch.max((source - restored).abs()).item() < 0.9


def _forbid_get(cache):
    def raise_on_get():
        raise AssertionError("the attention path materialized the full cache")
    cache.get = raise_on_get


@gpu
def test_streamed_attention_matches_dense_materialized_cache_without_get():
    """tests/test_attention.py:6-30."""
    torch.manual_seed(7)
    keys = torch.randn(1, 2, 19, 8).to(DEV)
    values = torch.randn_like(keys)
    query = torch.randn(1, 4, 3, 8).to(DEV)
    cache = DartKVCache(DartKVCacheConfig(page_size=5, key_group_size=5, value_group_size=4, promote_ratio=0.25,
                                          sink_tokens=1, metadata_dtype=torch.float32))
    cache.update(keys, values)
    dense_keys, dense_values = cache.get()
    expected = dart.dense_attention(query, dense_keys.repeat_interleave(2, dim=1),
                                    dense_values.repeat_interleave(2, dim=1))
    _forbid_get(cache)
    actual = dart.streamed_dart_attention(query, cache)
    assert actual.shape == expected.shape
    torch.testing.assert_close(actual, expected, rtol=2e-3, atol=2e-3)


@gpu
def test_streamed_attention_supports_pending_page():
    """tests/test_attention.py:33-49."""
    torch.manual_seed(8)
    keys = torch.randn(1, 1, 7, 8).to(DEV)
    values = torch.randn_like(keys)
    query = torch.randn(1, 1, 1, 8).to(DEV)
    cache = DartKVCache(DartKVCacheConfig(page_size=4, hold_partial_pages=True, key_group_size=4, value_group_size=4,
                                          metadata_dtype=torch.float32))
    cache.update(keys, values)
    dense_keys, dense_values = cache.get()
    expected = dart.dense_attention(query, dense_keys, dense_values)
    actual = dart.streamed_dart_attention(query, cache)
    torch.testing.assert_close(actual, expected, rtol=2e-3, atol=2e-3)


@gpu
def test_fused_attention_matches_streaming_reference():
    """tests/test_fused_attention.py:14-24 (there a CPU fallback; here both entry points on the GPU)."""
    torch.manual_seed(71)
    keys = torch.randn(1, 1, 9, 8).to(DEV)
    values = torch.randn_like(keys)
    query = torch.randn(1, 1, 1, 8).to(DEV)
    cache = DartKVCache(DartKVCacheConfig(page_size=4, hold_partial_pages=True, metadata_dtype=torch.float32))
    cache.update(keys, values)
    actual = dart.fused_dart_attention(query, cache)
    expected = dart.streamed_dart_attention(query, cache)
    torch.testing.assert_close(actual, expected, rtol=2e-3, atol=2e-3)


@gpu
def test_fused_attention_handles_sink_pages_pending_and_gqa_without_get():
    """tests/test_fused_attention.py:27-53."""
    torch.manual_seed(72)
    keys = torch.randn(1, 2, 21, 16, device=DEV, dtype=torch.float16)
    values = torch.randn_like(keys)
    query = torch.randn(1, 4, 1, 16, device=DEV, dtype=torch.float16)
    cache = DartKVCache(DartKVCacheConfig(page_size=8, sink_tokens=3, hold_partial_pages=True, key_group_size=8,
                                          value_group_size=8, promote_ratio=0.25, metadata_dtype=torch.float16))
    cache.update(keys, values)
    dense_keys, dense_values = cache.get()
    expected = dart.dense_attention(query, dense_keys.repeat_interleave(2, dim=1),
                                    dense_values.repeat_interleave(2, dim=1))
    _forbid_get(cache)
    actual = dart.fused_dart_attention(query, cache, fallback=False)
    torch.testing.assert_close(actual, expected, rtol=3e-2, atol=3e-3)


@gpu
def test_fused_attention_page_run_matches_per_page_kernel():
    """tests/test_fused_attention.py:56-79."""
    torch.manual_seed(73)
    keys = torch.randn(1, 2, 35, 32, device=DEV, dtype=torch.float16)
    values = torch.randn_like(keys)
    query = torch.randn(1, 8, 1, 32, device=DEV, dtype=torch.float16)
    cache = DartKVCache(DartKVCacheConfig(page_size=8, sink_tokens=3, hold_partial_pages=True, key_group_size=8,
                                          value_group_size=8, metadata_dtype=torch.float16))
    cache.update(keys, values)
    table = cache.page_table(device=query.device).validate()
    runs = table.uniform_quantized_runs(cache)
    assert runs and runs[0].page_count >= 3
    page_run = dart.fused_dart_attention(query, cache, page_table=table, page_runs=runs, fallback=False)
    per_page = dart.fused_dart_attention(query, cache, page_table=table, page_runs=(), fallback=False)
    torch.testing.assert_close(page_run, per_page, rtol=2e-3, atol=2e-3)


# ----------------------------------------------- beyond the reference tests -----

@gpu
@pytest.mark.parametrize("side,bad,promote", [("key", float("nan"), 0.25), ("key", float("inf"), 0.0),
                                              ("value", float("-inf"), 0.25), ("value", float("nan"), 0.0),
                                              ("key", float("nan"), 0.0)])
@pytest.mark.parametrize("head_dim,dtype", [(128, torch.bfloat16), (12, torch.bfloat16), (32, torch.float64)])
def test_non_finite_page_inputs_raise_like_the_reference(side, bad, promote, head_dim, dtype):
    """A NaN or an infinity in a token that is quantized raises the reference's ValueError
    (mixed keys: mixed.py:187-188; uniform keys and values: quantization.py:159-160); the cache
    is left as it was, and a finite append afterwards works.  Head dims 128 and 12 reach the
    single-pass and the general key kernels; float64 caches the double-precision kernels."""
    cfg = DartKVCacheConfig(bits=2, page_size=16, key_group_size=16, value_group_size=4, promote_ratio=promote,
                            sink_tokens=2, hold_partial_pages=True, metadata_dtype=torch.float16)
    torch.manual_seed(9)
    keys = torch.randn(2, 2, 40, head_dim, device=DEV, dtype=dtype)
    values = torch.randn_like(keys)
    cache = DartKVCache(cfg)
    cache.update(keys[..., :20, :], values[..., :20, :])
    before = [(s.sequence_start, s.token_count) for s in cache.page_metadata()]
    bad_keys, bad_values = keys[..., 20:, :].clone(), values[..., 20:, :].clone()
    (bad_keys if side == "key" else bad_values)[1, 0, 7, 3] = bad
    msg = "key_states must contain finite values" if (side == "key" and promote > 0) else \
        "quantize expects all values to be finite"
    held = [t.clone() for t in cache.get()]
    with pytest.raises(ValueError, match=msg):
        cache.update(bad_keys, bad_values)
    assert cache.get_seq_length() == 20
    assert [(s.sequence_start, s.token_count) for s in cache.page_metadata()] == before
    # the held tail lives in buffers the failed append overwrote: its tokens are back, bit for bit
    assert all(torch.equal(a, b) for a, b in zip(cache.get(), held))
    cache.update(keys[..., 20:, :], values[..., 20:, :])
    assert cache.get_seq_length() == 40
    k, v = cache.get()
    assert bool(torch.isfinite(k).all()) and bool(torch.isfinite(v).all())


@gpu
@pytest.mark.parametrize("first", [True, False])
def test_failed_append_leaves_sink_tail_and_device_count_as_they_were(first):
    """A non-finite token in a page an append seals: the append raises and the cache is as before it,
    including the dense sink tokens of that append (copied after the quantize launches), the held tail
    and the device-side tail count; the same cache then takes the finite tokens and ends up bit for
    bit like a cache that never saw the bad append."""
    cfg = DartKVCacheConfig(bits=2, page_size=16, key_group_size=16, value_group_size=4, promote_ratio=0.25,
                            sink_tokens=3, hold_partial_pages=True, metadata_dtype=torch.float16)
    torch.manual_seed(4)
    keys = torch.randn(2, 2, 70, 32, device=DEV, dtype=torch.bfloat16)
    values = torch.randn_like(keys)
    cache, clean = DartKVCache(cfg), DartKVCache(cfg)
    start = 0 if first else 25
    for c in (cache, clean):
        if start:
            c.update(keys[..., :start, :], values[..., :start, :])
    if not first:
        cache.enable_device_tail()
        clean.enable_device_tail()
    before = [t.clone() for t in cache.get()] if start else None
    bad = keys[..., start:, :].clone()
    bad[0, 1, 20, 5] = float("nan")
    with pytest.raises(ValueError, match="finite"):
        cache.update(bad, values[..., start:, :])
    assert cache.get_seq_length() == start
    if first:
        assert cache.iter_segments() == [] and cache.page_metadata() == []
    else:
        assert all(torch.equal(a, b) for a, b in zip(cache.get(), before))
        assert int(cache.device_tail.item()) == (start - 3) % 16
    for c in (cache, clean):
        c.update(keys[..., start:, :], values[..., start:, :])
    assert cache.get_seq_length() == clean.get_seq_length() == 70
    assert all(torch.equal(a, b) for a, b in zip(cache.get(), clean.get()))
    if not first:
        assert int(cache.device_tail.item()) == int(clean.device_tail.item())


@gpu
def test_failed_kitty_append_restores_the_key_page_packed_again_in_its_slot():
    """Kitty key window (local_tokens 1) after a prefill that ends on a page boundary: the next one-token
    append packs the last key page again, from its dequantized values, into the same pool slot.  When a
    value packed later in that append is non-finite (a NaN in the value window), the append raises and
    the slot must hold its first packing again: packing dequantized 16-bit values twice is not
    idempotent, so a retry from the second packing would drift from the reference."""
    cfg = DartKVCacheConfig(bits=2, page_size=16, key_group_size=16, value_group_size=4, promote_ratio=0.25,
                            local_tokens=1, value_local_tokens=4, metadata_dtype=torch.float16)
    torch.manual_seed(11)
    keys = torch.randn(2, 2, 33, 32, device=DEV, dtype=torch.bfloat16) * 3.1
    values = torch.randn_like(keys)
    values[1, 0, 28, 7] = float("nan")  # token 28: in the value window after the prefill, packed next
    cache, clean = DartKVCache(cfg), DartKVCache(cfg)
    for c in (cache, clean):
        c.update(keys[..., :32, :], values[..., :32, :])
    with pytest.raises(ValueError, match="finite"):
        cache.update(keys[..., 32:33, :], values[..., 32:33, :])
    assert cache.get_seq_length() == clean.get_seq_length() == 32

    def packed(c):
        out = []
        for seg in c._keys:
            if isinstance(seg, torch.Tensor):
                out.append(seg)
            else:
                names = ("low_values", "high_values", "channel_indices", "scale", "zero_point", "values")
                out += [getattr(seg, f) for f in names if isinstance(getattr(seg, f, None), torch.Tensor)]
        return out

    from tests.golden_util import bits_equal
    # the premise: packing the last page again from its dequantized values changes its bytes, so a
    # slot left holding the second packing would show below
    last = clean._keys[-1]
    again = dart.quantize_key_mixed(last.dequantize(), group_size=16, promote_ratio=0.25,
                                    metadata_dtype=torch.float16)
    assert not all(torch.equal(x, y) for x, y in zip(
        (again.low_values, again.high_values, again.channel_indices, again.scale, again.zero_point),
        (last.low_values, last.high_values, last.channel_indices, last.scale, last.zero_point)))
    a, b = packed(cache), packed(clean)
    assert len(a) == len(b) and len(a) > 0
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    # the NaN token is still in both value windows: compare bits
    assert all(bits_equal(x.cpu(), y.cpu()) for x, y in zip(cache.get(), clean.get()))


@gpu
def test_cache_filled_under_inference_mode_takes_later_calls_outside_it():
    """A cache whose storage (pools, held tail, device tail count, dense sink) was created by appends
    under ``torch.inference_mode()`` (a model's prefill) takes later appends, a failed append's restore,
    device tail counts and batch reordering outside that mode: its storage is made of normal tensors."""
    cfg = DartKVCacheConfig(bits=2, page_size=16, key_group_size=16, value_group_size=4, promote_ratio=0.25,
                            sink_tokens=3, hold_partial_pages=True, metadata_dtype=torch.float16)
    torch.manual_seed(21)
    keys = torch.randn(2, 2, 90, 32, device=DEV, dtype=torch.bfloat16)
    values = torch.randn_like(keys)
    cache, clean = DartKVCache(cfg), DartKVCache(cfg)
    with torch.inference_mode():
        cache.update(keys[..., :40, :], values[..., :40, :])
    clean.update(keys[..., :40, :], values[..., :40, :])
    bad = keys[..., 40:70, :].clone()
    bad[1, 0, 3, 9] = float("inf")
    with pytest.raises(ValueError, match="finite"):
        cache.update(bad, values[..., 40:70, :])
    for c in (cache, clean):
        c.update(keys[..., 40:70, :], values[..., 40:70, :])
        c.enable_device_tail()
        c.update(keys[..., 70:71, :], values[..., 70:71, :])
        c.reorder_batch(torch.tensor([1, 0], device=DEV))
        c.update(keys[..., 71:, :].flip(0).contiguous(), values[..., 71:, :].flip(0).contiguous())
    assert cache.get_seq_length() == clean.get_seq_length() == 90
    assert all(torch.equal(a, b) for a, b in zip(cache.get(), clean.get()))


@gpu
def test_non_finite_token_in_the_held_tail_is_kept_like_the_reference():
    """The reference checks only tokens it quantizes: a NaN that stays in the dense held tail raises
    nothing until a later append seals its page."""
    cfg = DartKVCacheConfig(bits=2, page_size=16, key_group_size=16, value_group_size=4, promote_ratio=0.25,
                            hold_partial_pages=True, metadata_dtype=torch.float16)
    keys = torch.randn(1, 2, 20, 16, device=DEV)
    keys[0, 1, 18, 2] = float("nan")
    cache = DartKVCache(cfg)
    cache.update(keys, keys)  # tokens 16..19 stay dense
    assert cache.get_seq_length() == 20
    with pytest.raises(ValueError, match="finite"):
        cache.update(torch.randn(1, 2, 12, 16, device=DEV), torch.randn(1, 2, 12, 16, device=DEV))
    assert cache.get_seq_length() == 20


@gpu
def test_dense_attention_matches_the_golden_dense_output(golden):
    """reference attention.py:14-29 on the materialized golden lifecycles: dense_attention over this
    build's materialized cache equals the reference's stored output within one ulp of its dtype."""
    from tests.test_oracle_golden import _lifecycle_inputs
    from tests.test_gpu_parity import _config
    for e in golden.manifest["cache"]:
        keys, values, query = _lifecycle_inputs(golden, e)
        cache = DartKVCache(_config(e["config"]))
        start = 0
        for n in e["updates"]:
            cache.update(keys[..., start:start + n, :].to(DEV), values[..., start:start + n, :].to(DEV))
            start += n
        mk, mv = cache.get()
        g = e["Hq"] // e["Hkv"]
        out = dart.dense_attention(query.to(DEV), mk.repeat_interleave(g, dim=1), mv.repeat_interleave(g, dim=1))
        ref = golden.get(e["dense_attn"])
        assert out.dtype == ref.dtype and out.shape == ref.shape
        # float64 caches: attention computes in fp32 (attention.py:28-29), so fp32's ulp
        ulp = {torch.float64: 2e-6, torch.float32: 2e-6, torch.float16: 1e-3, torch.bfloat16: 8e-3}[ref.dtype]
        tol = ulp * float(ref.float().abs().max())
        err = float((out.float().cpu() - ref.float()).abs().max())
        print("dense_attention", e["name"], err, tol, flush=True)
        assert err <= tol, (e["name"], err, tol)


@gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_random_strategy_given_channels_match_the_oracle(dtype):
    """The "random" strategy with the channels given (reference mixed.py:145-153 draws them with
    randperm per KV head): codes, high rows in the given slot order, scales and zero points equal the
    oracle fed the same channels; a cache whose pages draw them itself promotes exactly its stored set."""
    from oracle import dart_oracle as O
    from tests.golden_util import bits_equal
    g = torch.Generator().manual_seed(31)
    keys = (torch.randn(3, 4, 100, 64, generator=g) * 3).to(dtype)
    chans = torch.stack([torch.randperm(64, generator=g)[:16] for _ in range(4)])
    mk = dart.quantize_key_mixed(keys.to(DEV), group_size=32, promote_ratio=0.25, strategy="random",
                                 metadata_dtype=torch.float16, channel_indices=chans.to(DEV))
    ok = O.quantize_key_mixed(keys, group_size=32, promote_ratio=0.25, strategy="random",
                              metadata_dtype=torch.float16, random_indices=chans)
    for a, b in ((mk.low_values, ok.low_values), (mk.high_values, ok.high_values),
                 (mk.channel_indices, ok.channel_indices), (mk.scale, ok.scale), (mk.zero_point, ok.zero_point)):
        assert bits_equal(a.cpu(), b)
    assert bits_equal(mk.dequantize().cpu(), ok.dequantize())
    cache = DartKVCache(DartKVCacheConfig(bits=2, page_size=32, key_group_size=32, value_group_size=16,
                                          promote_ratio=0.25, channel_selection="random",
                                          metadata_dtype=torch.float16))
    cache.update(keys.to(DEV), keys.to(DEV))
    kseg = cache.iter_segments()[0][0]
    idx = kseg.channel_indices.cpu()
    assert idx.shape == (3, 4, 16)
    assert torch.equal(idx[0], idx[1]) and torch.equal(idx[0], idx[2])  # one draw per KV head, shared by the batch
    assert all(len(set(row.tolist())) == 16 for row in idx[0])
    ref = O.quantize_key_mixed(keys[..., :32, :], group_size=32, promote_ratio=0.25, strategy="random",
                               metadata_dtype=torch.float16, random_indices=idx[0])
    for a, b in ((kseg.low_values, ref.low_values), (kseg.high_values, ref.high_values), (kseg.scale, ref.scale),
                 (kseg.zero_point, ref.zero_point)):
        assert bits_equal(a.cpu(), b)

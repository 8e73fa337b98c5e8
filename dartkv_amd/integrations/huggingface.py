"""Transformers ``Cache`` facade over HIP-packed Dart layers.

Mirrors reference src/dart/integrations/huggingface.py:19-147 (``DartHFCache``):
same constructor, ``update`` lifecycle, accessors and properties.  The
installed Transformers (5.x) builds a ``Cache`` from a list of per-layer
objects and asks those layers for sequence length and mask sizes, so every
Dart layer here is a ``DartCacheLayer`` (a ``CacheLayerMixin``) that owns one
``DartKVCache``.  The reference's ``_layers`` mapping (layer index ->
``DartKVCache``) is kept as a view for callers that use it.

Update lifecycle (reference huggingface.py:39-69, Kitty's PostQuant timing):

* layer 0 counts every token into ``_seen_tokens``;
* the first update of a layer is the prefill: it returns clones of the new
  key/value states, then packs them;
* later updates return ``cat(materialized cache, new)`` -- the state before
  this call's tokens are packed -- or, when ``cache_kwargs`` carries
  ``dart_fused_attention``, only clones of the new tokens, because the fused
  decode reads the packed pages itself;
* the new tokens are appended to the packed store after the return values are
  taken.
"""

from __future__ import annotations

from typing import Dict, Optional

import torch

from ..cache import DartKVCache, DartKVCacheConfig

try:
    from transformers import Cache
    from transformers.cache_utils import CacheLayerMixin
except ImportError as exc:  # pragma: no cover - only without the optional dependency
    raise ImportError("DartHFCache requires transformers; install the DartKV model dependencies first.") from exc


class DartCacheLayer(CacheLayerMixin):
    """One decoder layer's packed cache, in Transformers' per-layer interface."""

    is_sliding = False
    is_compileable = False

    def __init__(self, config: DartKVCacheConfig, requantize_on_reorder: bool = False) -> None:
        super().__init__()
        self.dart_config = config
        self.requantize_on_reorder = requantize_on_reorder
        self.cache = DartKVCache(config)
        self.last_update_prefill = False

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        self.dtype, self.device = key_states.dtype, key_states.device
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, cache_kwargs: Optional[dict] = None,
               *args, **kwargs) -> tuple[torch.Tensor, torch.Tensor]:
        """Reference huggingface.py:46-69 for one layer."""
        fused_update = bool(cache_kwargs and cache_kwargs.get("dart_fused_attention"))
        prefill = not self.is_initialized
        if prefill or fused_update:
            keys_out = key_states.detach().clone()
            values_out = value_states.detach().clone()
        else:
            prior_keys, prior_values = self.cache.get()
            keys_out = torch.cat((prior_keys, key_states), dim=-2)
            values_out = torch.cat((prior_values, value_states), dim=-2)
        self.cache.append(key_states, value_states)
        if prefill:
            self.lazy_initialization(key_states, value_states)
        self.last_update_prefill = prefill
        return keys_out, values_out

    def get_seq_length(self) -> int:
        return self.cache.get_seq_length()

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.get_seq_length() + query_length, 0

    def get_max_length(self) -> int:
        return -1

    def reset(self) -> None:
        self.cache.clear()
        self.is_initialized = False
        self.last_update_prefill = False

    # Batch reordering gathers the packed bytes along the batch axis (DartKVCache.reorder_batch).  With
    # requantize_on_reorder the layer is rebuilt as the reference rebuilds it (huggingface.py:117-127): a
    # fresh cache appends the selected rows of the materialized contents, so they are quantized again and
    # the page lifecycle restarts from one prefill.
    def _reorder(self, rows: torch.Tensor) -> None:
        if not self.requantize_on_reorder:
            self.cache.reorder_batch(rows)
            return
        if self.cache.shape is None:
            return
        keys, values = self.cache.get()
        index = rows.to(keys.device)
        if index.dtype == torch.bool:
            index = index.nonzero().flatten()
        rebuilt = DartKVCache(self.dart_config)
        rebuilt.append(keys.index_select(0, index), values.index_select(0, index))
        self.cache = rebuilt

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        self._reorder(torch.as_tensor(beam_idx))

    def batch_repeat_interleave(self, repeats: int) -> None:
        if self.cache.shape is not None:
            rows = torch.arange(self.cache.shape[0], device=self.cache.device)
            self._reorder(rows.repeat_interleave(repeats))

    def batch_select_indices(self, indices: torch.Tensor) -> None:
        if self.cache.shape is not None:
            rows = torch.arange(self.cache.shape[0], device=self.cache.device)
            self._reorder(rows[indices.to(rows.device) if isinstance(indices, torch.Tensor) else indices])

    def crop(self, tokens_to_remove: int) -> None:
        raise NotImplementedError("DartHFCache pages are append-only; crop is not supported")


class DartHFCache(Cache):
    """A standard Transformers cache facade backed by compressed Dart layers.

    ``update`` returns dense tensors for the standard eager/SDPA attention
    path; the Qwen3 adapter (``attach_dart_fused_attention``) reads the packed
    pages directly for one-token decode.
    """

    is_compileable = False

    def __init__(self, config: Optional[DartKVCacheConfig] = None, *, requantize_on_reorder: bool = False) -> None:
        """``requantize_on_reorder``: beam reordering and batch selection rebuild each layer from its
        materialized rows, quantized again, exactly as the reference does (huggingface.py:117-127);
        by default they gather the packed bytes instead (no second quantization, no pass over the cache)."""
        super().__init__(layers=[])
        self.dart_config = config or DartKVCacheConfig()
        self.requantize_on_reorder = requantize_on_reorder
        self._seen_tokens = 0
        self.graph_epoch = 0  # bumps when batch rows move: captured decode graphs must be captured again

    # ---- lifecycle ----
    def _layer(self, layer_idx: int) -> DartCacheLayer:
        while len(self.layers) <= layer_idx:
            self.layers.append(DartCacheLayer(self.dart_config, self.requantize_on_reorder))
        return self.layers[layer_idx]

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs: Optional[dict] = None, *args, **kwargs) -> tuple[torch.Tensor, torch.Tensor]:
        out = self._layer(layer_idx).update(key_states, value_states, cache_kwargs)
        if layer_idx == 0:
            self._seen_tokens += key_states.shape[-2]
        return out

    @property
    def _layers(self) -> Dict[int, DartKVCache]:
        """Initialized layers by index, as the reference stores them."""
        return {i: layer.cache for i, layer in enumerate(self.layers) if layer.is_initialized}

    def layer_for_attention(self, layer_idx: int) -> DartKVCache:
        """Return a layer's packed cache for fused attention integration."""
        if layer_idx >= len(self.layers) or not self.layers[layer_idx].is_initialized:
            raise RuntimeError(f"layer {layer_idx} has not been initialized")
        return self.layers[layer_idx].cache

    def last_update_was_prefill(self, layer_idx: int) -> bool:
        """Whether the most recent update for ``layer_idx`` created the layer."""
        if layer_idx >= len(self.layers):
            return False
        return self.layers[layer_idx].last_update_prefill

    def get_seq_length(self, layer_idx: Optional[int] = 0) -> int:
        if layer_idx is None:
            layer_idx = 0
        if layer_idx >= len(self.layers):
            return 0
        return self.layers[layer_idx].get_seq_length()

    def get_max_cache_shape(self, layer_idx: int = 0) -> None:
        return None

    def get_max_length(self, layer_idx: Optional[int] = None) -> int:
        return -1

    # ---- replayable decode steps ----
    def enable_graph_decode(self) -> None:
        """Keep every layer's held-tail length on the device (``DartKVCache.enable_device_tail``).

        A one-token decode step through the fused adapter then launches the
        same kernels with the same arguments every step, so it can be captured
        in a HIP graph and replayed; call ``advance_graph_step`` once per
        replay after the first one (capturing runs the host-side bookkeeping of
        one step).  A step whose append would seal a page
        (``graph_step_seals``) must run eagerly, and the graph be captured
        again after it.
        """
        for layer in self.layers:
            if layer.is_initialized:
                layer.cache.enable_device_tail()

    def graph_decode_ready(self) -> bool:
        """Whether every layer keeps its held-tail length on the device (``enable_graph_decode``)."""
        return bool(self.layers) and all(layer.is_initialized and layer.cache.device_tail is not None
                                         for layer in self.layers)

    def prepared_append_ok(self, layer_idx: int) -> bool:
        """Whether layer ``layer_idx`` can take its next token from the decode-step preparation kernel."""
        return (layer_idx < len(self.layers) and self.layers[layer_idx].is_initialized
                and self.layers[layer_idx].cache.prepared_append_ok())

    def commit_prepared_append(self, layer_idx: int) -> None:
        """The update bookkeeping (reference huggingface.py:46-68) of a token written by the
        preparation kernel into layer ``layer_idx``'s tail."""
        layer = self.layers[layer_idx]
        layer.cache.commit_prepared_append()
        layer.last_update_prefill = False
        if layer_idx == 0:
            self._seen_tokens += 1

    def graph_step_seals(self) -> bool:
        """Whether the next one-token step would seal a page in any layer."""
        return any(layer.cache.next_append_seals(1) for layer in self.layers if layer.is_initialized)

    def advance_graph_step(self, steps: int = 1) -> None:
        """Host-side bookkeeping of ``steps`` replayed one-token decode steps."""
        for layer in self.layers:
            layer.cache.advance_device_tail(steps)
        self._seen_tokens += steps

    # ---- descriptors ----
    def page_table(self, layer_idx: int = 0, *, device: torch.device | str | None = None, rebuild: bool = False):
        """Expose a layer's cached Dart page table to fused attention callers."""
        layer = self._layers.get(layer_idx)
        return layer.page_table(device=device, rebuild=rebuild) if layer is not None else None

    def page_runs(self, layer_idx: int = 0, *, device: torch.device | str | None = None, rebuild: bool = False):
        """Expose a layer's cached uniform page runs."""
        layer = self._layers.get(layer_idx)
        return layer.page_runs(device=device, rebuild=rebuild) if layer is not None else None

    def reorder_cache(self, beam_idx: torch.LongTensor) -> "DartHFCache":
        """Reorder the beams of every layer: packed pages keep their bytes, or, with
        ``requantize_on_reorder``, every layer is rebuilt from its selected materialized rows."""
        for layer in self.layers:
            layer.reorder_cache(beam_idx)
            layer.last_update_prefill = False
        self.graph_epoch += 1
        return self

    def batch_repeat_interleave(self, repeats: int) -> None:
        super().batch_repeat_interleave(repeats)
        self.graph_epoch += 1

    def batch_select_indices(self, indices: torch.Tensor) -> None:
        super().batch_select_indices(indices)
        self.graph_epoch += 1

    # ---- dense views and accounting ----
    @property
    def key_cache(self) -> list[torch.Tensor]:
        return [layer.key_states for _, layer in sorted(self._layers.items())]

    @property
    def value_cache(self) -> list[torch.Tensor]:
        return [layer.value_states for _, layer in sorted(self._layers.items())]

    @property
    def storage_bytes(self) -> int:
        return sum(layer.storage_bytes for layer in self._layers.values())

    @property
    def dense_bytes(self) -> int:
        return sum(layer.dense_bytes for layer in self._layers.values())

    @property
    def compression_ratio(self) -> float:
        return self.dense_bytes / self.storage_bytes if self.storage_bytes else 1.0


__all__ = ["DartCacheLayer", "DartHFCache"]

"""The HIP entry points as PyTorch operators: ``torch.ops.dartkv.*``.

Registered with ``torch.library.custom_op``, each operator is one dispatcher
node: ``torch.compile`` keeps it whole instead of tracing into ctypes, its
fake implementation gives output shapes and dtypes without touching the GPU
(meta and fake tensors), and ``torch.library.opcheck`` can test it.  Each one
runs the same C ABI call as the Python API beside it
(``quantization.quantize``, ``QuantizedTensor.dequantize``,
``mixed.quantize_key_mixed``, ``MixedQuantizedKey.dequantize``,
``attention.decode_attention``); there is no second implementation.

``decode_attention`` reads a ``DartKVCache``, which is not a tensor: the
operator takes an integer handle from ``cache_handle(cache)``, valid while the
cache lives.  The cache's packed pages are not operator inputs, so a compiled
graph must not move the operator across appends to that cache; appends run
Python control flow, which ends a compiled region anyway.
"""

from __future__ import annotations

import itertools
import weakref
from typing import Optional, Tuple

import torch

from . import attention as _attention
from . import mixed as _mixed
from . import quantization as _quantization
from .cache import DartKVCache

Tensor = torch.Tensor

_caches: "weakref.WeakValueDictionary[int, DartKVCache]" = weakref.WeakValueDictionary()
_handles: "weakref.WeakKeyDictionary[DartKVCache, int]" = weakref.WeakKeyDictionary()
_next_handle = itertools.count(1)


def cache_handle(cache: DartKVCache) -> int:
    """Integer naming ``cache`` for ``torch.ops.dartkv.decode_attention`` (valid while it lives).  Handles
    come from a counter and are never reused, so a graph that keeps the handle of a cache that has since
    been freed gets 'unknown handle' rather than another cache."""
    if not isinstance(cache, DartKVCache):
        raise TypeError("cache_handle expects a DartKVCache")
    handle = _handles.get(cache)
    if handle is None:
        handle = _handles[cache] = next(_next_handle)
        _caches[handle] = cache
    return handle


def _cache(handle: int) -> DartKVCache:
    cache = _caches.get(handle)
    if cache is None:
        raise ValueError("unknown DartKVCache handle; get one from dartkv_amd.torch_ops.cache_handle(cache)")
    return cache


def _row_layout(n: int, bits: int, group_size: int) -> Tuple[int, int]:
    """(groups, packed bytes) of one quantized row of n elements."""
    groups = -(-n // group_size)
    per_byte = 8 // bits
    packed = -(-groups * group_size // per_byte)
    return groups, packed


def _meta(data: Tensor, meta_dtype: Optional[torch.dtype]) -> torch.dtype:
    return _quantization._metadata_dtype(data, meta_dtype)


# ---- uniform rows (reference quantization.py:134-204) ----

@torch.library.custom_op("dartkv::quantize_rows", mutates_args=())
def quantize_rows(data: Tensor, bits: int, group_size: int,
                  meta_dtype: Optional[torch.dtype] = None) -> Tuple[Tensor, Tensor, Tensor]:
    """Codes [..., packed], scale and zero point [..., groups] of ``data`` quantized along its last dim."""
    q = _quantization.quantize(data, bits=bits, group_size=group_size, metadata_dtype=meta_dtype)
    return q.values, q.scale, q.zero_point


@quantize_rows.register_fake
def _(data, bits, group_size, meta_dtype=None):
    groups, packed = _row_layout(data.shape[-1], bits, group_size)
    meta = _meta(data, meta_dtype)
    outer = tuple(data.shape[:-1])
    return (data.new_empty(outer + (packed,), dtype=torch.uint8), data.new_empty(outer + (groups,), dtype=meta),
            data.new_empty(outer + (groups,), dtype=meta))


@torch.library.custom_op("dartkv::dequantize_rows", mutates_args=())
def dequantize_rows(values: Tensor, scale: Tensor, zero_point: Tensor, bits: int, group_size: int, n: int,
                    dtype: torch.dtype) -> Tensor:
    """Rows of ``quantize_rows`` back to [..., n] in ``dtype`` with the reference's rounding chain."""
    groups = scale.shape[-1]
    per_byte = 8 // bits
    q = _quantization.QuantizedTensor(
        values=values, scale=scale, zero_point=zero_point, original_shape=tuple(scale.shape[:-1]) + (n,),
        original_dim=n, padded_dim=groups * group_size, packed_dim=values.shape[-1] * per_byte,
        group_size=group_size, bits=bits, output_dtype=dtype, axis=scale.ndim - 1)
    return q.dequantize(dtype=dtype)


@dequantize_rows.register_fake
def _(values, scale, zero_point, bits, group_size, n, dtype):
    return scale.new_empty(tuple(scale.shape[:-1]) + (n,), dtype=dtype)


# ---- Dart keys (reference mixed.py:119-244) ----

@torch.library.custom_op("dartkv::quantize_key_mixed", mutates_args=())
def quantize_key_mixed(key_states: Tensor, group_size: int, promote_ratio: float, strategy: str,
                       meta_dtype: Optional[torch.dtype] = None,
                       channel_indices: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(low codes, high codes, channel indices, scale, zero point) of a key chunk [B, H, T, D]."""
    k = _mixed.quantize_key_mixed(key_states, group_size=group_size, promote_ratio=promote_ratio, strategy=strategy,
                                  metadata_dtype=meta_dtype, channel_indices=channel_indices)
    return k.low_values, k.high_values, k.channel_indices, k.scale, k.zero_point


@quantize_key_mixed.register_fake
def _(key_states, group_size, promote_ratio, strategy, meta_dtype=None, channel_indices=None):
    B, H, T, D = key_states.shape
    K = _mixed.promoted_count(D, promote_ratio)
    G = -(-T // group_size)
    nb = (group_size + 3) // 4
    meta = meta_dtype or (key_states.dtype if key_states.dtype in (torch.float16, torch.bfloat16) else torch.float32)
    u8 = torch.uint8
    return (key_states.new_empty((B, H, D, G, nb), dtype=u8), key_states.new_empty((B, H, K, G, nb if K else nb * 4),
                                                                                    dtype=u8),
            key_states.new_empty((B, H, K), dtype=torch.int32), key_states.new_empty((B, H, D, G), dtype=meta),
            key_states.new_empty((B, H, D, G), dtype=meta))


@torch.library.custom_op("dartkv::dequantize_key_mixed", mutates_args=())
def dequantize_key_mixed(low: Tensor, high: Tensor, channel_indices: Tensor, scale: Tensor, zero_point: Tensor,
                         tokens: int, group_size: int, dtype: torch.dtype) -> Tensor:
    """Keys [B, H, tokens, D] in ``dtype`` from the fields of ``quantize_key_mixed``."""
    B, H, D, G = scale.shape
    k = _mixed.MixedQuantizedKey(low_values=low, high_values=high, channel_indices=channel_indices, scale=scale,
                                 zero_point=zero_point, original_shape=(B, H, tokens, D), padded_tokens=G * group_size,
                                 group_size=group_size, low_bits=2, promote_bits=4, output_dtype=dtype)
    return k.dequantize(dtype=dtype)


@dequantize_key_mixed.register_fake
def _(low, high, channel_indices, scale, zero_point, tokens, group_size, dtype):
    B, H, D, _ = scale.shape
    return scale.new_empty((B, H, tokens, D), dtype=dtype)


# ---- decode (reference fused_attention.py:654-771, attention.py:32-87 for one token) ----

@torch.library.custom_op("dartkv::decode_attention", mutates_args=())
def decode_attention(query: Tensor, cache: int, scale: Optional[float] = None) -> Tensor:
    """One-token attention [B, Hq, 1, D] of ``query`` over the packed cache named by ``cache``."""
    return _attention.decode_attention(query, _cache(cache), scale=scale)


@decode_attention.register_fake
def _(query, cache, scale=None):
    B, Hq, D = query.shape[0], query.shape[1], query.shape[-1]
    return query.new_empty((B, Hq, 1, D))


__all__ = ["cache_handle", "decode_attention", "dequantize_key_mixed", "dequantize_rows", "quantize_key_mixed",
           "quantize_rows"]

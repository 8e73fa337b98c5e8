"""Single-token packed-page decode attention (reference src/dart/fused_attention.py:654-771).

``fused_dart_attention`` keeps the reference signature, checks and messages.
It runs one split-K HIP kernel plus a merge pass over every segment of the
cache (sink, pages, held tail); ``page_table``/``page_runs`` are validated
against the cache exactly as the reference does and describe the same pages.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch

from .attention import MAX_GROUP, MAX_HEAD_DIM, decode_attention, segment_attention, streamed_dart_attention
from .cache import DartKVCache
from .page_table import DartPageRun, DartPageTable


def fused_dart_attention(
    query: torch.Tensor,
    cache: DartKVCache,
    *,
    scale: Optional[float] = None,
    fallback: bool = True,
    page_table: Optional[DartPageTable] = None,
    page_runs: Optional[Sequence[DartPageRun]] = None,
) -> torch.Tensor:
    """Attention of one query token per head over the packed cache -> [B, Hq, 1, D]."""
    if query.ndim != 4:
        raise ValueError("query must have shape [B, Hq, 1, D]")
    if query.shape[-2] != 1:
        if fallback:
            return streamed_dart_attention(query, cache, scale=scale)
        raise ValueError("fused_dart_attention currently supports one query token")
    if query.device.type != "cuda":
        raise RuntimeError("fused_dart_attention requires a ROCm device (dartkv_amd has no CPU path)")
    cache_shape = cache.shape
    if cache_shape is None or cache_shape[2] == 0:
        raise ValueError("cache is empty")
    batch, kv_heads, _, head_dim = cache_shape
    if query.shape[0] != batch or query.shape[-1] != head_dim:
        raise ValueError("query batch and head_dim must match the cache")
    if query.shape[1] % kv_heads:
        raise ValueError("query heads must be divisible by cache KV heads")
    if page_table is not None or page_runs is not None:
        _validate_descriptors(query, cache, page_table, page_runs)
    if query.shape[1] // kv_heads > MAX_GROUP or head_dim > MAX_HEAD_DIM:
        if not fallback:
            raise ValueError(f"the HIP decode kernels take at most {MAX_GROUP} query heads per KV head and "
                             f"head_dim {MAX_HEAD_DIM}")
        return segment_attention(query, cache, scale=scale)
    return decode_attention(query, cache, scale=scale)


def _validate_descriptors(query, cache, page_table, page_runs) -> None:
    """The reference's descriptor checks (fused_attention.py:262-292)."""
    segments = cache.iter_segments()
    table = page_table if page_table is not None else cache.page_table(device=query.device)
    if table.device != query.device:
        table = table.to(query.device)
    if table.page_count != len(segments) or table.seen_tokens != cache.seen_tokens:
        raise ValueError("page_table does not describe the current cache segments")
    if page_runs is None:
        runs = tuple(table.uniform_quantized_runs(cache)) if page_table is not None else cache.page_runs(device=query.device)
    else:
        runs = tuple(page_runs)
    starts = set()
    for run in runs:
        run.validate()
        if run.first_page_index in starts:
            raise ValueError("page_runs contain duplicate first_page_index")
        stop = run.first_page_index + run.page_count
        if run.first_page_index < 0 or stop > len(segments):
            raise ValueError("page_run is outside the current cache page range")
        expected = table.page_ids[0, run.first_page_index:stop].to(run.page_indices.device)
        if not torch.equal(expected, run.page_indices):
            raise ValueError("page_run logical IDs do not match page_table")
        if bool((table.key_modes[run.first_page_index:stop] != 1).any()) or bool(
                (table.value_modes[run.first_page_index:stop] != 1).any()):
            raise ValueError("page_runs may only contain uniform quantized pages")
        starts.add(run.first_page_index)
    for index, (kseg, _) in enumerate(segments):
        tokens = kseg.shape[-2] if isinstance(kseg, torch.Tensor) else kseg.original_shape[-2]
        if int(table.token_counts[index]) != tokens:
            raise ValueError(f"page_table token count mismatch at page {index}")


__all__ = ["fused_dart_attention"]

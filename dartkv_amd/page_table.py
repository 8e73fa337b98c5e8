"""Page descriptors for DartKV cache segments (reference src/dart/page_table.py:1-401).

``DartPageTable`` and ``DartPageRun`` keep the reference's fields, validation
order and messages.  They describe the cache for callers that inspect or
reorder pages; the decode kernel itself reads the cache's device segment table
(``DartKVCache.decode_plan``), so building these objects is never on the decode
hot path.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import TYPE_CHECKING, Sequence

import torch

from .mixed import MixedQuantizedKey
from .quantization import QuantizedTensor

if TYPE_CHECKING:
    from .cache import DartKVCache

DENSE_PAGE = 0
QUANTIZED_PAGE = 1
MIXED_PAGE = 2
_VALID_PAGE_MODES = (DENSE_PAGE, QUANTIZED_PAGE, MIXED_PAGE)


def _tokens(seg) -> int:
    return seg.shape[-2] if isinstance(seg, torch.Tensor) else seg.original_shape[-2]


def _mode(seg) -> int:
    if isinstance(seg, torch.Tensor):
        return DENSE_PAGE
    return MIXED_PAGE if isinstance(seg, MixedQuantizedKey) else QUANTIZED_PAGE


@dataclass(frozen=True)
class DartPageTable:
    """Batch-indexed page descriptors on one device (reference page_table.py:30-48).

    ``page_ids`` [B, N] maps each batch row to the segment index in
    ``cache.iter_segments()``; the other arrays are page-major.
    """

    page_ids: torch.Tensor
    sequence_starts: torch.Tensor
    token_counts: torch.Tensor
    key_modes: torch.Tensor
    value_modes: torch.Tensor
    valid: torch.Tensor
    seen_tokens: int
    page_size: int

    @classmethod
    def from_cache(cls, cache: "DartKVCache", *, device=None) -> "DartPageTable":
        """reference page_table.py:50-87."""
        shape = cache.shape
        batch = shape[0] if shape is not None else 0
        segments = cache.iter_segments()
        starts, counts, kmodes, vmodes = [], [], [], []
        start = 0
        for kseg, vseg in segments:
            kt, vt = _tokens(kseg), _tokens(vseg)
            if kt != vt:
                raise RuntimeError("DartKVCache key/value page lengths diverged")
            starts.append(start)
            counts.append(kt)
            kmodes.append(_mode(kseg))
            vmodes.append(_mode(vseg))
            start += kt
        if start != cache.seen_tokens:
            raise RuntimeError(f"page table covers {start} tokens, expected {cache.seen_tokens}")
        target = torch.device(device) if device is not None else (cache.device or torch.device("cpu"))
        n = len(segments)
        ids = torch.arange(n, dtype=torch.int64, device=target).unsqueeze(0).expand(batch, -1).contiguous()
        return cls(
            page_ids=ids,
            sequence_starts=torch.tensor(starts, dtype=torch.int32, device=target),
            token_counts=torch.tensor(counts, dtype=torch.int32, device=target),
            key_modes=torch.tensor(kmodes, dtype=torch.int8, device=target),
            value_modes=torch.tensor(vmodes, dtype=torch.int8, device=target),
            valid=torch.ones((batch, n), dtype=torch.bool, device=target),
            seen_tokens=cache.seen_tokens,
            page_size=cache.config.page_size,
        )

    @property
    def batch_size(self) -> int:
        return self.page_ids.shape[0]

    @property
    def page_count(self) -> int:
        return self.page_ids.shape[1]

    @property
    def device(self) -> torch.device:
        return self.page_ids.device

    def __len__(self) -> int:
        return self.page_count

    def validate(self) -> "DartPageTable":
        """Shape, mode, id, order and total-length invariants (reference page_table.py:104-141)."""
        n = self.page_count
        if self.page_ids.ndim != 2 or self.valid.shape != self.page_ids.shape:
            raise ValueError("page_ids and valid must have shape [batch, page_count]")
        for name, t in (("sequence_starts", self.sequence_starts), ("token_counts", self.token_counts),
                        ("key_modes", self.key_modes), ("value_modes", self.value_modes)):
            if t.ndim != 1 or t.shape[0] != n:
                raise ValueError(f"{name} must have shape [page_count]")
        if self.page_size <= 0 or self.seen_tokens < 0:
            raise ValueError("page_size and seen_tokens must be non-negative/positive")
        if n:
            counts = self.token_counts.to("cpu", torch.int64)
            starts = self.sequence_starts.to("cpu", torch.int64)
            expected = torch.cumsum(torch.cat((torch.zeros(1, dtype=torch.int64), counts[:-1])), dim=0)
            if not torch.equal(starts, expected):
                raise ValueError("sequence_starts are not contiguous")
            if bool((counts <= 0).any()):
                raise ValueError("token_counts must be positive")
            if int(counts.sum()) != self.seen_tokens:
                raise ValueError("token_counts do not cover seen_tokens")
            modes = torch.tensor(_VALID_PAGE_MODES)
            if bool((~(self.key_modes.cpu().long()[:, None] == modes).any(dim=-1)).any()):
                raise ValueError("key_modes contain an unsupported mode")
            if bool((~(self.value_modes.cpu().long()[:, None] == modes).any(dim=-1)).any()):
                raise ValueError("value_modes contain an unsupported mode")
            ids = self.page_ids.cpu()[self.valid.cpu()]
            if bool((ids < 0).any()) or bool((ids >= n).any()):
                raise ValueError("valid page IDs are outside the page range")
        elif self.seen_tokens != 0:
            raise ValueError("an empty page table cannot cover non-empty cache")
        return self

    def sequence_ranges(self) -> torch.Tensor:
        """[start, stop) per page on the table device."""
        return torch.stack((self.sequence_starts, self.sequence_starts + self.token_counts), dim=-1)

    def reorder(self, batch_indices) -> "DartPageTable":
        """Reorder batch rows like a beam update without touching packed storage."""
        indices = torch.as_tensor(batch_indices, dtype=torch.long, device=self.device)
        if indices.ndim != 1:
            raise ValueError("batch_indices must be one-dimensional")
        if indices.numel() and bool(((indices < 0) | (indices >= self.batch_size)).any()):
            raise IndexError("batch_indices contain an invalid batch row")
        return DartPageTable(self.page_ids.index_select(0, indices), self.sequence_starts, self.token_counts,
                             self.key_modes, self.value_modes, self.valid.index_select(0, indices),
                             self.seen_tokens, self.page_size)

    def to(self, device) -> "DartPageTable":
        return DartPageTable(self.page_ids.to(device), self.sequence_starts.to(device), self.token_counts.to(device),
                             self.key_modes.to(device), self.value_modes.to(device), self.valid.to(device),
                             self.seen_tokens, self.page_size)

    def uniform_quantized_runs(self, cache: "DartKVCache") -> tuple:
        """Stack consecutive full uniform pages page-major (reference page_table.py:181-211)."""
        segments = cache.iter_segments()
        if len(segments) != self.page_count or cache.seen_tokens != self.seen_tokens:
            raise ValueError("cache and page_table describe different page lifecycles")
        runs = []
        start = 0
        while start < len(segments):
            k0, v0 = segments[start]
            if not _uniform_full(k0, v0, self.page_size):
                start += 1
                continue
            end = start + 1
            while end < len(segments):
                k1, v1 = segments[end]
                if not _uniform_full(k1, v1, self.page_size) or not _same_layout(k0, v0, k1, v1):
                    break
                end += 1
            runs.append(_stack_run(self, segments[start:end], start))
            start = end
        return tuple(runs)


@dataclass(frozen=True)
class DartPageRun:
    """Page-major packed fields of one run of consecutive uniform pages (reference page_table.py:214-299)."""

    first_page_index: int
    page_indices: torch.Tensor
    sequence_starts: torch.Tensor
    token_counts: torch.Tensor
    key_values: torch.Tensor
    key_scale: torch.Tensor
    key_zero_point: torch.Tensor
    value_values: torch.Tensor
    value_scale: torch.Tensor
    value_zero_point: torch.Tensor
    key_bits: int
    value_bits: int
    key_group_size: int
    value_group_size: int
    page_size: int

    @property
    def page_count(self) -> int:
        return self.page_indices.shape[0]

    @property
    def device(self) -> torch.device:
        return self.key_values.device

    def validate(self) -> "DartPageRun":
        if self.page_indices.ndim != 1:
            raise ValueError("page_indices must have shape [run_pages]")
        n = self.page_count
        if n == 0:
            raise ValueError("a page run cannot be empty")
        if self.first_page_index < 0:
            raise ValueError("first_page_index must be non-negative")
        for name, t in (("sequence_starts", self.sequence_starts), ("token_counts", self.token_counts)):
            if t.ndim != 1 or t.shape[0] != n:
                raise ValueError(f"{name} must have shape [run_pages]")
        for name, t in (("key_values", self.key_values), ("key_scale", self.key_scale),
                        ("key_zero_point", self.key_zero_point), ("value_values", self.value_values),
                        ("value_scale", self.value_scale), ("value_zero_point", self.value_zero_point)):
            if t.ndim < 1 or t.shape[0] != n:
                raise ValueError(f"{name} must be page-major with first dimension {n}")
        if bool((self.token_counts <= 0).any()):
            raise ValueError("run token_counts must be positive")
        if n > 1:
            if not torch.equal(self.page_indices[1:], self.page_indices[:-1] + 1):
                raise ValueError("page IDs in a run must be consecutive")
            if not torch.equal(self.sequence_starts[1:], self.sequence_starts[:-1] + self.token_counts[:-1]):
                raise ValueError("run sequence_starts are not contiguous")
        if self.key_bits not in (2, 4, 8) or self.value_bits not in (2, 4, 8):
            raise ValueError("run bit widths must be 2, 4, or 8")
        if self.key_group_size <= 0 or self.value_group_size <= 0 or self.page_size <= 0:
            raise ValueError("run group sizes and page_size must be positive")
        return self

    def to(self, device) -> "DartPageRun":
        return DartPageRun(self.first_page_index, self.page_indices.to(device), self.sequence_starts.to(device),
                           self.token_counts.to(device), self.key_values.to(device), self.key_scale.to(device),
                           self.key_zero_point.to(device), self.value_values.to(device),
                           self.value_scale.to(device), self.value_zero_point.to(device), self.key_bits,
                           self.value_bits, self.key_group_size, self.value_group_size, self.page_size)


def _uniform_full(kseg, vseg, page_size: int) -> bool:
    return (isinstance(kseg, QuantizedTensor) and isinstance(vseg, QuantizedTensor)
            and kseg.original_shape[-2] == page_size and vseg.original_shape[-2] == page_size)


def _same_layout(k0, v0, k1, v1) -> bool:
    if not isinstance(k1, QuantizedTensor) or not isinstance(v1, QuantizedTensor):
        return False
    return (k0.original_shape == k1.original_shape and v0.original_shape == v1.original_shape
            and k0.values.shape == k1.values.shape and v0.values.shape == v1.values.shape
            and k0.scale.shape == k1.scale.shape and v0.scale.shape == v1.scale.shape
            and k0.bits == k1.bits and v0.bits == v1.bits
            and k0.group_size == k1.group_size and v0.group_size == v1.group_size)


def _stack_run(table: DartPageTable, segments: Sequence, first: int) -> DartPageRun:
    keys = [p[0] for p in segments]
    values = [p[1] for p in segments]
    dev = keys[0].values.device
    stop = first + len(segments)
    run = DartPageRun(
        first_page_index=first,
        page_indices=table.page_ids[0, first:stop].to(dev),
        sequence_starts=table.sequence_starts[first:stop].to(dev),
        token_counts=table.token_counts[first:stop].to(dev),
        key_values=torch.stack([s.values for s in keys], 0),
        key_scale=torch.stack([s.scale for s in keys], 0),
        key_zero_point=torch.stack([s.zero_point for s in keys], 0),
        value_values=torch.stack([s.values for s in values], 0),
        value_scale=torch.stack([s.scale for s in values], 0),
        value_zero_point=torch.stack([s.zero_point for s in values], 0),
        key_bits=keys[0].bits, value_bits=values[0].bits, key_group_size=keys[0].group_size,
        value_group_size=values[0].group_size, page_size=table.page_size,
    )
    return run.validate()


__all__ = ["DENSE_PAGE", "MIXED_PAGE", "QUANTIZED_PAGE", "DartPageTable", "DartPageRun"]

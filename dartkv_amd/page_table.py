"""Page descriptors of a DartKV cache: the public ``DartPageTable`` / ``DartPageRun`` types.

The field names, mode codes, validation messages and the run semantics are
the reference's interface (reference src/dart/page_table.py:19-299).  The
arrays themselves are views of the cache's own page directory and page pool:

* ``DartPageTable.from_cache`` reads the cache's device page directory (an
  int32 [N, 4] table of start, tokens, key mode and value mode per segment,
  rebuilt only when a page is sealed), so a table costs no walk over Python
  segment objects; ``page_ids`` and ``valid`` are broadcast views;
* ``uniform_quantized_runs`` hands out slices of the page pool (keys are
  page-major slots, values token-major rows), not stacked copies;
* ``validate`` evaluates every per-page invariant on the device and reads
  them back in one transfer.

The decode kernels do not read these objects: they walk the descriptor table
``DartKVCache.decode_plan`` builds.
"""

from __future__ import annotations

import dataclasses
from dataclasses import dataclass
from typing import TYPE_CHECKING, Sequence

import torch

if TYPE_CHECKING:
    from .cache import DartKVCache

DENSE_PAGE = 0
QUANTIZED_PAGE = 1
MIXED_PAGE = 2


def _require(ok: bool, message: str) -> None:
    if not ok:
        raise ValueError(message)


@dataclass(frozen=True)
class DartPageTable:
    """Batch-indexed page descriptors on one device (reference page_table.py:30-48).

    ``page_ids`` [B, N] maps a batch row to a segment index of
    ``cache.iter_segments()``; ``sequence_starts`` / ``token_counts`` [N]
    int32, ``key_modes`` / ``value_modes`` [N] int8 (``DENSE_PAGE``,
    ``QUANTIZED_PAGE``, ``MIXED_PAGE``), ``valid`` [B, N] bool.
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
        """The table of ``cache`` as it is now (reference page_table.py:50-87), on ``device``."""
        target = torch.device(device) if device is not None else (cache.device or torch.device("cpu"))
        if target.type == "cuda" and target.index is None:
            target = torch.device("cuda", torch.cuda.current_device())
        shape = cache.shape
        if shape is None:
            directory = torch.zeros(0, 4, dtype=torch.int32, device=target)
            batch = 0
        else:
            directory = cache._directory(target)
            batch = shape[0]
        n = directory.shape[0]
        return cls(
            page_ids=torch.arange(n, dtype=torch.int64, device=target).expand(batch, n),
            sequence_starts=directory[:, 0],
            token_counts=directory[:, 1],
            key_modes=directory[:, 2].to(torch.int8),
            value_modes=directory[:, 3].to(torch.int8),
            valid=torch.ones((), dtype=torch.bool, device=target).expand(batch, n),
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
        """Shape, order, length, mode and id invariants, checked in the reference's order
        (reference page_table.py:104-141)."""
        n = self.page_count
        _require(self.page_ids.ndim == 2 and self.valid.shape == self.page_ids.shape,
                 "page_ids and valid must have shape [batch, page_count]")
        for name in ("sequence_starts", "token_counts", "key_modes", "value_modes"):
            t = getattr(self, name)
            _require(t.ndim == 1 and t.shape[0] == n, f"{name} must have shape [page_count]")
        _require(self.page_size > 0 and self.seen_tokens >= 0, "page_size and seen_tokens must be non-negative/positive")
        if n == 0:
            _require(self.seen_tokens == 0, "an empty page table cannot cover non-empty cache")
            return self
        counts = self.token_counts.to(torch.int64)
        starts = self.sequence_starts.to(torch.int64)
        ids_ok = ((self.page_ids >= 0) & (self.page_ids < n)) | ~self.valid
        checks = torch.stack([
            (starts == torch.cumsum(counts, 0) - counts).all(),
            (counts > 0).all(),
            counts.sum() == self.seen_tokens,
            ((self.key_modes >= DENSE_PAGE) & (self.key_modes <= MIXED_PAGE)).all(),
            ((self.value_modes >= DENSE_PAGE) & (self.value_modes <= MIXED_PAGE)).all(),
            ids_ok.all(),
        ]).tolist()
        for ok, message in zip(checks, ("sequence_starts are not contiguous", "token_counts must be positive",
                                        "token_counts do not cover seen_tokens", "key_modes contain an unsupported mode",
                                        "value_modes contain an unsupported mode",
                                        "valid page IDs are outside the page range")):
            _require(ok, message)
        return self

    def sequence_ranges(self) -> torch.Tensor:
        """[start, stop) of every page, [N, 2] on the table's device."""
        return torch.stack((self.sequence_starts, self.sequence_starts + self.token_counts), dim=-1)

    def reorder(self, batch_indices) -> "DartPageTable":
        """Batch rows in a new order (a beam update); the packed storage is not touched."""
        indices = torch.as_tensor(batch_indices, dtype=torch.long, device=self.device)
        if indices.ndim != 1:
            raise ValueError("batch_indices must be one-dimensional")
        if indices.numel() and bool(((indices < 0) | (indices >= self.batch_size)).any()):
            raise IndexError("batch_indices contain an invalid batch row")
        return dataclasses.replace(self, page_ids=self.page_ids.index_select(0, indices),
                                   valid=self.valid.index_select(0, indices))

    def to(self, device) -> "DartPageTable":
        """The same table with its arrays on ``device``."""
        moved = {f.name: getattr(self, f.name).to(device) for f in dataclasses.fields(self)
                 if isinstance(getattr(self, f.name), torch.Tensor)}
        return dataclasses.replace(self, **moved)

    def uniform_quantized_runs(self, cache: "DartKVCache") -> tuple:
        """Runs of consecutive full uniform pages with one layout, as page-major slices of the cache's
        page pool (reference page_table.py:181-211).  Dense sink pages, mixed keys and the pending tail
        end a run."""
        return cache.uniform_page_runs(self)


@dataclass(frozen=True)
class DartPageRun:
    """Page-major packed fields of consecutive uniform pages (reference page_table.py:214-299).

    ``key_values`` [n, B, H, D, packed], ``key_scale`` / ``key_zero_point``
    [n, B, H, D, groups], ``value_values`` [n, B, H, page, packed],
    ``value_scale`` / ``value_zero_point`` [n, B, H, page, groups].
    """

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

    _PAGE_MAJOR = ("key_values", "key_scale", "key_zero_point", "value_values", "value_scale", "value_zero_point")

    @property
    def page_count(self) -> int:
        return self.page_indices.shape[0]

    @property
    def device(self) -> torch.device:
        return self.key_values.device

    def validate(self) -> "DartPageRun":
        """Shape, id order, contiguity, width and size checks with the reference's messages."""
        _require(self.page_indices.ndim == 1, "page_indices must have shape [run_pages]")
        n = self.page_count
        _require(n > 0, "a page run cannot be empty")
        _require(self.first_page_index >= 0, "first_page_index must be non-negative")
        for name in ("sequence_starts", "token_counts"):
            t = getattr(self, name)
            _require(t.ndim == 1 and t.shape[0] == n, f"{name} must have shape [run_pages]")
        for name in self._PAGE_MAJOR:
            t = getattr(self, name)
            _require(t.ndim >= 1 and t.shape[0] == n, f"{name} must be page-major with first dimension {n}")
        _require(not bool((self.token_counts <= 0).any()), "run token_counts must be positive")
        if n > 1:
            _require(torch.equal(self.page_indices[1:] - self.page_indices[:-1],
                                 torch.ones_like(self.page_indices[1:])), "page IDs in a run must be consecutive")
            _require(torch.equal(self.sequence_starts[1:], self.sequence_starts[:-1] + self.token_counts[:-1]),
                     "run sequence_starts are not contiguous")
        _require(self.key_bits in (2, 4, 8) and self.value_bits in (2, 4, 8), "run bit widths must be 2, 4, or 8")
        _require(min(self.key_group_size, self.value_group_size, self.page_size) > 0,
                 "run group sizes and page_size must be positive")
        return self

    def to(self, device) -> "DartPageRun":
        """The same run with every array on ``device``."""
        moved = {f.name: getattr(self, f.name).to(device) for f in dataclasses.fields(self)
                 if isinstance(getattr(self, f.name), torch.Tensor)}
        return dataclasses.replace(self, **moved)


__all__ = ["DENSE_PAGE", "MIXED_PAGE", "QUANTIZED_PAGE", "DartPageTable", "DartPageRun"]

"""Append-only compressed KV cache whose pages are produced by HIP kernels.

Lifecycle semantics follow the reference ``DartKVCache``
(reference src/dart/cache.py:45-661): dense sink prefix, page-sized
quantization, held partial pages, Kitty local / value-local buffers, value
page merging and union-boundary segment iteration.  What differs is where
the work happens:

* every page of one append is quantized by one ``dkv_quantize_key_pages``
  launch (keys along tokens) that also quantizes the values
  (values along head_dim, read in place from the appended tensor's token
  slice); page fields are views into page-major chunk tensors;
* the held partial page lives in a preallocated tail buffer, so a one-token
  decode append is a single device copy with no concatenation;
* the decode kernel reads a device table of segment descriptors that is
  rebuilt only when a page is sealed, never on a plain tail append.
"""

from __future__ import annotations

import contextlib
from dataclasses import dataclass
from typing import TYPE_CHECKING, List, Optional, Tuple, Union

import torch

from . import _lib
from .mixed import MixedQuantizedKey, launch_key_pages, promoted_count, random_channels
from .quantization import QuantizedTensor

Segment = Union[torch.Tensor, QuantizedTensor, MixedQuantizedKey]


class _PageRun:
    """Pages quantized by one launch: each field is one tensor with a page
    dimension (`dim`; page p is `size` entries of it starting at p * size,
    and dim 0 is dropped from the page's view), plus the fields every page
    shares.  A prefill of 127 pages would otherwise create about a thousand
    tensor views in Python before the first page is read."""

    __slots__ = ("tensors", "dim", "size", "shared")

    def __init__(self, tensors: dict, dim: int, size: int, shared: dict) -> None:
        self.tensors, self.dim, self.size, self.shared = tensors, dim, size, shared

    def view(self, name: str, page: int) -> torch.Tensor:
        t = self.tensors[name]
        return t[page] if self.dim == 0 else t.narrow(self.dim, page * self.size, self.size)

    def block(self, name: str, page: int) -> Optional[Tuple[int, int]]:
        """(address, (batch, head) stride) of the page's block as _bh_block gives it, or None when
        _bh_block would need a copy (then the caller materializes the view)."""
        t = self.tensors[name]
        if t.numel() == 0:
            return 0, 0
        strides, shape = t.stride(), t.shape
        if self.dim == 0:
            strides, shape = strides[1:], shape[1:]
        else:
            shape = shape[:self.dim] + (self.size,) + shape[self.dim + 1:]
        B, H = shape[0], shape[1]
        inner = 1
        for size, stride in zip(reversed(shape[2:]), reversed(strides[2:])):
            if size != 1 and stride != inner:
                return None
            inner *= size
        if H > 1:
            bh = strides[1]
            if not (B == 1 or strides[0] == H * bh):
                return None
        else:
            bh = strides[0] if B > 1 else inner
        offset = page * (t.stride(0) if self.dim == 0 else self.size * t.stride(self.dim))
        return t.data_ptr() + offset * t.element_size(), bh


class _RunField:
    """A segment field read from the segment's page run: a tensor field becomes the page's view
    on first access (then cached in the instance), a shared field is the run's value."""

    def __init__(self, name: str, tensor: bool) -> None:
        self.name, self.tensor = name, tensor

    def __get__(self, obj, cls=None):
        if obj is None:
            return self
        if not self.tensor:
            return obj._run.shared[self.name]
        v = obj._run.view(self.name, obj._page)
        obj.__dict__[self.name] = v
        return v


class _PagedMixedKey(MixedQuantizedKey):
    """One page of a `_PageRun` of mixed keys; behaves as a MixedQuantizedKey."""

    low_values = _RunField("low_values", True)
    high_values = _RunField("high_values", True)
    channel_indices = _RunField("channel_indices", True)
    scale = _RunField("scale", True)
    zero_point = _RunField("zero_point", True)
    original_shape = _RunField("original_shape", False)
    padded_tokens = _RunField("padded_tokens", False)
    group_size = _RunField("group_size", False)
    low_bits = _RunField("low_bits", False)
    promote_bits = _RunField("promote_bits", False)
    output_dtype = _RunField("output_dtype", False)

    def __init__(self, run: _PageRun, page: int) -> None:  # pylint: disable=super-init-not-called
        self._run, self._page = run, page


class _PagedQuantized(QuantizedTensor):
    """One page of a `_PageRun` of uniform codes; behaves as a QuantizedTensor."""

    values = _RunField("values", True)
    scale = _RunField("scale", True)
    zero_point = _RunField("zero_point", True)
    original_shape = _RunField("original_shape", False)
    original_dim = _RunField("original_dim", False)
    padded_dim = _RunField("padded_dim", False)
    packed_dim = _RunField("packed_dim", False)
    group_size = _RunField("group_size", False)
    bits = _RunField("bits", False)
    output_dtype = _RunField("output_dtype", False)
    axis = _RunField("axis", False)

    def __init__(self, run: _PageRun, page: int) -> None:  # pylint: disable=super-init-not-called
        self._run, self._page = run, page

if TYPE_CHECKING:
    from .page_table import DartPageRun, DartPageTable


@dataclass(frozen=True)
class DartSegmentLayout:
    """Storage layout for one logical K/V segment (reference cache.py:20-31).

    ``fields`` lists (name, shape, element strides) of the packed tensors.
    """

    kind: str
    logical_shape: Tuple[int, ...]
    fields: Tuple[Tuple[str, Tuple[int, ...], Tuple[int, ...]], ...]


@dataclass(frozen=True)
class DartPageMetadata:
    """Sequence-order metadata for one page, sink segment, or pending buffer (reference cache.py:34-42)."""

    index: int
    sequence_start: int
    token_count: int
    key: DartSegmentLayout
    value: DartSegmentLayout


@dataclass(frozen=True)
class DartKVCacheConfig:
    """Cache configuration; fields, defaults and validation as reference cache.py:45-112."""

    bits: int = 2
    group_size: int = 64
    sink_tokens: int = 0
    metadata_dtype: torch.dtype = torch.float16
    key_bits: Optional[int] = None
    value_bits: Optional[int] = None
    key_group_size: Optional[int] = None
    value_group_size: Optional[int] = None
    page_size: int = 128
    hold_partial_pages: bool = False
    local_tokens: int = 0
    value_local_tokens: int = 0
    promote_bits: int = 4
    promote_ratio: float = 0.0
    channel_selection: str = "magnitude"

    def __post_init__(self) -> None:
        if self.bits not in (2, 4, 8):
            raise ValueError("bits must be one of 2, 4, or 8")
        if self.group_size <= 0:
            raise ValueError("group_size must be positive")
        if self.sink_tokens < 0:
            raise ValueError("sink_tokens must be non-negative")
        for name, value in (("key_bits", self.key_bits), ("value_bits", self.value_bits)):
            if value is not None and value not in (2, 4, 8):
                raise ValueError(f"{name} must be one of 2, 4, or 8")
        for name, value in (("key_group_size", self.key_group_size), ("value_group_size", self.value_group_size)):
            if value is not None and (not isinstance(value, int) or value <= 0):
                raise ValueError(f"{name} must be a positive integer")
        if self.page_size <= 0:
            raise ValueError("page_size must be positive")
        if not isinstance(self.local_tokens, int) or self.local_tokens < 0:
            raise ValueError("local_tokens must be a non-negative integer")
        if not isinstance(self.value_local_tokens, int) or self.value_local_tokens < 0:
            raise ValueError("value_local_tokens must be a non-negative integer")
        if self.promote_bits != 4:
            raise ValueError("the reference mixed representation currently supports promote_bits=4")
        if not 0.0 <= self.promote_ratio <= 1.0:
            raise ValueError("promote_ratio must be in [0, 1]")
        if self.channel_selection not in {"magnitude", "random", "variance"}:
            raise ValueError("channel_selection must be 'magnitude', 'random', or 'variance'")
        if self.metadata_dtype not in (torch.float16, torch.bfloat16, torch.float32, torch.float64):
            raise TypeError("metadata_dtype must be a floating-point torch dtype")

    @property
    def resolved_key_bits(self) -> int:
        return self.key_bits if self.key_bits is not None else self.bits

    @property
    def resolved_value_bits(self) -> int:
        return self.value_bits if self.value_bits is not None else self.bits

    @property
    def resolved_key_group_size(self) -> int:
        return self.key_group_size if self.key_group_size is not None else self.group_size

    @property
    def resolved_value_group_size(self) -> int:
        return self.value_group_size if self.value_group_size is not None else self.group_size


class _DecodePlan:
    """Device table of sealed segment descriptors plus the tensors it points into.

    ``fast_first``/``fast_count`` mark the run of table entries a page kernel
    may take (full 128-token pages in its layout); ``fast_promoted`` (0 for
    uniform pages), ``fast_value_group``, ``fast_key_bits`` and
    ``fast_value_bits`` describe that run.  ``rest_dense`` is the most tokens of any sealed entry outside
    that run when the dense decode kernel can read all of them, else -1.
    """

    def __init__(self, version: int, device: torch.device, table: Optional[torch.Tensor], count: int,
                 keepalive: list, tail_is_pending: bool, n_tokens: int, fast: Tuple[int, int, int, int, int, int],
                 rest_dense: int = -1) -> None:
        self.version = version
        self.device = device
        self.table = table
        self.count = count
        self.keepalive = keepalive
        self.tail_is_pending = tail_is_pending
        self.n_tokens = n_tokens
        (self.fast_first, self.fast_count, self.fast_promoted, self.fast_value_group, self.fast_key_bits,
         self.fast_value_bits) = fast
        self.rest_dense = rest_dense


class DartKVCache:
    """Append-only KV cache over HIP-quantized pages (reference cache.py:115-542).

    Inputs and returned tensors use ``[batch, kv_heads, sequence, head_dim]``
    on a ROCm device.  The cache owns detached copies of appended tensors.
    """

    def __init__(self, config: Optional[DartKVCacheConfig] = None) -> None:
        self.config = config or DartKVCacheConfig()
        self._key_segments: List[Segment] = []
        self._value_segments: List[Segment] = []
        self._pending_key: Optional[torch.Tensor] = None
        self._pending_value: Optional[torch.Tensor] = None
        self._shape: Optional[Tuple[int, int, int]] = None
        self._dtype: Optional[torch.dtype] = None
        self._device: Optional[torch.device] = None
        self._seen_tokens = 0
        self._layout_version = 0
        self._page_table_cache: dict = {}
        self._page_run_cache: dict = {}
        # Sealed-structure version: bumps when any segment other than the
        # held tail changes; the decode table is rebuilt only then.
        self._sealed_version = 0
        self._tail_key: Optional[torch.Tensor] = None
        self._tail_value: Optional[torch.Tensor] = None
        self._decode_plan_cache: Optional[_DecodePlan] = None
        self._random_channels: Optional[torch.Tensor] = None
        # device copy of the held tail's length (replayable decode steps); None when off
        self._tail_count_dev: Optional[torch.Tensor] = None
        # int32 [2] device flags (keys, values) the quantize kernels set on a NaN or an infinity
        self._nonfinite: Optional[torch.Tensor] = None
        self._nonfinite_ptrs: Tuple[int, int] = (0, 0)

    # ---- reference properties ----
    @property
    def seen_tokens(self) -> int:
        return self._seen_tokens

    @property
    def layout_version(self) -> int:
        """Monotonic descriptor version changed by append, clear, or device move."""
        return self._layout_version

    def get_seq_length(self) -> int:
        return self._seen_tokens

    @property
    def shape(self) -> Optional[Tuple[int, int, int, int]]:
        if self._shape is None:
            return None
        batch, heads, head_dim = self._shape
        return batch, heads, self._seen_tokens, head_dim

    @property
    def dtype(self) -> Optional[torch.dtype]:
        return self._dtype

    @property
    def device(self) -> Optional[torch.device]:
        return self._device

    def __len__(self) -> int:
        return self._seen_tokens

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Append a chunk and return the materialized cache contents."""
        self.append(key_states, value_states)
        return self.get()

    def append(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        """Append a chunk without materializing the cache (reference cache.py:168-190)."""
        _lib.require_device(key_states, value_states)
        self._validate_inputs(key_states, value_states)
        key_states = key_states.detach()
        value_states = value_states.detach()
        if key_states.stride(-1) != 1:
            key_states = key_states.contiguous()
        if value_states.stride(-1) != 1:
            value_states = value_states.contiguous()
        chunk = key_states.shape[-2]
        sink_remaining = max(0, self.config.sink_tokens - self._seen_tokens)
        sink = min(sink_remaining, chunk)
        if sink:
            self._key_segments.append(key_states[..., :sink, :].clone())
            self._value_segments.append(value_states[..., :sink, :].clone())
            self._sealed_version += 1
        if sink < chunk:
            if not self._device_tail_append(key_states[..., sink:, :], value_states[..., sink:, :]):
                if self._tail_count_dev is not None and torch.cuda.is_current_stream_capturing():
                    raise RuntimeError("a captured append may only extend the held tail by one token")
                self._append_remainder(key_states[..., sink:, :], value_states[..., sink:, :])
                self._sync_device_tail()
        self._seen_tokens += chunk
        self._layout_version += 1
        self._invalidate_page_descriptors()

    def get(self) -> Tuple[torch.Tensor, torch.Tensor]:
        if self._seen_tokens == 0:
            raise RuntimeError("DartKVCache is empty; call update() before get()")
        keys = [_materialize(s) for s in self._key_segments]
        values = [_materialize(s) for s in self._value_segments]
        if self._pending_key is not None:
            keys.append(self._pending_key)
        if self._pending_value is not None:
            values.append(self._pending_value)
        return torch.cat(keys, dim=-2), torch.cat(values, dim=-2)

    @property
    def key_states(self) -> torch.Tensor:
        return self.get()[0]

    @property
    def value_states(self) -> torch.Tensor:
        return self.get()[1]

    @property
    def storage_bytes(self) -> int:
        pending = 0
        if self._pending_key is not None:
            pending += self._pending_key.numel() * self._pending_key.element_size()
        if self._pending_value is not None:
            pending += self._pending_value.numel() * self._pending_value.element_size()
        return sum(_segment_nbytes(s) for s in (*self._key_segments, *self._value_segments)) + pending

    @property
    def dense_bytes(self) -> int:
        if self._shape is None or self._dtype is None:
            return 0
        batch, heads, head_dim = self._shape
        return 2 * batch * heads * self._seen_tokens * head_dim * torch.tensor([], dtype=self._dtype).element_size()

    @property
    def compression_ratio(self) -> float:
        return self.dense_bytes / self.storage_bytes if self.storage_bytes else 1.0

    def iter_segments(self) -> list:
        """K/V segments in sequence order over the union of their boundaries (reference cache.py:229-274)."""
        key_segments = list(self._key_segments)
        value_segments = list(self._value_segments)
        if self._pending_key is not None:
            if self._pending_value is None:
                raise RuntimeError("DartKVCache has a pending key without a pending value")
            key_segments.append(self._pending_key)
            value_segments.append(self._pending_value)
        if not key_segments or not value_segments:
            return []
        pairs = []
        ki = vi = ko = vo = 0
        while ki < len(key_segments) and vi < len(value_segments):
            kseg, vseg = key_segments[ki], value_segments[vi]
            klen, vlen = _segment_tokens(kseg), _segment_tokens(vseg)
            take = min(klen - ko, vlen - vo)
            if take <= 0:
                raise RuntimeError("DartKVCache contains an empty logical segment")
            pairs.append((_slice_segment(kseg, ko, ko + take), _slice_segment(vseg, vo, vo + take)))
            ko += take
            vo += take
            if ko == klen:
                ki, ko = ki + 1, 0
            if vo == vlen:
                vi, vo = vi + 1, 0
        if ki != len(key_segments) or vi != len(value_segments):
            raise RuntimeError("DartKVCache key/value logical lengths diverged")
        return pairs

    def page_metadata(self) -> list:
        """Page order, logical lengths, shapes and element strides (reference cache.py:276-300)."""
        metadata = []
        start = 0
        for index, (kseg, vseg) in enumerate(self.iter_segments()):
            klay, vlay = _segment_layout(kseg), _segment_layout(vseg)
            ktok, vtok = klay.logical_shape[-2], vlay.logical_shape[-2]
            if ktok != vtok:
                raise RuntimeError("DartKVCache key/value page lengths diverged")
            metadata.append(DartPageMetadata(index=index, sequence_start=start, token_count=ktok, key=klay,
                                             value=vlay))
            start += ktok
        if start != self._seen_tokens:
            raise RuntimeError(f"page metadata covers {start} tokens, expected {self._seen_tokens}")
        return metadata

    def page_table(self, *, device=None, rebuild: bool = False) -> "DartPageTable":
        """Cached page descriptors, invalidated on append/clear/move (reference cache.py:302-323)."""
        from .page_table import DartPageTable

        target = _descriptor_device(device, self._device)
        cached = self._page_table_cache.get(target)
        if cached is not None and not rebuild and cached[0] == self._layout_version:
            return cached[1]
        table = DartPageTable.from_cache(self, device=target)
        self._page_table_cache[target] = (self._layout_version, table)
        return table

    def page_runs(self, *, device=None, page_table=None, rebuild: bool = False) -> tuple:
        """Cached page-major uniform runs (reference cache.py:325-352)."""
        target = _descriptor_device(device, self._device)
        if page_table is None:
            cached = self._page_run_cache.get(target)
            if cached is not None and not rebuild and cached[0] == self._layout_version:
                return cached[1]
            table = self.page_table(device=target, rebuild=rebuild)
        else:
            table = page_table
        runs = table.uniform_quantized_runs(self)
        if device is not None:
            runs = tuple(run if run.device == target else run.to(target) for run in runs)
        if page_table is None:
            self._page_run_cache[target] = (self._layout_version, runs)
        return runs

    def to(self, device) -> "DartKVCache":
        """Move backing tensors to ``device`` (reference cache.py:354-366)."""
        self._key_segments = [s.to(device) for s in self._key_segments]
        self._value_segments = [s.to(device) for s in self._value_segments]
        if self._pending_key is not None:
            self._pending_key = self._pending_key.to(device)
        if self._pending_value is not None:
            self._pending_value = self._pending_value.to(device)
        self._tail_key = self._tail_value = None
        self._tail_count_dev = None
        self._device = _descriptor_device(device, self._device)
        self._layout_version += 1
        self._sealed_version += 1
        self._invalidate_page_descriptors()
        return self

    def clear(self) -> None:
        self._key_segments.clear()
        self._value_segments.clear()
        self._pending_key = None
        self._pending_value = None
        self._tail_key = self._tail_value = None
        self._shape = None
        self._dtype = None
        self._device = None
        self._seen_tokens = 0
        self._layout_version += 1
        self._sealed_version += 1
        self._decode_plan_cache = None
        self._tail_count_dev = None
        self._invalidate_page_descriptors()

    def _invalidate_page_descriptors(self) -> None:
        self._page_table_cache.clear()
        self._page_run_cache.clear()

    def _validate_inputs(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        """Same checks and messages as reference cache.py:384-401."""
        if key_states.ndim != 4 or value_states.ndim != 4:
            raise ValueError("key_states and value_states must have shape [B, H, T, D]")
        if key_states.shape != value_states.shape:
            raise ValueError(f"key/value shapes must match, got {key_states.shape} and {value_states.shape}")
        if key_states.dtype != value_states.dtype or key_states.device != value_states.device:
            raise ValueError("key_states and value_states must use the same dtype and device")
        if key_states.shape[-2] == 0 or key_states.shape[-1] == 0:
            raise ValueError("key/value sequence and head dimensions must be non-empty")
        if not torch.is_floating_point(key_states) or not torch.is_floating_point(value_states):
            raise TypeError("key_states and value_states must be floating-point tensors")
        shape = (key_states.shape[0], key_states.shape[1], key_states.shape[3])
        if self._shape is None:
            if key_states.dtype == torch.float64:
                raise TypeError("dartkv_amd caches float16, bfloat16 and float32 tensors")
            self._shape = shape
            self._dtype = key_states.dtype
            self._device = key_states.device
        elif shape != self._shape or key_states.dtype != self._dtype or key_states.device != self._device:
            raise ValueError("all updates must keep batch/head/head_dim, dtype, and device unchanged")

    # ---- held tail ----
    def _tail_capacity(self) -> int:
        return self.config.page_size + self.config.local_tokens

    def _store_pending(self, keys: Optional[torch.Tensor], values: Optional[torch.Tensor]) -> None:
        """Keep ``keys``/``values`` as the pending tail, in the preallocated tail buffers when they fit."""
        if keys is None or values is None or keys.shape[-2] != values.shape[-2] or \
                keys.shape[-2] > self._tail_capacity():
            self._pending_key = keys.clone() if keys is not None else None
            self._pending_value = values.clone() if values is not None else None
            return
        n = keys.shape[-2]
        if self._tail_key is None or self._tail_key.device != keys.device:
            B, H, _, D = keys.shape
            cap = self._tail_capacity()
            self._tail_key = torch.empty(B, H, cap, D, dtype=keys.dtype, device=keys.device)
            self._tail_value = torch.empty(B, H, cap, D, dtype=values.dtype, device=values.device)
        self._tail_key[..., :n, :].copy_(keys)
        self._tail_value[..., :n, :].copy_(values)
        self._pending_key = self._tail_key[..., :n, :]
        self._pending_value = self._tail_value[..., :n, :]

    def _pending_in_tail(self) -> bool:
        pk, tk = self._pending_key, self._tail_key
        return (pk is not None and tk is not None and self._pending_value is not None
                and pk.data_ptr() == tk.data_ptr() and self._pending_value.data_ptr() == self._tail_value.data_ptr()
                and pk.shape[-2] == self._pending_value.shape[-2])

    # ---- append paths (reference cache.py:403-542) ----
    def _append_remainder(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        c = self.config
        if c.value_local_tokens:
            self._append_key_remainder(key_states)
            self._append_value_remainder(value_states)
            self._sealed_version += 1
            return
        if c.hold_partial_pages or c.local_tokens:
            pending = 0 if self._pending_key is None else self._pending_key.shape[-2]
            total = pending + key_states.shape[-2]
            available = max(0, total - c.local_tokens)
            full = (available // c.page_size) * c.page_size
            if full == 0 and self._pending_in_tail() and total <= self._tail_capacity():
                # fast path: the new tokens only extend the held tail
                self._tail_key[..., pending:total, :].copy_(key_states)
                self._tail_value[..., pending:total, :].copy_(value_states)
                self._pending_key = self._tail_key[..., :total, :]
                self._pending_value = self._tail_value[..., :total, :]
                return
            if self._pending_key is not None:
                key_states = torch.cat((self._pending_key, key_states), dim=-2)
                value_states = torch.cat((self._pending_value, value_states), dim=-2)
            if full:
                self._quantize_pages(key_states[..., :full, :], value_states[..., :full, :])
            if full < key_states.shape[-2]:
                self._store_pending(key_states[..., full:, :], value_states[..., full:, :])
            else:
                self._pending_key = self._pending_value = None
            self._sealed_version += 1
            return
        self._quantize_pages(key_states, value_states)
        self._sealed_version += 1

    def _append_key_remainder(self, key_states: torch.Tensor) -> None:
        """Kitty key Q-buffer lifecycle (reference cache.py:424-455)."""
        c = self.config
        if (self._seen_tokens > 0 and self._pending_key is None and c.local_tokens == 1
                and key_states.shape[-2] == 1 and self._key_segments
                and not isinstance(self._key_segments[-1], torch.Tensor)):
            final_page = _materialize(self._key_segments.pop())
            self._key_pages_only(final_page)
        if self._pending_key is not None:
            key_states = torch.cat((self._pending_key, key_states), dim=-2)
        local = 0 if self._seen_tokens == 0 else c.local_tokens
        available = max(0, key_states.shape[-2] - local)
        full = (available // c.page_size) * c.page_size
        if full:
            self._key_pages_only(key_states[..., :full, :])
        self._pending_key = key_states[..., full:, :].clone() if full < key_states.shape[-2] else None

    def _append_value_remainder(self, value_states: torch.Tensor) -> None:
        """Kitty value Local buffer (reference cache.py:457-470)."""
        c = self.config
        if self._pending_value is not None:
            value_states = torch.cat((self._pending_value, value_states), dim=-2)
        quantized = max(0, value_states.shape[-2] - c.value_local_tokens)
        if quantized:
            with self._finite_inputs():
                for start in range(0, quantized, c.page_size):
                    stop = min(start + c.page_size, quantized)
                    for seg in self._quantize_value_chunks(value_states[..., start:stop, :], stop - start):
                        self._append_quantized_value_page(seg)
        self._pending_value = value_states[..., quantized:, :].clone() if quantized < value_states.shape[-2] else None

    @contextlib.contextmanager
    def _finite_inputs(self):
        """Quantize launches inside this scope report NaN or infinite inputs through device flags;
        on exit the flags are read (one host synchronization) and such an input raises the reference's
        ValueError (quantization.py:159-160, mixed.py:187-188) with the segment lists restored."""
        flags = self._nonfinite
        if flags is None or flags.device != self._device:
            flags = self._nonfinite = torch.zeros(2, dtype=torch.int32, device=self._device)
        else:
            flags.zero_()
        keys, values = list(self._key_segments), list(self._value_segments)
        self._nonfinite_ptrs = (flags.data_ptr(), flags.data_ptr() + 4)
        try:
            yield
        finally:
            self._nonfinite_ptrs = (0, 0)
        bad_keys, bad_values = flags.tolist()
        if bad_keys or bad_values:
            self._key_segments, self._value_segments = keys, values
            if bad_keys and self.config.promote_ratio > 0.0:
                raise ValueError("key_states must contain finite values")
            raise ValueError("quantize expects all values to be finite")

    def _quantize_pages(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        """Quantize consecutive pages; the last may be partial (reference cache.py:472-479)."""
        if key_states.shape[-2] != value_states.shape[-2]:
            raise RuntimeError("key/value page lengths diverged before quantization")
        with self._finite_inputs():
            jobs: list = []
            values = self._quantize_value_chunks(value_states, self.config.page_size, jobs)
            keys = self._quantize_key_chunks(key_states, jobs)
            for kseg, vseg in zip(keys, values):
                self._key_segments.append(kseg)
                self._append_quantized_value_page(vseg)

    def _key_pages_only(self, key_states: torch.Tensor) -> None:
        with self._finite_inputs():
            self._key_segments.extend(self._quantize_key_chunks(key_states))

    def _quantize_key_chunks(self, key_states: torch.Tensor, value_jobs: Optional[list] = None) -> List[Segment]:
        """Key pages of ``page_size`` tokens (last may be shorter), one launch per page size.

        ``value_jobs`` from _quantize_value_chunks: each goes into the key
        launch that covers the same tokens.
        """
        c = self.config
        T = key_states.shape[-2]
        P = c.page_size
        full = T // P
        jobs = {start: (n, job) for start, n, job, _ in (value_jobs or [])}

        def job_for(start: int, n: int):
            entry = jobs.pop(start, None)
            if entry is None:
                return None
            if entry[0] != n:
                raise RuntimeError("value rows and key pages cover different tokens")
            return entry[1]

        out: List[Segment] = []
        if full:
            out.extend(self._quantize_key_launch(key_states[..., : full * P, :], P, full, job_for(0, full * P)))
        if T - full * P:
            out.extend(self._quantize_key_launch(key_states[..., full * P:, :], T - full * P, 1,
                                                 job_for(full * P, T - full * P)))
        if jobs:
            raise RuntimeError("value rows left without a key launch")
        return out

    def _quantize_key_launch(self, src: torch.Tensor, tokens: int, n_pages: int, values=None) -> List[Segment]:
        c = self.config
        B, H, _, D = src.shape
        dev = src.device
        meta = c.metadata_dtype
        kg = c.resolved_key_group_size
        G = (tokens + kg - 1) // kg
        if c.promote_ratio > 0.0:
            K = promoted_count(D, c.promote_ratio)
            nb = (kg + 3) // 4
            low = torch.empty(n_pages, B, H, D, G, nb, dtype=torch.uint8, device=dev)
            high = torch.empty(n_pages, B, H, K, G, nb if K else nb * 4, dtype=torch.uint8, device=dev)
            idx = torch.empty(n_pages, B, H, K, dtype=torch.int32, device=dev)
            scale = torch.empty(n_pages, B, H, D, G, dtype=meta, device=dev)
            zero = torch.empty(n_pages, B, H, D, G, dtype=meta, device=dev)
            strategy = c.channel_selection
            given = None
            if strategy == "random" and 0 < K < D:
                # one randperm per KV head per page, shared across the batch (mixed.py:145-153)
                given = torch.stack([random_channels(H, D, K, dev) for _ in range(n_pages)], 0).to(torch.int32)
            selection = {"magnitude": _lib.SELECT_MAGNITUDE, "variance": _lib.SELECT_VARIANCE,
                         "random": _lib.SELECT_GIVEN}[strategy]
            if given is not None and n_pages > 1:
                for p in range(n_pages):
                    launch_key_pages(src[..., p * tokens:(p + 1) * tokens, :], page_tokens=tokens, n_pages=1,
                                     key_mode=_lib.KEY_MIXED, bits=2, group=kg, promoted=K, selection=selection,
                                     given_idx=given[p].contiguous(), meta=meta, low=low[p], high=high[p],
                                     idx=idx[p], scale=scale[p], zero=zero[p],
                                     values=values if p == n_pages - 1 else None,
                                     nonfinite=self._nonfinite_ptrs[0])
            else:
                launch_key_pages(src, page_tokens=tokens, n_pages=n_pages, key_mode=_lib.KEY_MIXED, bits=2,
                                 group=kg, promoted=K, selection=selection,
                                 given_idx=None if given is None else given[0].contiguous(), meta=meta,
                                 low=low, high=high, idx=idx, scale=scale, zero=zero, values=values,
                                 nonfinite=self._nonfinite_ptrs[0])
            run = _PageRun(dict(low_values=low, high_values=high, channel_indices=idx, scale=scale, zero_point=zero),
                           0, 1, dict(original_shape=(B, H, tokens, D), padded_tokens=G * kg, group_size=kg,
                                      low_bits=2, promote_bits=c.promote_bits, output_dtype=src.dtype))
            return [_PagedMixedKey(run, p) for p in range(n_pages)]
        bits = c.resolved_key_bits
        per = 8 // bits
        padded = G * kg
        packed_dim = ((padded + per - 1) // per) * per
        codes = torch.empty(n_pages, B, H, D, packed_dim // per, dtype=torch.uint8, device=dev)
        scale = torch.empty(n_pages, B, H, D, G, dtype=meta, device=dev)
        zero = torch.empty(n_pages, B, H, D, G, dtype=meta, device=dev)
        launch_key_pages(src, page_tokens=tokens, n_pages=n_pages, key_mode=_lib.KEY_UNIFORM, bits=bits, group=kg,
                         promoted=0, selection=0, given_idx=None, meta=meta, low=codes, high=None, idx=None,
                         scale=scale, zero=zero, values=values, nonfinite=self._nonfinite_ptrs[0])
        run = _PageRun(dict(values=codes, scale=scale, zero_point=zero), 0, 1,
                       dict(original_shape=(B, H, tokens, D), original_dim=tokens, padded_dim=padded,
                            packed_dim=packed_dim, group_size=kg, bits=bits, output_dtype=src.dtype, axis=2))
        return [_PagedQuantized(run, p) for p in range(n_pages)]

    def _quantize_value_chunks(self, value_states: torch.Tensor, chunk: int,
                               jobs: Optional[list] = None) -> List[QuantizedTensor]:
        """Value segments of ``chunk`` tokens (last may be shorter) quantized along head_dim.

        All full chunks share one launch and one [B,H,T,P] code tensor; each
        segment is a token-range view of it.  With ``jobs`` (a list) nothing is
        launched here: each launch's (token start, token count, job, keepalive)
        is appended for the caller to hand to the key launch of the same tokens.
        """
        c = self.config
        B, H, T, D = value_states.shape
        dev = value_states.device
        bits, vg, meta = c.resolved_value_bits, c.resolved_value_group_size, c.metadata_dtype
        Gv = (D + vg - 1) // vg
        per = 8 // bits
        padded = Gv * vg
        packed_dim = ((padded + per - 1) // per) * per
        full = T // chunk
        out: List[QuantizedTensor] = []
        for start, count, size in ((0, full, chunk), (full * chunk, 1 if T - full * chunk else 0, T - full * chunk)):
            if not count:
                continue
            n = count * size
            src = value_states[..., start:start + n, :]
            values = torch.empty(B, H, n, packed_dim // per, dtype=torch.uint8, device=dev)
            scale = torch.empty(B, H, n, Gv, dtype=meta, device=dev)
            zero = torch.empty(B, H, n, Gv, dtype=meta, device=dev)
            if jobs is None:
                _launch_value_rows(src, bits, vg, meta, values, scale, zero, self._nonfinite_ptrs[1])
            else:
                job, keep = _value_rows_job(src, bits, vg, meta, values, scale, zero, self._nonfinite_ptrs[1])
                jobs.append((start, n, job, keep))
            run = _PageRun(dict(values=values, scale=scale, zero_point=zero), 2, size,
                           dict(original_shape=(B, H, size, D), original_dim=D, padded_dim=padded,
                                packed_dim=packed_dim, group_size=vg, bits=bits, output_dtype=value_states.dtype,
                                axis=3))
            out.extend(_PagedQuantized(run, i) for i in range(count))
        return out

    def _append_quantized_value_page(self, segment: QuantizedTensor) -> None:
        """Merge token-wise values into page-sized segments (reference cache.py:514-542)."""
        if not self._value_segments or isinstance(self._value_segments[-1], torch.Tensor):
            self._value_segments.append(segment)
            return
        previous = self._value_segments[-1]
        if not isinstance(previous, QuantizedTensor):
            raise RuntimeError("unexpected value segment type while coalescing pages")
        if previous.original_shape[-2] == self.config.page_size:
            self._value_segments.append(segment)
            return
        combined = _merge_quantized_tensors([previous, segment])
        n = combined.original_shape[-2]
        self._value_segments[-1] = _slice_quantized_tensor(combined, 0, min(self.config.page_size, n))
        if n > self.config.page_size:
            self._value_segments.append(_slice_quantized_tensor(combined, self.config.page_size, n))

    # ---- replayable decode steps ----
    def enable_device_tail(self) -> None:
        """Keep the held tail's length in device memory as well.

        One-token appends that only extend the tail then write at the device
        count and advance it on the device, and decode reads the count there,
        so a decode step's launches can be captured in a graph and replayed.
        The host-side state of a replayed append is advanced afterwards with
        ``advance_device_tail``.  Appends that seal a page take the ordinary
        path and resynchronize the device count.
        """
        if self.config.value_local_tokens:
            raise ValueError("device-side tail counts need value_local_tokens == 0")
        if not (self.config.hold_partial_pages or self.config.local_tokens):
            raise ValueError("device-side tail counts need a held tail (hold_partial_pages or local_tokens)")
        if self._shape is None:
            raise RuntimeError("append the prompt before enabling device-side tail counts")
        if self._tail_key is None:
            B, H, D = self._shape
            cap = self._tail_capacity()
            self._tail_key = torch.empty(B, H, cap, D, dtype=self._dtype, device=self._device)
            self._tail_value = torch.empty(B, H, cap, D, dtype=self._dtype, device=self._device)
        if self._pending_key is not None and not self._pending_in_tail():
            self._store_pending(self._pending_key, self._pending_value)
            if not self._pending_in_tail():
                raise RuntimeError("the held tail does not fit the tail buffer")
        self._tail_count_dev = torch.zeros(1, dtype=torch.int64, device=self._device)
        self._sync_device_tail()
        self._sealed_version += 1

    @property
    def device_tail(self) -> Optional[torch.Tensor]:
        """int64 [1] device tensor holding the held tail's length, or None."""
        return self._tail_count_dev

    def _pending_tokens(self) -> int:
        return 0 if self._pending_key is None else self._pending_key.shape[-2]

    def _sync_device_tail(self) -> None:
        if self._tail_count_dev is not None:
            if self._pending_key is not None and not self._pending_in_tail():
                self._store_pending(self._pending_key, self._pending_value)
            self._tail_count_dev.fill_(self._pending_tokens())

    def next_append_seals(self, tokens: int = 1) -> bool:
        """Whether appending ``tokens`` tokens now would seal a page (or overflow the tail buffer)."""
        c = self.config
        total = self._pending_tokens() + tokens
        return (max(0, total - c.local_tokens) // c.page_size) > 0 or total > self._tail_capacity()

    def _device_tail_append(self, key_states: torch.Tensor, value_states: torch.Tensor) -> bool:
        if self._tail_count_dev is None or key_states.shape[-2] != 1 or self.next_append_seals(1):
            return False
        if self._pending_key is not None and not self._pending_in_tail():
            return False
        self._tail_key.index_copy_(2, self._tail_count_dev, key_states)
        self._tail_value.index_copy_(2, self._tail_count_dev, value_states)
        self._tail_count_dev.add_(1)
        total = self._pending_tokens() + 1
        self._pending_key = self._tail_key[..., :total, :]
        self._pending_value = self._tail_value[..., :total, :]
        return True

    def prepared_append_ok(self) -> bool:
        """Whether the next one-token append may be written into the tail by the decode-step
        preparation kernel (``dkv_decode_prep``) and committed with ``commit_prepared_append``."""
        return (self._tail_count_dev is not None and self._seen_tokens >= self.config.sink_tokens
                and not self.next_append_seals(1)
                and (self._pending_key is None or self._pending_in_tail()))

    def commit_prepared_append(self) -> None:
        """Account for one token per sequence written at the device tail count: advance the count
        on the device and the host-side state."""
        if not self.prepared_append_ok():
            raise RuntimeError("no prepared one-token append is possible now")
        self._tail_count_dev.add_(1)
        total = self._pending_tokens() + 1
        self._pending_key = self._tail_key[..., :total, :]
        self._pending_value = self._tail_value[..., :total, :]
        self._seen_tokens += 1
        self._layout_version += 1
        self._invalidate_page_descriptors()

    def advance_device_tail(self, tokens: int = 1) -> None:
        """Host-side bookkeeping of ``tokens`` one-token appends replayed on the device."""
        if self._tail_count_dev is None:
            raise RuntimeError("device-side tail counts are not enabled")
        for _ in range(tokens):
            if self.next_append_seals(1):
                raise RuntimeError("a replayed append cannot seal a page")
            total = self._pending_tokens() + 1
            self._pending_key = self._tail_key[..., :total, :]
            self._pending_value = self._tail_value[..., :total, :]
            self._seen_tokens += 1
        self._layout_version += 1
        self._invalidate_page_descriptors()

    # ---- decode plan ----
    def decode_plan(self, device: torch.device) -> _DecodePlan:
        """Device table of segment descriptors for the decode kernel.

        Rebuilt only when the sealed structure changed; the held tail (when it
        lives in the tail buffer) is described per call instead.
        """
        plan = self._decode_plan_cache
        if plan is not None and plan.version == self._sealed_version and plan.device == device:
            return plan
        pairs = self.iter_segments()
        tail_in_pairs = self.config.value_local_tokens == 0 and self._pending_in_tail()
        sealed = pairs[:-1] if tail_in_pairs else pairs
        tail_is_pending = tail_in_pairs or self._tail_count_dev is not None
        keepalive: list = []
        descs = (_lib.Segment * max(1, len(sealed)))()
        n_tokens = 0
        for i, (kseg, vseg) in enumerate(sealed):
            fill_segment(descs[i], kseg, vseg, keepalive)
            n_tokens += descs[i].tokens
        table = None
        if sealed:
            raw = torch.frombuffer(bytearray(bytes(descs)), dtype=torch.uint8)
            table = raw.to(device)
        fast = _fast_run(self, descs, len(sealed))
        rest_dense = _rest_dense(self, descs, len(sealed), fast)
        plan = _DecodePlan(self._sealed_version, device, table, len(sealed), keepalive, tail_is_pending, n_tokens,
                           fast, rest_dense)
        self._decode_plan_cache = plan
        return plan


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------

def _value_rows_job(src: torch.Tensor, bits: int, group: int, meta: torch.dtype, values: torch.Tensor,
                    scale: torch.Tensor, zero: torch.Tensor, nonfinite: int = 0):
    """The C description of quantizing [B,H,T,D] value rows along head_dim.

    A token slice of a [B,H,T',D] tensor is B*H blocks of T contiguous rows;
    the kernel reads it in place.  Other layouts are copied first.  Returns
    (``_lib.ValueRowsArgs``, the source tensor to keep alive until launch).
    ``nonfinite`` is the address of a device uint32 flag (0: no check).
    """
    B, H, T, D = src.shape
    sb, sh, st, sd = src.stride()
    row_stride = st if T > 1 else D
    if sd != 1 or row_stride != D:
        blocks = None
    elif H == 1:
        blocks, block_stride = B, sb
    elif B == 1 or sb == H * sh:
        blocks, block_stride = B * H, sh
    else:
        blocks = None
    if blocks is None:
        src = src.contiguous()
        blocks, block_stride = B * H, T * D
    job = _lib.ValueRowsArgs(src=src.data_ptr(), src_dtype=_lib.dtype_code(src.dtype), blocks=blocks,
                             block_stride=block_stride, block_rows=T, n=D, row_stride=D, bits=bits, group=group,
                             values=values.data_ptr(), scale=scale.data_ptr(), zero=zero.data_ptr(),
                             meta_dtype=_lib.dtype_code(meta), nonfinite=nonfinite or None)
    return job, src


def _launch_value_rows(src: torch.Tensor, bits: int, group: int, meta: torch.dtype, values: torch.Tensor,
                       scale: torch.Tensor, zero: torch.Tensor, nonfinite: int = 0) -> None:
    """Quantize [B,H,T,D] value rows along head_dim (dkv_quantize_value_rows)."""
    job, src = _value_rows_job(src, bits, group, meta, values, scale, zero, nonfinite)
    lib = _lib.load()
    _lib.check(lib.dkv_quantize_value_rows(job, _lib.stream_ptr(src.device)), "dkv_quantize_value_rows")


def _materialize(segment: Segment) -> torch.Tensor:
    return segment if isinstance(segment, torch.Tensor) else segment.dequantize()


def _segment_tokens(segment: Segment) -> int:
    return segment.shape[-2] if isinstance(segment, torch.Tensor) else segment.original_shape[-2]


def _slice_segment(segment: Segment, start: int, stop: int) -> Segment:
    if start == 0 and stop == _segment_tokens(segment):
        return segment
    return _materialize(segment)[..., start:stop, :].contiguous()


def _slice_quantized_tensor(segment: QuantizedTensor, start: int, stop: int) -> QuantizedTensor:
    shape = list(segment.original_shape)
    shape[-2] = stop - start
    return QuantizedTensor(values=segment.values[..., start:stop, :], scale=segment.scale[..., start:stop, :],
                           zero_point=segment.zero_point[..., start:stop, :], original_shape=tuple(shape),
                           original_dim=segment.original_dim, padded_dim=segment.padded_dim,
                           packed_dim=segment.packed_dim, group_size=segment.group_size, bits=segment.bits,
                           output_dtype=segment.output_dtype, axis=segment.axis)


def _merge_quantized_tensors(segments: list) -> QuantizedTensor:
    if not segments:
        raise ValueError("cannot merge an empty quantized segment list")
    ref = segments[0]
    if any((s.original_shape[:-2] != ref.original_shape[:-2] or s.original_dim != ref.original_dim
            or s.padded_dim != ref.padded_dim or s.packed_dim != ref.packed_dim or s.group_size != ref.group_size
            or s.bits != ref.bits or s.output_dtype != ref.output_dtype or s.axis != ref.axis)
           for s in segments[1:]):
        raise ValueError("quantized segments have incompatible layouts")
    shape = list(ref.original_shape)
    shape[-2] = sum(s.original_shape[-2] for s in segments)
    return QuantizedTensor(values=torch.cat([s.values for s in segments], dim=-2),
                           scale=torch.cat([s.scale for s in segments], dim=-2),
                           zero_point=torch.cat([s.zero_point for s in segments], dim=-2),
                           original_shape=tuple(shape), original_dim=ref.original_dim, padded_dim=ref.padded_dim,
                           packed_dim=ref.packed_dim, group_size=ref.group_size, bits=ref.bits,
                           output_dtype=ref.output_dtype, axis=ref.axis)


def _segment_layout(segment: Segment) -> DartSegmentLayout:
    if isinstance(segment, torch.Tensor):
        return DartSegmentLayout("dense", tuple(segment.shape), (("values", tuple(segment.shape), tuple(segment.stride())),))
    if isinstance(segment, QuantizedTensor):
        fields = tuple((name, tuple(t.shape), tuple(t.stride())) for name, t in (
            ("values", segment.values), ("scale", segment.scale), ("zero_point", segment.zero_point)))
        return DartSegmentLayout("quantized", segment.original_shape, fields)
    fields = tuple((name, tuple(t.shape), tuple(t.stride())) for name, t in (
        ("low_values", segment.low_values), ("high_values", segment.high_values),
        ("channel_indices", segment.channel_indices), ("scale", segment.scale), ("zero_point", segment.zero_point)))
    return DartSegmentLayout("mixed_key", segment.original_shape, fields)


def _segment_nbytes(segment: Segment) -> int:
    return segment.numel() * segment.element_size() if isinstance(segment, torch.Tensor) else segment.nbytes


def _descriptor_device(device, fallback: Optional[torch.device]) -> torch.device:
    target = torch.device(device) if device is not None else (fallback or torch.device("cpu"))
    if target.type == "cuda" and target.index is None:
        target = torch.device("cuda", torch.cuda.current_device())
    return target


def _bh_block(t: torch.Tensor, keepalive: list) -> Tuple[int, int]:
    """(address, stride between (batch, head) blocks) of a [B, H, ...] tensor.

    The kernels index block (b, h) at address + (b*H + h) * stride and expect
    the dims after H to be contiguous; other layouts are copied first.
    """
    B, H = t.shape[0], t.shape[1]
    inner = 1
    inner_ok = True
    for size, stride in zip(reversed(t.shape[2:]), reversed(t.stride()[2:])):
        if size != 1 and stride != inner:
            inner_ok = False
        inner *= size
    if H > 1:
        bh = t.stride(1)
        blocks_ok = B == 1 or t.stride(0) == H * bh
    else:
        bh = t.stride(0) if B > 1 else inner
        blocks_ok = True
    if inner_ok and blocks_ok:
        return t.data_ptr(), bh
    c = t.contiguous()
    keepalive.append(c)
    return c.data_ptr(), inner


def _field_block(seg, name: str, keepalive: list) -> Tuple[int, int]:
    """_bh_block of a segment field; a page of a run that has not materialized the field is read
    from the run's tensor directly (no view); empty fields give (0, 0)."""
    run = getattr(seg, "_run", None)
    if run is not None and name not in seg.__dict__:
        blk = run.block(name, seg._page)
        if blk is not None:
            return blk
    t = getattr(seg, name)
    if t.numel() == 0:
        return 0, 0
    return _bh_block(t, keepalive)


def fill_segment(desc, kseg: Segment, vseg: Segment, keepalive: list) -> None:
    """Fill one dkv_segment descriptor from a (key, value) segment pair."""
    keepalive.append((kseg, vseg))
    desc.tokens = _segment_tokens(kseg)
    if isinstance(kseg, torch.Tensor):
        desc.key_kind = _lib.KEY_DENSE
        desc.key[0], desc.key_bh[0] = _dense_block(kseg, keepalive)
    elif isinstance(kseg, MixedQuantizedKey):
        desc.key_kind = _lib.KEY_MIXED
        desc.key_group = kseg.group_size
        desc.promoted = kseg.promoted_channels
        for i, name in enumerate(("low_values", "high_values", "channel_indices", "scale", "zero_point")):
            desc.key[i], desc.key_bh[i] = _field_block(kseg, name, keepalive)
    else:
        if kseg.axis != 2:
            raise ValueError("key pages must be quantized along the token axis")
        desc.key_kind = _lib.KEY_UNIFORM
        desc.key_bits = kseg.bits
        desc.key_group = kseg.group_size
        desc.key[0], desc.key_bh[0] = _field_block(kseg, "values", keepalive)
        desc.key[3], desc.key_bh[3] = _field_block(kseg, "scale", keepalive)
        desc.key[4], desc.key_bh[4] = _field_block(kseg, "zero_point", keepalive)
    if isinstance(vseg, torch.Tensor):
        desc.value_kind = _lib.VALUE_DENSE
        desc.value[0], desc.value_bh[0] = _dense_block(vseg, keepalive)
    else:
        if vseg.axis != 3:
            raise ValueError("value pages must be quantized along head_dim")
        desc.value_kind = _lib.VALUE_UNIFORM
        desc.value_bits = vseg.bits
        desc.value_group = vseg.group_size
        desc.value[0], desc.value_bh[0] = _field_block(vseg, "values", keepalive)
        desc.value[1], desc.value_bh[1] = _field_block(vseg, "scale", keepalive)
        desc.value[2], desc.value_bh[2] = _field_block(vseg, "zero_point", keepalive)


def _dense_block(t: torch.Tensor, keepalive: list) -> Tuple[int, int]:
    """Dense [B,H,T,D] block: rows of D contiguous elements, token stride D."""
    B, H, T, D = t.shape
    if t.stride(-1) == 1 and (t.stride(-2) == D or T == 1):
        if H == 1:
            return t.data_ptr(), t.stride(0)
        if B == 1 or t.stride(0) == H * t.stride(1):
            return t.data_ptr(), t.stride(1)
    c = t.contiguous()
    keepalive.append(c)
    return c.data_ptr(), T * D


def _fast_run(cache: DartKVCache, descs, count: int) -> Tuple[int, int, int, int, int, int]:
    """Longest run of descriptors a page kernel handles:
    (first, count, promoted, value group, key bits, value bits).

    Dart pages (promoted > 0: 2-bit keys with 4-bit promoted channels, 2-bit
    values) go to the lookup-table page kernel; uniform pages (promoted 0:
    2/4/8-bit keys along the tokens in one group per page, 2/4/8-bit values)
    to the arithmetic one.  Both need full 128-token pages, head_dim 128, fp16
    metadata, value groups that are multiples of 16 dividing 128, and every
    block 16-byte aligned per (batch, head)."""
    none = (0, 0, 0, 0, 0, 0)
    if cache.shape is None or cache.dtype not in (torch.bfloat16, torch.float16):
        return none
    c = cache.config
    if (cache.shape[-1] != 128 or c.page_size != 128 or c.metadata_dtype != torch.float16
            or c.resolved_key_group_size != 128):
        return none
    vg = c.resolved_value_group_size
    if vg % 16 or 128 % vg:
        return none
    if c.promote_ratio > 0.0:
        K = promoted_count(128, c.promote_ratio)
        kbits, vbits = 2, c.resolved_value_bits
        if K % 16 or K > 64 or vbits != 2:
            return none
        key_blocks = ((0, 1), (1, 1), (2, 4), (3, 2), (4, 2))  # (descriptor slot, element bytes)
    else:
        K = 0
        kbits, vbits = c.resolved_key_bits, c.resolved_value_bits
        key_blocks = ((0, 1), (3, 2), (4, 2))
    key_kind = _lib.KEY_MIXED if K else _lib.KEY_UNIFORM

    def ok(d) -> bool:
        if not (d.tokens == 128 and d.key_kind == key_kind and d.value_kind == _lib.VALUE_UNIFORM
                and d.key_group == 128 and d.value_bits == vbits and d.value_group == vg):
            return False
        if (d.promoted != K) if K else (d.key_bits != kbits):
            return False
        for i, size in key_blocks:
            if d.key[i] % 16 or (d.key_bh[i] * size) % 16:
                return False
        for i, size in enumerate((1, 2, 2)):
            if d.value[i] % 16 or (d.value_bh[i] * size) % 16:
                return False
        return True

    best = (0, 0)
    i = 0
    while i < count:
        if not ok(descs[i]):
            i += 1
            continue
        j = i
        while j < count and ok(descs[j]):
            j += 1
        if j - i > best[1]:
            best = (i, j - i)
        i = j
    if best[1] == 0:
        return none
    return (best[0], best[1], K, vg, kbits, vbits)


def _dense16_ok(d) -> bool:
    """Dense segment whose K/V rows the dense decode kernel reads with 16-byte loads."""
    return (d.key_kind == _lib.KEY_DENSE and d.value_kind == _lib.VALUE_DENSE and d.key[0] % 16 == 0
            and d.value[0] % 16 == 0 and (d.key_bh[0] * 2) % 16 == 0 and (d.value_bh[0] * 2) % 16 == 0)


def _rest_dense(cache: DartKVCache, descs, count: int, fast: Tuple[int, ...]) -> int:
    """Most tokens of any sealed entry outside the fast run when all of them are
    dense 16-bit with aligned rows and head_dim is 128 (0 if there are none);
    -1 when the dense decode kernel cannot take them."""
    if cache.shape is None or cache.dtype not in (torch.bfloat16, torch.float16) or cache.shape[-1] != 128:
        return -1
    first, n = fast[0], fast[1]
    rest = [descs[i] for i in range(count) if not first <= i < first + n]
    if not all(_dense16_ok(d) for d in rest):
        return -1
    return max((d.tokens for d in rest), default=0)


def tail_segment(cache: DartKVCache):
    """Descriptor of the held tail (pending tokens in the tail buffer).

    With device-side tail counts the descriptor spans the whole tail buffer
    (its capacity) and the kernels read the live count from the device.
    """
    desc = _lib.Segment()
    if cache._tail_count_dev is not None:
        pk, pv = cache._tail_key, cache._tail_value
    elif cache._pending_key is None:
        return desc
    else:
        pk, pv = cache._pending_key, cache._pending_value
    desc.tokens = pk.shape[-2]
    desc.key_kind = _lib.KEY_DENSE
    desc.value_kind = _lib.VALUE_DENSE
    keep: list = []
    desc.key[0], desc.key_bh[0] = _dense_block(pk, keep)
    desc.value[0], desc.value_bh[0] = _dense_block(pv, keep)
    if keep:
        raise RuntimeError("held tail is not in the tail buffer layout")
    return desc


__all__ = ["DartKVCache", "DartKVCacheConfig", "DartPageMetadata", "DartSegmentLayout"]

"""Device page pool: growable storage for the packed pages of one cache.

Key pages are page-major: every packed field is one tensor
``[slots, B, H, ...]`` and a key page is one slot.  Value pages are
token-major: every field is one tensor ``[B, H, rows, ...]`` with one row per
token, so a value page is a run of consecutive rows, and value tokens
quantized a few at a time fill their page in place.  The quantize kernels
write straight into the pool (key pages with a page stride, value rows at a
row offset inside each (batch, head) block), the decode kernels read it
through descriptors, and a run of consecutive pages is a slice of the pool
tensors, never a copy.

Segments are views of a pool (a key slot, or a run of value rows) that
behave as the reference's ``MixedQuantizedKey`` / ``QuantizedTensor``
(reference src/dart/mixed.py:13-35, src/dart/quantization.py:56-76): their
field tensors are read from the pool on access, so they follow the pool when
it grows, moves or has its batch rows reordered.
"""

from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch

from .mixed import MixedQuantizedKey
from .quantization import QuantizedTensor


class FieldRef:
    """A contiguous pool field known by its address, shape and dtype before its tensor view exists:
    enough for a launch (``data_ptr``, ``stride``, ``element_size``), built without any torch call."""

    __slots__ = ("_ptr", "_strides", "_size", "shape")

    def __init__(self, ptr: int, shape: Tuple[int, ...], element_size: int) -> None:
        self._ptr, self.shape, self._size = ptr, shape, element_size
        strides, acc = [], 1
        for n in reversed(shape):
            strides.append(acc)
            acc *= n
        self._strides = tuple(reversed(strides))

    def data_ptr(self) -> int:
        return self._ptr

    def stride(self, dim: int) -> int:
        return self._strides[dim]

    def element_size(self) -> int:
        return self._size


class PagePool:
    """Growable packed storage.  ``fields`` maps a field name to (shape, dtype) with the slot axis
    ``axis`` sized 0; ``batch_axis`` is the batch dimension.  Slots [0, used) hold data.

    A pool's fields share one allocation (each at a 256-byte aligned offset).  Right after it is made,
    only their addresses are known (``ref``): a launch can write them before any tensor view exists,
    and the views (``tensors``) are made on first use, usually while that launch runs."""

    _ALIGN = 256

    def __init__(self, fields: Dict[str, Tuple[Tuple[int, ...], torch.dtype]], axis: int, batch_axis: int,
                 device: torch.device, align: int = 1) -> None:
        self.shapes = {name: tuple(shape) for name, (shape, _) in fields.items()}
        self.dtypes = {name: dtype for name, (_, dtype) in fields.items()}
        self.axis, self.batch_axis, self.align = axis, batch_axis, align
        self.device = device
        self.capacity = 0
        self.used = 0
        self._tensors: Optional[Dict[str, torch.Tensor]] = {}
        self._buffer: Optional[torch.Tensor] = None
        self._layout: Dict[str, Tuple[int, Tuple[int, ...]]] = {}  # name -> (byte offset, full shape)
        self.generation = 0  # bumps whenever the tensors are replaced (field addresses change)

    @property
    def tensors(self) -> Dict[str, torch.Tensor]:
        """The fields as tensors (views of the pool's allocation, made on first use after a resize)."""
        if self._tensors is None:
            views = {}
            with torch.inference_mode(False):  # views updated in place by later calls in any mode
                for name, (offset, full) in self._layout.items():
                    dtype = self.dtypes[name]
                    nbytes = dtype.itemsize
                    for n in full:
                        nbytes *= n
                    views[name] = self._buffer.narrow(0, offset, nbytes).view(dtype).view(full)
            self._tensors = views
        return self._tensors

    def ref(self, name: str):
        """Field ``name`` (all slots) as a tensor, or as a FieldRef while its view is not made yet."""
        if self._tensors is not None:
            return self._tensors[name]
        offset, full = self._layout[name]
        return FieldRef(self._buffer.data_ptr() + offset, full, self.dtypes[name].itemsize)

    @property
    def batch(self) -> int:
        return next(iter(self.shapes.values()))[self.batch_axis]

    def capacity_for(self, n: int, headroom: Optional[int] = None) -> int:
        """The capacity ``reserve(n, headroom)`` grows to when the n slots do not fit."""
        extra = max(self.align, (self.used + n) // 8) if headroom is None else headroom
        cap = self.used + n + extra
        return -(-cap // self.align) * self.align

    def reserve(self, n: int, headroom: Optional[int] = None) -> int:
        """Slots [start, start + n) for new data; grows (copying the used slots) when they do not fit."""
        if self.used + n > self.capacity:
            self._resize(self.capacity_for(n, headroom))
        start = self.used
        self.used += n
        return start

    def plan(self, capacity: int) -> Tuple[Dict[str, Tuple[int, Tuple[int, ...]]], int]:
        """(name -> (byte offset, full shape), bytes) of the fields at ``capacity`` slots."""
        layout, total = {}, 0
        for name, shape in self.shapes.items():
            full = list(shape)
            full[self.axis] = capacity
            nbytes = self.dtypes[name].itemsize
            for n in full:
                nbytes *= n
            layout[name] = (total, tuple(full))
            total += -(-nbytes // self._ALIGN) * self._ALIGN
        return layout, max(total, 1)

    def place(self, buffer: torch.Tensor, layout: Dict[str, Tuple[int, Tuple[int, ...]]], capacity: int) -> None:
        """Take ``buffer`` (uint8, on the pool's device, ``plan(capacity)``'s bytes) as the storage of a
        pool that holds no data yet."""
        if self.used:
            raise RuntimeError("PagePool.place needs an empty pool")
        self._buffer, self._layout, self._tensors, self.capacity = buffer, layout, None, capacity
        self.generation += 1

    def _resize(self, capacity: int) -> None:
        old = self.tensors if self.used else None
        layout, total = self.plan(capacity)
        with torch.inference_mode(False):  # kept and updated in place across calls in any mode
            self._buffer = torch.empty(total, dtype=torch.uint8, device=self.device)
        self._layout, self._tensors, self.capacity = layout, None, capacity
        if old is not None:
            for name, t in self.tensors.items():
                t.narrow(self.axis, 0, self.used).copy_(old[name].narrow(self.axis, 0, self.used))
        self.generation += 1

    def field(self, name: str, at: int, n: Optional[int] = None) -> torch.Tensor:
        """Field ``name`` of slot ``at`` (n None: the slot axis dropped) or of slots [at, at + n)."""
        t = self.tensors[name]
        return t.select(self.axis, at) if n is None else t.narrow(self.axis, at, n)

    def block(self, name: str, at: int) -> Tuple[int, int]:
        """(address of slot ``at``'s (batch 0, head 0) block, elements between consecutive (batch, head)
        blocks) of field ``name``: the form the decode descriptors take."""
        t = self.tensors[name]
        bh = t.stride(self.batch_axis + 1) if t.shape[self.batch_axis + 1] > 1 or t.shape[self.batch_axis] == 1 \
            else t.stride(self.batch_axis)
        return t.data_ptr() + at * t.stride(self.axis) * t.element_size(), bh

    def select_batch(self, index: torch.Tensor) -> None:
        """Keep batch rows ``index`` (a permutation or any selection): bytes are gathered, not recomputed.
        With the batch size unchanged the gather lands in the same tensors, so descriptors stay valid."""
        index = index.to(self.device)
        same = index.numel() == self.batch
        tensors = self.tensors
        with torch.inference_mode(False):  # new pool tensors are kept and updated in place in any mode
            for name, t in list(tensors.items()):
                picked = t.index_select(self.batch_axis, index)
                if same:
                    t.copy_(picked)
                else:
                    tensors[name] = picked
        if not same:
            for name, shape in self.shapes.items():
                s = list(shape)
                s[self.batch_axis] = index.numel()
                self.shapes[name] = tuple(s)
            self._buffer = None  # the fields are now tensors of their own: the old allocation can go
            self.generation += 1

    def to(self, device: torch.device) -> None:
        with torch.inference_mode(False):
            self._tensors = {name: t.to(device) for name, t in self.tensors.items()}
        self._buffer = None  # the views keep what they still use; a copied-out allocation can go
        self.device = device
        self.generation += 1


class _PoolField:
    """A packed field of a pool-backed segment, read from the pool on every access."""

    def __init__(self, name: str) -> None:
        self.name = name

    def __get__(self, obj, cls=None):
        if obj is None:
            return self
        return obj._pool.field(self.name, obj._at, obj._rows)


class PoolMixedKey(MixedQuantizedKey):
    """One Dart key page stored in a key pool slot."""

    low_values = _PoolField("low_values")
    high_values = _PoolField("high_values")
    channel_indices = _PoolField("channel_indices")
    scale = _PoolField("scale")
    zero_point = _PoolField("zero_point")

    def __init__(self, pool: PagePool, slot: int, tokens: int, head_dim: int, padded_tokens: int, group_size: int,
                 promote_bits: int, output_dtype: torch.dtype) -> None:  # pylint: disable=super-init-not-called
        self._pool, self._at, self._rows = pool, slot, None
        self._tokens, self._head_dim = tokens, head_dim
        self.padded_tokens, self.group_size = padded_tokens, group_size
        self.low_bits, self.promote_bits, self.output_dtype = 2, promote_bits, output_dtype

    @property
    def original_shape(self) -> Tuple[int, ...]:
        s = self._pool.shapes["low_values"]
        return (s[1], s[2], self._tokens, self._head_dim)

    def block(self, name: str) -> Tuple[int, int]:
        return self._pool.block(name, self._at)


class PoolKeys(QuantizedTensor):
    """One uniform key page (codes along the tokens) stored in a key pool slot."""

    values = _PoolField("values")
    scale = _PoolField("scale")
    zero_point = _PoolField("zero_point")

    def __init__(self, pool: PagePool, slot: int, tokens: int, head_dim: int, padded_dim: int, packed_dim: int,
                 group_size: int, bits: int, output_dtype: torch.dtype) -> None:  # pylint: disable=super-init-not-called
        self._pool, self._at, self._rows = pool, slot, None
        self._head_dim = head_dim
        self.original_dim, self.padded_dim, self.packed_dim = tokens, padded_dim, packed_dim
        self.group_size, self.bits, self.output_dtype, self.axis = group_size, bits, output_dtype, 2

    @property
    def original_shape(self) -> Tuple[int, ...]:
        s = self._pool.shapes["values"]
        return (s[1], s[2], self.original_dim, self._head_dim)

    def block(self, name: str) -> Tuple[int, int]:
        return self._pool.block(name, self._at)


class PoolValues(QuantizedTensor):
    """Value rows [row0, row0 + rows) of a value pool: one value segment (codes along head_dim)."""

    values = _PoolField("values")
    scale = _PoolField("scale")
    zero_point = _PoolField("zero_point")

    def __init__(self, pool: PagePool, row0: int, rows: int, head_dim: int, padded_dim: int, packed_dim: int,
                 group_size: int, bits: int, output_dtype: torch.dtype) -> None:  # pylint: disable=super-init-not-called
        self._pool, self._at, self._rows = pool, row0, rows
        self.original_dim, self.padded_dim, self.packed_dim = head_dim, padded_dim, packed_dim
        self.group_size, self.bits, self.output_dtype, self.axis = group_size, bits, output_dtype, 3

    @property
    def original_shape(self) -> Tuple[int, ...]:
        s = self._pool.shapes["values"]
        return (s[0], s[1], self._rows, self.original_dim)

    def rows(self, start: int, count: int) -> "PoolValues":
        """The segment's rows [start, start + count) as a segment of their own."""
        return PoolValues(self._pool, self._at + start, count, self.original_dim, self.padded_dim, self.packed_dim,
                          self.group_size, self.bits, self.output_dtype)

    def block(self, name: str) -> Tuple[int, int]:
        return self._pool.block(name, self._at)


__all__ = ["PagePool", "PoolMixedKey", "PoolKeys", "PoolValues"]

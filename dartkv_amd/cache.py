"""Append-only compressed KV cache whose pages live in a device page pool.

The observable lifecycle is the reference ``DartKVCache``'s (reference
src/dart/cache.py:45-661): a dense sink prefix, page-sized quantization,
held partial pages, Kitty local / value-local windows, value pages that grow
token-wise up to a page, and segments cut at the union of the key and value
boundaries.  How it is stored is this build's own:

* packed pages live in two growable device pools (``pool.PagePool``): key
  pages page-major, one slot per page; value pages token-major, one row per
  token.  Every page of one append is quantized by one key launch that also
  quantizes the values, straight into the pools; a value page that grows
  token-wise is a run of consecutive pool rows, filled in place;
* the held partial page lives in a preallocated tail buffer, so a one-token
  decode append is one device copy;
* the (key, value) segment list is rebuilt only when a page is sealed, and the
  device descriptor table the decode kernels read (with the page directory
  ``page_table()`` views) is built once per sealed layout;
* batch reordering (beam search) gathers the packed bytes along the batch
  axis; nothing is quantized again.
"""

from __future__ import annotations

import contextlib
import ctypes
import threading
import time
from dataclasses import dataclass, fields as dataclass_fields
from itertools import accumulate
from typing import TYPE_CHECKING, List, Optional, Tuple, Union

import torch

from . import _lib
from .mixed import MixedQuantizedKey, launch_key_pages, promoted_count, random_channels
from .pool import PagePool, PoolKeys, PoolMixedKey, PoolValues
from .quantization import QuantizedTensor

if TYPE_CHECKING:
    from .page_table import DartPageTable

Segment = Union[torch.Tensor, QuantizedTensor, MixedQuantizedKey]


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
        # the field values as one tuple: a cheap dictionary key for plans made per configuration
        object.__setattr__(self, "_key", tuple(getattr(self, f.name) for f in dataclass_fields(self)))

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


_flag_store = threading.local()


def _nonfinite_flags(device: torch.device) -> torch.Tensor:
    """int32 [2] flags (keys, values) for the quantizers' non-finite reports on ``device``, one pair per
    thread and device and shared by that thread's caches (an append's scope reads them before the next
    append can start on the thread).  They live in pinned host memory, which the kernels write directly:
    reading them after the append's launches takes a stream synchronization and no device-to-host copy.
    They are zero between appends."""
    flags = getattr(_flag_store, "flags", None)
    if flags is None:
        flags = _flag_store.flags = {}
    t = flags.get(device)
    if t is None:
        with torch.inference_mode(False):  # updated in place whatever mode a later append runs in
            t = flags[device] = torch.zeros(2, dtype=torch.int32, pin_memory=True)
    return t


_DRAIN_SPIN_S = 1e-3  # poll this long, then block (a long append does not keep a CPU core busy)


def _drain(device: torch.device) -> None:
    """Wait until the device's current stream has run everything enqueued so far, by polling an event
    recorded on it: the wait ends within a few microseconds of the GPU finishing, where a blocking
    stream synchronization returns about 10-15 µs later (measured on MI355X).  Work still running
    after ``_DRAIN_SPIN_S`` of polling is waited for with a blocking synchronization."""
    events = getattr(_flag_store, "events", None)
    if events is None:
        events = _flag_store.events = {}
    ev = events.get(device)
    if ev is None:
        ev = events[device] = torch.cuda.Event()
    ev.record(torch.cuda.current_stream(device))
    t0 = time.perf_counter()
    while not ev.query():
        if time.perf_counter() - t0 > _DRAIN_SPIN_S:
            ev.synchronize()
            return


def _storage(shape, dtype: torch.dtype, device) -> torch.Tensor:
    """Uninitialized storage a cache keeps and updates in place across calls.  It is allocated as a
    normal tensor even inside ``torch.inference_mode()`` (an inference tensor could not be updated in
    place by a later call made outside that mode)."""
    with torch.inference_mode(False):
        return torch.empty(shape, dtype=dtype, device=device)


class _FiniteScope:
    """Bookkeeping of one append's non-finite check: the flags once a quantize launch uses them, and
    what a failed check restores.  Within an append the tracks only grow, or change their last
    element (a value page filled further, a key page packed again), so their lengths and last
    elements are a complete snapshot."""

    __slots__ = ("flags", "tracks", "pools", "pending", "undo")

    def __init__(self, cache: "DartKVCache") -> None:
        self.flags: Optional[torch.Tensor] = None
        self.tracks = [(len(t), t[-1] if t else None) for t in (cache._keys, cache._values)]
        self.pools = [(p, p.used) for p in (cache._key_pool, cache._value_pool) if p is not None]
        self.pending = (cache._pending_key, cache._pending_value)
        self.undo: list = []

    def restore(self, cache: "DartKVCache") -> None:
        for fn in reversed(self.undo):
            fn()
        cache._keys, cache._values = [self._trimmed(track, *t) for track, t in
                                      zip((cache._keys, cache._values), self.tracks)]
        known = [p for p, _ in self.pools]
        for pool, used in self.pools:
            pool.used = used
        for pool in (cache._key_pool, cache._value_pool):  # pools first created by this append
            if pool is not None and all(pool is not p for p in known):
                pool.used = 0
        cache._pending_key, cache._pending_value = self.pending
        cache._sealed_version += 1
        if cache._tail_count_dev is not None:
            cache._tail_count_dev.fill_(cache._pending_tokens())

    @staticmethod
    def _trimmed(track: list, n: int, last) -> list:
        kept = track[:max(0, n - 1)]
        return kept + [last] if n else kept


class _PrefillPlan:
    """What the first append of an empty cache (``DartKVCache._prefill``) needs that depends only on
    the configuration and the inputs' shape, strides, dtype and device: the token split (dense sink,
    full pages, held tail), the pools' fields, capacities and layouts, and the library arguments with
    every address left to fill in (offsets into the sources, pools and dense buffer instead).  The
    capacities are those the general path's reserve calls make, so later appends grow the pools at the
    same points."""

    __slots__ = ("B", "H", "T", "D", "sink", "sealable", "pending", "n_pages", "mixed", "key_group",
                 "key_groups", "key_bits", "key_packed", "value_group", "value_bits", "value_padded",
                 "value_packed", "key_fields", "value_fields", "key_layout", "key_bytes", "key_capacity",
                 "value_layout", "value_bytes", "value_capacity", "key_offsets", "value_offsets", "row",
                 "sink_bytes", "tail_capacity", "tail_bytes", "dense_bytes", "key_src", "value_src", "key_args",
                 "value_args", "copies", "copy_type", "copy_blocks")

    @staticmethod
    def build(c: DartKVCacheConfig, key_states: torch.Tensor, value_states: torch.Tensor):
        """The plan, or False where the general path must run: a Kitty value window, a random channel
        choice, nothing to seal, a short last page, inputs whose last dim is not contiguous, or a value
        layout the rows kernel cannot read in place."""
        if c.value_local_tokens or key_states.stride(-1) != 1 or value_states.stride(-1) != 1:
            return False
        B, H, T, D = key_states.shape
        P = c.page_size
        sink = min(c.sink_tokens, T)
        rest = T - sink
        held = c.hold_partial_pages or c.local_tokens
        sealable = (max(0, rest - c.local_tokens) // P) * P if held else rest
        pending = rest - sealable
        if sealable == 0 or sealable % P or pending > P + c.local_tokens:
            return False
        mixed = c.promote_ratio > 0.0
        K = promoted_count(D, c.promote_ratio) if mixed else 0
        if mixed and c.channel_selection == "random" and 0 < K < D:
            return False
        vsb, vsh, vst, _ = value_states.stride()
        if sealable > 1 and vst != D:
            return False
        if H == 1:
            vblocks, vblock_stride = B, vsb
        elif B == 1 or vsb == H * vsh:
            vblocks, vblock_stride = B * H, vsh
        else:
            return False
        self = _PrefillPlan()
        self.B, self.H, self.T, self.D = B, H, T, D
        self.sink, self.sealable, self.pending, self.n_pages = sink, sealable, pending, sealable // P
        kg, vg, meta = c.resolved_key_group_size, c.resolved_value_group_size, c.metadata_dtype
        kb, vb = c.resolved_key_bits, c.resolved_value_bits
        groups = -(-P // kg)
        self.mixed, self.key_group, self.key_groups, self.key_bits = mixed, kg, groups, kb
        self.value_group, self.value_bits = vg, vb
        # the pools _key_pool_for / _value_pool_for make, at the capacities their first reserve gives
        if mixed:
            nb = (kg + 3) // 4
            self.key_fields = {"low_values": ((0, B, H, D, groups, nb), torch.uint8),
                               "high_values": ((0, B, H, K, groups, nb if K else nb * 4), torch.uint8),
                               "channel_indices": ((0, B, H, K), torch.int32),
                               "scale": ((0, B, H, D, groups), meta), "zero_point": ((0, B, H, D, groups), meta)}
            names = ("low_values", "high_values", "channel_indices", "scale", "zero_point")
        else:
            kpacked = -(-groups * kg // (8 // kb))
            self.key_fields = {"values": ((0, B, H, D, kpacked), torch.uint8),
                               "scale": ((0, B, H, D, groups), meta), "zero_point": ((0, B, H, D, groups), meta)}
            names = ("values", None, None, "scale", "zero_point")
            self.key_packed = kpacked * (8 // kb)
        vgroups = -(-D // vg)
        vpacked = -(-vgroups * vg // (8 // vb))
        self.value_fields = {"values": ((B, H, 0, vpacked), torch.uint8), "scale": ((B, H, 0, vgroups), meta),
                             "zero_point": ((B, H, 0, vgroups), meta)}
        self.value_padded, self.value_packed = vgroups * vg, vpacked * (8 // vb)
        kpool = PagePool(self.key_fields, axis=0, batch_axis=1, device=key_states.device)
        vpool = PagePool(self.value_fields, axis=2, batch_axis=0, device=key_states.device, align=64)
        self.key_capacity = kpool.capacity_for(self.n_pages, max(2, self.n_pages // 16))
        self.value_capacity = vpool.capacity_for(sealable, max(vpool.align, sealable // 16))
        self.key_layout, self.key_bytes = kpool.plan(self.key_capacity)
        self.value_layout, self.value_bytes = vpool.plan(self.value_capacity)
        self.key_offsets = tuple(0 if n is None else self.key_layout[n][0] for n in names)
        self.value_offsets = tuple(self.value_layout[n][0] for n in ("values", "scale", "zero_point"))
        # the dense buffer: sink keys, sink values, tail keys, tail values (each 256-byte aligned)
        e = key_states.element_size()
        row = self.row = D * e
        self.sink_bytes = -(-B * H * sink * row // 256) * 256
        self.tail_capacity = P + c.local_tokens if pending else 0
        self.tail_bytes = -(-B * H * self.tail_capacity * row // 256) * 256
        self.dense_bytes = 2 * (self.sink_bytes + self.tail_bytes)
        ksb, ksh, kst, ksd = key_states.stride()
        self.key_src, self.value_src = sink * kst * e, sink * vst * e
        v = _lib.ValueRowsArgs(src_dtype=_lib.dtype_code(value_states.dtype), blocks=vblocks,
                               block_stride=vblock_stride, block_rows=sealable, n=D, row_stride=D, bits=vb, group=vg,
                               meta_dtype=_lib.dtype_code(meta), out_block_rows=self.value_capacity, out_row0=0)
        self.value_args = bytes(v)
        a = _lib.KeyPagesArgs()
        a.src_dtype = _lib.dtype_code(key_states.dtype)
        a.B, a.H, a.D, a.page_tokens, a.n_pages = B, H, D, P, self.n_pages
        a.sb, a.sh, a.st, a.sd = ksb, ksh, kst, ksd
        a.group, a.meta_dtype = kg, _lib.dtype_code(meta)
        if mixed:
            a.key_mode, a.bits, a.promoted = _lib.KEY_MIXED, 2, K
            a.selection = _lib.SELECT_VARIANCE if c.channel_selection == "variance" else _lib.SELECT_MAGNITUDE
        else:
            a.key_mode, a.bits = _lib.KEY_UNIFORM, kb
        if self.n_pages > 1:
            for attr, name in zip(("low", "high", "idx", "scale", "zero"), names):
                if name is not None:
                    _, full = self.key_layout[name]
                    stride = self.key_fields[name][1].itemsize
                    for n in full[1:]:
                        stride *= n
                    setattr(a, attr + "_page_stride", stride)
        self.key_args = bytes(a)
        # the copies: (source byte offset, dense byte offset, from the values) and their fixed fields
        runs = ([(0, sink, sink, 0, self.sink_bytes)] if sink else []) + \
            ([(sink + sealable, pending, self.tail_capacity, 2 * self.sink_bytes,
               2 * self.sink_bytes + self.tail_bytes)] if pending else [])
        self.copy_type = _lib.CopyBlock * max(1, 2 * len(runs))
        blocks = self.copy_type()
        self.copies = []
        for t0, count, cap, koff, voff in runs:
            for from_values, (sb, sh, st), off in ((False, (ksb, ksh, kst), koff), (True, (vsb, vsh, vst), voff)):
                blk = blocks[len(self.copies)]
                blk.B, blk.H, blk.T, blk.row_bytes = B, H, count, row
                blk.src_sb, blk.src_sh, blk.src_st = sb * e, sh * e, st * e
                blk.dst_sb, blk.dst_sh, blk.dst_st = H * cap * row, cap * row, row
                self.copies.append((t0 * st * e, off, from_values))
        self.copies = tuple(self.copies)
        self.copy_blocks = bytes(blocks)
        return self


# prefill plans by (config fields, key shape, key strides, value strides, dtype, device)
_PREFILL_PLANS: dict = {}


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
        self.host_table = None  # the descriptors in host memory (dkv_decode_args.segments_host)
        self.call_layouts: dict = {}  # decode call shape -> (DecodeArgs template, workspace bytes)


class DartKVCache:
    """Append-only KV cache over HIP-quantized pages (reference cache.py:115-542).

    Inputs and returned tensors use ``[batch, kv_heads, sequence, head_dim]``
    on a ROCm device.  The cache owns detached copies of appended tensors.
    """

    def __init__(self, config: Optional[DartKVCacheConfig] = None) -> None:
        self.config = config or DartKVCacheConfig()
        # the key and the value track: segments in sequence order (dense tensors or pool views)
        self._keys: List[Segment] = []
        self._values: List[Segment] = []
        self._pending_key: Optional[torch.Tensor] = None
        self._pending_value: Optional[torch.Tensor] = None
        self._shape: Optional[Tuple[int, int, int]] = None
        self._dtype: Optional[torch.dtype] = None
        self._device: Optional[torch.device] = None
        self._seen_tokens = 0
        self._layout_version = 0
        # bumps when anything but the held tail changes; segment lists and descriptors follow it
        self._sealed_version = 0
        self._key_pool: Optional[PagePool] = None
        self._value_pool: Optional[PagePool] = None
        self._value_job = None  # a value-row launch waiting for the key launch of the same tokens
        self._tail_key: Optional[torch.Tensor] = None
        self._tail_value: Optional[torch.Tensor] = None
        self._tail_count_dev: Optional[torch.Tensor] = None  # held tail length on the device (graph replay)
        self._finite_scope: Optional[_FiniteScope] = None
        self._copy_queue: Optional[list] = None  # an append's dense token copies, launched once at its end
        self._tail_job: Optional[tuple] = None  # _tail_copy_job of the current tail buffers
        self._tail_desc = None  # [tail tensors' addresses and strides, descriptor, dense check, tokens, with them]
        self._sealed_pairs_cache: Optional[Tuple[int, list]] = None
        self._directory_cache: dict = {}
        self._decode_plan_cache: Optional[_DecodePlan] = None
        self._page_table_cache: dict = {}
        self._page_run_cache: dict = {}

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
        if self._extend_tail(key_states, value_states):
            return
        _lib.require_device(key_states, value_states)
        self._validate_inputs(key_states, value_states)
        if self._seen_tokens == 0 and self._prefill(key_states, value_states):
            return
        key_states = key_states.detach()
        value_states = value_states.detach()
        if key_states.stride(-1) != 1:
            key_states = key_states.contiguous()
        if value_states.stride(-1) != 1:
            value_states = value_states.contiguous()
        chunk = key_states.shape[-2]
        sink = min(max(0, self.config.sink_tokens - self._seen_tokens), chunk)
        with self._finite_inputs():
            at_keys, at_values = len(self._keys), len(self._values)
            self._copy_queue = []
            try:
                if sink < chunk:
                    keys, values = key_states[..., sink:, :], value_states[..., sink:, :]
                    if not self._device_tail_append(keys, values):
                        if self._tail_count_dev is not None and torch.cuda.is_current_stream_capturing():
                            raise RuntimeError("a captured append may only extend the held tail by one token")
                        self._append_tokens(keys, values)
                        self._sync_device_tail()
                if sink:
                    # the dense sink tokens precede this append's pages (every earlier token is a sink
                    # token too); they are copied after the quantize launches, which then start sooner
                    ks, vs = key_states[..., :sink, :], value_states[..., :sink, :]
                    kd = _storage(ks.shape, ks.dtype, ks.device)
                    vd = _storage(vs.shape, vs.dtype, vs.device)
                    self._copy_tokens((kd, ks), (vd, vs))
                    self._keys.insert(at_keys, kd)
                    self._values.insert(at_values, vd)
                    self._sealed_version += 1
                copies = self._copy_queue
            finally:
                self._copy_queue = None
            if copies:
                _lib.copy_token_blocks(copies, self._device)
        self._seen_tokens += chunk
        self._layout_version += 1
        self._invalidate_page_descriptors()

    def _prefill(self, key_states: torch.Tensor, value_states: torch.Tensor) -> bool:
        """The first append of an empty cache (a prefill) in few host steps: the dense sink, full pages
        and held tail of the general path from one library call that quantizes the pages' keys and values
        and copies the sink and tail tokens, with every output allocated and described before it (from a
        plan kept per configuration and input layout) and the segment objects made while it runs.  Same
        result as the general path; False (nothing done) when the plan does not apply, and the general
        path then runs.  Inputs are validated."""
        if (self._keys or self._values or self._key_pool is not None or self._value_pool is not None
                or self._tail_key is not None or self._tail_count_dev is not None or self._pending_key is not None
                or self._pending_value is not None):
            return False
        device = key_states.device
        key = (self.config._key, key_states.shape, key_states.stride(), value_states.stride(), key_states.dtype,
               device)
        plan = _PREFILL_PLANS.get(key)
        if plan is None:
            plan = _PrefillPlan.build(self.config, key_states, value_states)
            if len(_PREFILL_PLANS) >= 32:
                _PREFILL_PLANS.clear()
            _PREFILL_PLANS[key] = plan
        if plan is False:
            return False
        c = self.config
        with self._finite_inputs():  # (a failed check finds the pools made here and empties them)
            kpool = self._key_pool = PagePool(plan.key_fields, axis=0, batch_axis=1, device=device)
            vpool = self._value_pool = PagePool(plan.value_fields, axis=2, batch_axis=0, device=device, align=64)
            normal = torch.is_inference_mode_enabled()
            with torch.inference_mode(False) if normal else contextlib.nullcontext():
                # kept and updated in place by later calls in any mode
                kbuf = torch.empty(plan.key_bytes, dtype=torch.uint8, device=device)
                vbuf = torch.empty(plan.value_bytes, dtype=torch.uint8, device=device)
                dense = torch.empty(plan.dense_bytes, dtype=torch.uint8, device=device) if plan.dense_bytes else None
            kpool.place(kbuf, plan.key_layout, plan.key_capacity)
            vpool.place(vbuf, plan.value_layout, plan.value_capacity)
            kpool.used, vpool.used = plan.n_pages, plan.sealable
            a = _lib.KeyPagesArgs.from_buffer_copy(plan.key_args)
            v = _lib.ValueRowsArgs.from_buffer_copy(plan.value_args)
            kptr, vptr = key_states.data_ptr(), value_states.data_ptr()
            a.src, v.src = kptr + plan.key_src, vptr + plan.value_src
            kbase, vbase = kbuf.data_ptr(), vbuf.data_ptr()
            a.low = kbase + plan.key_offsets[0]
            if plan.mixed:
                a.high, a.idx = kbase + plan.key_offsets[1], kbase + plan.key_offsets[2]
            a.scale, a.zero = kbase + plan.key_offsets[3], kbase + plan.key_offsets[4]
            v.values = vbase + plan.value_offsets[0]
            v.scale, v.zero = vbase + plan.value_offsets[1], vbase + plan.value_offsets[2]
            v.nonfinite = self._flag_ptr(1)
            a.nonfinite = self._flag_ptr(0)
            a.values = ctypes.addressof(v)
            if plan.copies:
                copies = plan.copy_type.from_buffer_copy(plan.copy_blocks)
                dptr = dense.data_ptr()
                for blk, (src_off, dst_off, from_values) in zip(copies, plan.copies):
                    blk.src, blk.dst = (vptr if from_values else kptr) + src_off, dptr + dst_off
                a.copies, a.n_copies = ctypes.addressof(copies), len(plan.copies)
            _lib.check(_lib.load().dkv_quantize_key_pages(a, _lib.stream_ptr(device)), "dkv_quantize_key_pages")
            # the segments, while the launches run
            P, D, dtype, kg, vg = c.page_size, plan.D, key_states.dtype, plan.key_group, plan.value_group
            padded = plan.key_groups * kg
            if plan.mixed:
                keys = [PoolMixedKey(kpool, p, P, D, padded, kg, c.promote_bits, dtype) for p in range(plan.n_pages)]
            else:
                kb = plan.key_bits
                keys = [PoolKeys(kpool, p, P, D, padded, plan.key_packed, kg, kb, dtype) for p in range(plan.n_pages)]
            vb, vpadded, vpacked = plan.value_bits, plan.value_padded, plan.value_packed
            values = [PoolValues(vpool, i * P, P, D, vpadded, vpacked, vg, vb, dtype) for i in range(plan.n_pages)]
            self._sealed_version += 1
            if dense is not None:
                B, H = plan.B, plan.H
                with torch.inference_mode(False) if normal else contextlib.nullcontext():
                    if plan.sink:
                        n = B * H * plan.sink * plan.row
                        keys.insert(0, dense.narrow(0, 0, n).view(dtype).view(B, H, plan.sink, D))
                        values.insert(0, dense.narrow(0, plan.sink_bytes, n).view(dtype).view(B, H, plan.sink, D))
                        self._sealed_version += 1
                    if plan.pending:
                        at, cap = 2 * plan.sink_bytes, plan.tail_capacity
                        n = B * H * cap * plan.row
                        self._tail_key = dense.narrow(0, at, n).view(dtype).view(B, H, cap, D)
                        self._tail_value = dense.narrow(0, at + plan.tail_bytes, n).view(dtype).view(B, H, cap, D)
                        self._pending_key = self._tail_key.narrow(2, 0, plan.pending)
                        self._pending_value = self._tail_value.narrow(2, 0, plan.pending)
            self._keys, self._values = keys, values
        self._seen_tokens += plan.T
        self._layout_version += 1
        self._invalidate_page_descriptors()
        return True

    def get(self) -> Tuple[torch.Tensor, torch.Tensor]:
        if self._seen_tokens == 0:
            raise RuntimeError("DartKVCache is empty; call update() before get()")
        keys = [_materialize(s) for s in self._keys]
        values = [_materialize(s) for s in self._values]
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
        pending = sum(t.numel() * t.element_size() for t in (self._pending_key, self._pending_value) if t is not None)
        return sum(_segment_nbytes(s) for s in (*self._keys, *self._values)) + pending

    @property
    def dense_bytes(self) -> int:
        if self._shape is None or self._dtype is None:
            return 0
        batch, heads, head_dim = self._shape
        return 2 * batch * heads * self._seen_tokens * head_dim * torch.tensor([], dtype=self._dtype).element_size()

    @property
    def compression_ratio(self) -> float:
        return self.dense_bytes / self.storage_bytes if self.storage_bytes else 1.0

    # ---- segments and descriptors ----
    def _tail_resident(self) -> bool:
        """The pending tokens sit in the tail buffer and are described per call, not in the sealed layout."""
        return self.config.value_local_tokens == 0 and self._pending_in_tail()

    def _sealed_pairs(self) -> list:
        """(key, value) segments of everything but a tail-resident pending tail, cut at the union of the two
        tracks' boundaries; built once per sealed layout."""
        cached = self._sealed_pairs_cache
        if cached is not None and cached[0] == self._sealed_version:
            return cached[1]
        keys, values = list(self._keys), list(self._values)
        if not self._tail_resident():
            if self._pending_key is not None:
                if self._pending_value is None:
                    raise RuntimeError("DartKVCache has a pending key without a pending value")
                keys.append(self._pending_key)
            if self._pending_value is not None:
                values.append(self._pending_value)
        pairs = _union_pairs(keys, values)
        self._sealed_pairs_cache = (self._sealed_version, pairs)
        return pairs

    def iter_segments(self) -> list:
        """K/V segments in sequence order over the union of their boundaries (reference cache.py:229-274).

        Where a union piece covers only part of a packed segment, that part is returned dequantized."""
        pairs = list(self._sealed_pairs())
        if self._tail_resident():
            pairs.append((self._pending_key, self._pending_value))
        return pairs

    def page_metadata(self) -> list:
        """Page order, logical lengths, shapes and element strides (reference cache.py:276-300)."""
        out, start = [], 0
        for index, (kseg, vseg) in enumerate(self.iter_segments()):
            n = _segment_tokens(kseg)
            if _segment_tokens(vseg) != n:
                raise RuntimeError("DartKVCache key/value page lengths diverged")
            out.append(DartPageMetadata(index=index, sequence_start=start, token_count=n, key=_segment_layout(kseg),
                                        value=_segment_layout(vseg)))
            start += n
        if start != self._seen_tokens:
            raise RuntimeError(f"page metadata covers {start} tokens, expected {self._seen_tokens}")
        return out

    def _directory(self, device: torch.device) -> torch.Tensor:
        """int32 [N, 4] page directory on ``device``: (sequence start, tokens, key mode, value mode) per
        segment of ``iter_segments()``.  The sealed rows are built once per sealed layout; the held tail's
        row is added per call."""
        cached = self._directory_cache.get(device)
        if cached is None or cached[0] != self._sealed_version:
            rows, start = [], 0
            for kseg, vseg in self._sealed_pairs():
                n = _segment_tokens(kseg)
                rows.append((start, n, _page_mode(kseg), _page_mode(vseg)))
                start += n
            table = torch.tensor(rows, dtype=torch.int32).reshape(len(rows), 4).to(device)
            cached = (self._sealed_version, table, start)
            self._directory_cache = {device: cached}
        _, table, start = cached
        if self._tail_resident():
            tail = torch.tensor([[start, self._pending_key.shape[-2], 0, 0]], dtype=torch.int32).to(device)
            table = torch.cat((table, tail))
            start += self._pending_key.shape[-2]
        if start != self._seen_tokens:
            raise RuntimeError(f"page table covers {start} tokens, expected {self._seen_tokens}")
        return table

    def page_table(self, *, device=None, rebuild: bool = False) -> "DartPageTable":
        """Page descriptors, one object per layout version and device (reference cache.py:302-323).

        The table's arrays are views of the cache's page directory."""
        from .page_table import DartPageTable

        target = _descriptor_device(device, self._device)
        cached = self._page_table_cache.get(target)
        if cached is not None and not rebuild and cached[0] == self._layout_version:
            return cached[1]
        table = DartPageTable.from_cache(self, device=target)
        self._page_table_cache[target] = (self._layout_version, table)
        return table

    def page_runs(self, *, device=None, page_table=None, rebuild: bool = False) -> tuple:
        """Runs of consecutive full uniform pages, page-major (reference cache.py:325-352).

        Runs are slices of the page pool; a run is stacked (copied) only where its pages are not
        consecutive pool slots."""
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

    def uniform_page_runs(self, table: "DartPageTable") -> tuple:
        """The ``DartPageRun``s ``table`` describes over this cache's pages (``DartPageTable.uniform_quantized_runs``)."""
        from .page_table import DartPageRun

        pairs = self.iter_segments()
        if len(pairs) != table.page_count or self._seen_tokens != table.seen_tokens:
            raise ValueError("cache and page_table describe different page lifecycles")
        page = self.config.page_size
        full = [_full_uniform(k, v, page) for k, v in pairs]
        runs, i = [], 0
        while i < len(pairs):
            if not full[i]:
                i += 1
                continue
            j = i + 1
            while j < len(pairs) and full[j] and _same_run_layout(pairs[i], pairs[j]):
                j += 1
            keys, values = [p[0] for p in pairs[i:j]], [p[1] for p in pairs[i:j]]
            kf = _run_fields(keys, ("values", "scale", "zero_point"), page_major=True)
            vf = _run_fields(values, ("values", "scale", "zero_point"), page_major=False)
            dev = kf[0].device
            runs.append(DartPageRun(
                first_page_index=i, page_indices=table.page_ids[0, i:j].to(dev),
                sequence_starts=table.sequence_starts[i:j].to(dev), token_counts=table.token_counts[i:j].to(dev),
                key_values=kf[0], key_scale=kf[1], key_zero_point=kf[2],
                value_values=vf[0], value_scale=vf[1], value_zero_point=vf[2],
                key_bits=keys[0].bits, value_bits=values[0].bits, key_group_size=keys[0].group_size,
                value_group_size=values[0].group_size, page_size=page).validate())
            i = j
        return tuple(runs)

    def to(self, device) -> "DartKVCache":
        """Move backing tensors to ``device`` (reference cache.py:354-366)."""
        target = _descriptor_device(device, self._device)
        for pool in self._pools():
            pool.to(target)
        self._keys = [s.to(target) if isinstance(s, torch.Tensor) else s for s in self._keys]
        self._values = [s.to(target) if isinstance(s, torch.Tensor) else s for s in self._values]
        if self._pending_key is not None:
            self._pending_key = self._pending_key.to(target)
        if self._pending_value is not None:
            self._pending_value = self._pending_value.to(target)
        self._tail_key = self._tail_value = None
        self._tail_job = None
        self._tail_count_dev = None
        self._device = target
        self._layout_version += 1
        self._sealed_version += 1
        self._invalidate_page_descriptors()
        return self

    def clear(self) -> None:
        self._keys, self._values = [], []
        self._pending_key = self._pending_value = None
        self._key_pool = self._value_pool = None
        self._tail_key = self._tail_value = None
        self._tail_job = None
        self._shape = None
        self._dtype = None
        self._device = None
        self._seen_tokens = 0
        self._layout_version += 1
        self._sealed_version += 1
        self._decode_plan_cache = None
        self._directory_cache = {}
        self._tail_count_dev = None
        self._invalidate_page_descriptors()

    def reorder_batch(self, indices) -> None:
        """Keep batch rows ``indices`` in that order (beam reordering, batch selection, repeats).

        Every packed and dense tensor is gathered along its batch axis: the packed bytes are unchanged
        and nothing is quantized again (the reference re-quantizes dequantized rows,
        integrations/huggingface.py:117-127).  With the batch size unchanged the pools and the tail
        buffer are gathered in place, so descriptors and captured decode graphs stay valid."""
        if self._shape is None:
            return
        index = torch.as_tensor(indices, device=self._device)
        if index.dtype == torch.bool:
            index = index.nonzero().flatten()
        index = index.to(torch.long).flatten()
        batch = self._shape[0]
        if index.numel() and bool(((index < 0) | (index >= batch)).any()):
            raise IndexError("batch indices contain an invalid batch row")
        same = index.numel() == batch
        for pool in self._pools():
            pool.select_batch(index)
        self._keys = [s.index_select(0, index) if isinstance(s, torch.Tensor) else s for s in self._keys]
        self._values = [s.index_select(0, index) if isinstance(s, torch.Tensor) else s for s in self._values]
        in_tail = self._pending_in_tail()
        if self._tail_key is not None:
            if same:
                self._tail_key.copy_(self._tail_key.index_select(0, index))
                self._tail_value.copy_(self._tail_value.index_select(0, index))
            else:
                with torch.inference_mode(False):  # kept and updated in place by later calls
                    self._tail_key = self._tail_key.index_select(0, index)
                    self._tail_value = self._tail_value.index_select(0, index)
                self._tail_job = None
        if in_tail:
            n = self._pending_key.shape[-2]
            self._pending_key, self._pending_value = self._tail_key[..., :n, :], self._tail_value[..., :n, :]
        else:
            if self._pending_key is not None:
                self._pending_key = self._pending_key.index_select(0, index)
            if self._pending_value is not None:
                self._pending_value = self._pending_value.index_select(0, index)
        self._shape = (index.numel(), self._shape[1], self._shape[2])
        self._layout_version += 1
        self._sealed_version += 1
        self._invalidate_page_descriptors()

    def _pools(self) -> list:
        pools = {id(p): p for p in (self._key_pool, self._value_pool) if p is not None}
        for seg in (*self._keys, *self._values):
            pool = getattr(seg, "_pool", None)
            if pool is not None:
                pools[id(pool)] = pool
        return list(pools.values())

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
            self._tail_key = _storage((B, H, cap, D), keys.dtype, keys.device)
            self._tail_value = _storage((B, H, cap, D), values.dtype, values.device)
        self._copy_tokens((self._tail_key[..., :n, :], keys), (self._tail_value[..., :n, :], values))
        self._pending_key = self._tail_key[..., :n, :]
        self._pending_value = self._tail_value[..., :n, :]

    def _copy_tokens(self, *pairs) -> None:
        """dst <- src for (dst, src) [B, H, T, D] token blocks: inside an append they wait for the one
        copy launch at the append's end (dkv_copy_token_blocks)."""
        if self._copy_queue is not None:
            self._copy_queue.extend(pairs)
        else:
            _lib.copy_token_blocks(list(pairs), self._device)

    def _extend_tail(self, key_states: torch.Tensor, value_states: torch.Tensor) -> bool:
        """The decode-step append in few host steps: tokens that only extend the held tail in its
        buffers (no page sealed, no sink token, the cache's shape, dtype and device).  Same result as the
        general path; False (nothing done) whenever any of that does not hold, and the general path then
        runs, with its checks and messages."""
        tk = self._tail_key
        if tk is None or self._tail_count_dev is not None or self.config.value_local_tokens:
            return False
        ks = key_states.shape
        if (len(ks) != 4 or ks != value_states.shape or key_states.dtype is not self._dtype
                or value_states.dtype is not self._dtype or key_states.device != self._device
                or value_states.device != self._device or (ks[0], ks[1], ks[3]) != self._shape
                or key_states.stride(-1) != 1 or value_states.stride(-1) != 1):
            return False
        c = self.config
        n = ks[2]
        # a tail that already holds tokens: the sealed structure and the decode plan built for it (which
        # reads the tail per call) stay valid; starting a tail is left to the general path, which
        # invalidates them
        if self._pending_key is None or not self._pending_in_tail():
            return False
        pending = self._pending_key.shape[2]
        total = pending + n
        if (n == 0 or self._seen_tokens < c.sink_tokens or not (c.hold_partial_pages or c.local_tokens)
                or total > tk.shape[2] or (total - c.local_tokens) >= c.page_size):
            return False
        tv = self._tail_value
        job = self._tail_job
        if job is None or job[0] is not tk or job[1] is not tv:
            job = self._tail_job = _tail_copy_job(tk, tv)
        _, _, blocks, kb, vb, e, st, kbase, vbase = job
        kb.src, kb.dst, kb.T = key_states.data_ptr(), kbase + pending * st, n
        vb.src, vb.dst, vb.T = value_states.data_ptr(), vbase + pending * st, n
        sb, sh, s_t, _ = key_states.stride()
        kb.src_sb, kb.src_sh, kb.src_st = sb * e, sh * e, s_t * e
        sb, sh, s_t, _ = value_states.stride()
        vb.src_sb, vb.src_sh, vb.src_st = sb * e, sh * e, s_t * e
        _lib.check(_lib.load().dkv_copy_token_blocks(blocks, 2, _lib.stream_ptr(self._device)),
                   "dkv_copy_token_blocks")
        self._pending_key = tk.narrow(2, 0, total)
        self._pending_value = tv.narrow(2, 0, total)
        self._seen_tokens += n
        self._layout_version += 1
        self._invalidate_page_descriptors()
        return True

    def _pending_in_tail(self) -> bool:
        pk, tk = self._pending_key, self._tail_key
        return (pk is not None and tk is not None and self._pending_value is not None
                and pk.data_ptr() == tk.data_ptr() and self._pending_value.data_ptr() == self._tail_value.data_ptr()
                and pk.shape[-2] == self._pending_value.shape[-2])

    # ---- appends (the lifecycle of reference cache.py:403-542) ----
    def _append_tokens(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        c = self.config
        if c.value_local_tokens:  # Kitty: a key window and a separate value window
            self._sealed_version += 1
            self._append_window_keys(keys)
            self._append_window_values(values)
        elif c.hold_partial_pages or c.local_tokens:
            self._append_held(keys, values)
        else:
            self._sealed_version += 1
            self._seal(keys, values)  # every page, the last one possibly short

    def _append_held(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Pending tokens plus the new ones: every full page (past the local window) is sealed, the rest is
        held dense."""
        c = self.config
        pending = 0 if self._pending_key is None else self._pending_key.shape[-2]
        total = pending + keys.shape[-2]
        sealable = (max(0, total - c.local_tokens) // c.page_size) * c.page_size
        if sealable == 0 and self._pending_in_tail() and total <= self._tail_capacity():
            # the new tokens only extend the held tail
            self._copy_tokens((self._tail_key[..., pending:total, :], keys),
                              (self._tail_value[..., pending:total, :], values))
            self._pending_key = self._tail_key[..., :total, :]
            self._pending_value = self._tail_value[..., :total, :]
            return
        self._sealed_version += 1
        if pending:
            in_tail = self._pending_in_tail()
            keys = torch.cat((self._pending_key, keys), dim=-2)
            values = torch.cat((self._pending_value, values), dim=-2)
            if in_tail and self._finite_scope is not None:
                # the new tail overwrites the held tokens in the tail buffers: a failed check puts them back
                old_k, old_v = keys[..., :pending, :], values[..., :pending, :]
                tk, tv = self._tail_key, self._tail_value
                self._finite_scope.undo.append(lambda: (tk[..., :pending, :].copy_(old_k),
                                                        tv[..., :pending, :].copy_(old_v)))
        if sealable:
            self._seal(keys[..., :sealable, :], values[..., :sealable, :])
        if sealable < total:
            self._store_pending(keys[..., sealable:, :], values[..., sealable:, :])
        else:
            self._pending_key = self._pending_value = None

    def _append_window_keys(self, keys: torch.Tensor) -> None:
        """Kitty's key window (reference cache.py:424-455): with local_tokens == 1, the first one-token
        append after a prefill that ended on a page boundary packs the last page again from its
        dequantized values; later, a page is packed once a token past it arrives."""
        c = self.config
        last = self._keys[-1] if self._keys else None
        if (self._seen_tokens > 0 and self._pending_key is None and c.local_tokens == 1 and keys.shape[-2] == 1
                and last is not None and not isinstance(last, torch.Tensor)):
            dense = last.dequantize()
            self._keys.pop()
            pool = getattr(last, "_pool", None)
            if pool is not None and pool is self._key_pool and last._at == pool.used - 1:
                pool.used -= 1  # the page is packed again into the same slot
                if self._finite_scope is not None:
                    # a failed check later in this append puts the slot's first packing back (packing
                    # dequantized values again is not idempotent in 16-bit dtypes)
                    at = last._at
                    saved = {name: pool.field(name, at).clone() for name in pool.tensors}
                    self._finite_scope.undo.append(
                        lambda: [pool.field(name, at).copy_(t) for name, t in saved.items()])
            self._seal_keys(dense)
        if self._pending_key is not None:
            keys = torch.cat((self._pending_key, keys), dim=-2)
        window = 0 if self._seen_tokens == 0 else c.local_tokens
        sealable = (max(0, keys.shape[-2] - window) // c.page_size) * c.page_size
        if sealable:
            self._seal_keys(keys[..., :sealable, :])
        self._pending_key = keys[..., sealable:, :].clone() if sealable < keys.shape[-2] else None

    def _append_window_values(self, values: torch.Tensor) -> None:
        """Kitty's value window (reference cache.py:457-470): all but the newest value_local_tokens
        tokens are packed, page-sized chunks in order."""
        c = self.config
        if self._pending_value is not None:
            values = torch.cat((self._pending_value, values), dim=-2)
        packed = max(0, values.shape[-2] - c.value_local_tokens)
        if packed:
            with self._finite_inputs():
                rows = self._pack_values(values[..., :packed, :])
                for start in range(0, packed, c.page_size):
                    self._push_values(rows.rows(start, min(c.page_size, packed - start)))
        self._pending_value = values[..., packed:, :].clone() if packed < values.shape[-2] else None

    @contextlib.contextmanager
    def _finite_inputs(self):
        """Quantize launches inside this scope report NaN or infinite inputs through device flags
        (``_flag_ptr``).  The outermost scope (one append) reads them once on exit, after every launch of
        the append and only when a launch used them (one host synchronization); such an input raises the
        reference's ValueError (quantization.py:159-160, mixed.py:187-188) with the tracks, pools and
        held tail as they were.  The flags are zero between appends: only a failure clears them."""
        if self._finite_scope is not None:
            yield
            return
        scope = self._finite_scope = _FiniteScope(self)
        ok = False
        try:
            yield
            ok = True
        finally:
            self._finite_scope = None
            self._value_job = None
            if not ok and scope.flags is not None:
                # launches before the error may set them: clear them once those have run
                torch.cuda.current_stream(self._device).synchronize()
                scope.flags.zero_()
        if scope.flags is None:
            return
        _drain(self._device)
        bad_keys, bad_values = scope.flags.tolist()
        if bad_keys or bad_values:
            scope.flags.zero_()
            scope.restore(self)
            if bad_keys and self.config.promote_ratio > 0.0:
                raise ValueError("key_states must contain finite values")
            raise ValueError("quantize expects all values to be finite")

    def _flag_ptr(self, which: int) -> int:
        """Address (pinned host memory the kernels write) of the non-finite flag of keys (0) or values (1)
        for a launch inside the append's scope, which then checks it; 0 (no check) outside a scope."""
        scope = self._finite_scope
        if scope is None:
            return 0
        if scope.flags is None:
            scope.flags = _nonfinite_flags(self._device)
        return scope.flags.data_ptr() + 4 * which

    def _seal(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Pack consecutive pages of keys and values; the last may be short (reference cache.py:472-479).
        The key launch that covers the last page quantizes all the tokens' values too."""
        if keys.shape[-2] != values.shape[-2]:
            raise RuntimeError("key/value page lengths diverged before quantization")
        page = self.config.page_size
        T = values.shape[-2]
        with self._finite_inputs():
            rows = self._pack_values(values, defer=True)
            for i, kseg in enumerate(self._pack_key_pages(keys)):
                self._keys.append(kseg)
                self._push_values(rows.rows(i * page, min(page, T - i * page)))

    def _seal_keys(self, keys: torch.Tensor) -> None:
        with self._finite_inputs():
            self._keys.extend(self._pack_key_pages(keys))

    def _push_values(self, segment: PoolValues) -> None:
        """Add a value segment to the value track.  When it continues the pool rows of a value segment
        that is not yet a full page, it fills that page first (the reference concatenates such pieces,
        cache.py:514-542); rows past the page start the next segment."""
        page = self.config.page_size
        last = self._values[-1] if self._values else None
        if (isinstance(last, PoolValues) and last._pool is segment._pool and last._at + last._rows == segment._at
                and last._rows < page):
            take = min(page - last._rows, segment._rows)
            self._values[-1] = last.rows(0, last._rows + take)
            if take == segment._rows:
                return
            segment = segment.rows(take, segment._rows - take)
        self._values.append(segment)

    # ---- packing into the pools ----
    def _value_pool_for(self, values: torch.Tensor) -> PagePool:
        if self._value_pool is None:
            c = self.config
            B, H, _, D = values.shape
            vg = c.resolved_value_group_size
            groups = -(-D // vg)
            packed = -(-groups * vg // (8 // c.resolved_value_bits))
            meta = c.metadata_dtype
            self._value_pool = PagePool(
                {"values": ((B, H, 0, packed), torch.uint8), "scale": ((B, H, 0, groups), meta),
                 "zero_point": ((B, H, 0, groups), meta)}, axis=2, batch_axis=0, device=values.device, align=64)
        return self._value_pool

    def _pack_values(self, values: torch.Tensor, defer: bool = False) -> PoolValues:
        """Quantize value rows [B, H, T, D] along head_dim into new value pool rows.  With ``defer`` the
        launch rides with the key launch of the same tokens (``_value_job``)."""
        c = self.config
        B, H, T, D = values.shape
        pool = self._value_pool_for(values)
        row0 = pool.reserve(T, headroom=max(pool.align, T // 16) if pool.used == 0 else None)
        bits, vg = c.resolved_value_bits, c.resolved_value_group_size
        job, keep = _value_rows_job(values, bits, vg, c.metadata_dtype, pool, row0, self._flag_ptr(1))
        if defer:
            self._value_job = (job, keep)
        else:
            lib = _lib.load()
            _lib.check(lib.dkv_quantize_value_rows(job, _lib.stream_ptr(values.device)), "dkv_quantize_value_rows")
        groups = pool.shapes["scale"][3]
        return PoolValues(pool, row0, T, D, groups * vg, pool.shapes["values"][3] * (8 // bits), vg, bits,
                          values.dtype)

    def _key_pool_for(self, keys: torch.Tensor, groups: int, fresh: bool) -> PagePool:
        """The cache's key pool (pages with the full page's group count), or with ``fresh`` an exact pool
        for pages of another shape (a short last page)."""
        if not fresh and self._key_pool is not None:
            return self._key_pool
        c = self.config
        B, H, _, D = keys.shape
        kg, meta = c.resolved_key_group_size, c.metadata_dtype
        if c.promote_ratio > 0.0:
            K = promoted_count(D, c.promote_ratio)
            nb = (kg + 3) // 4
            fields = {"low_values": ((0, B, H, D, groups, nb), torch.uint8),
                      "high_values": ((0, B, H, K, groups, nb if K else nb * 4), torch.uint8),
                      "channel_indices": ((0, B, H, K), torch.int32),
                      "scale": ((0, B, H, D, groups), meta), "zero_point": ((0, B, H, D, groups), meta)}
        else:
            per = 8 // c.resolved_key_bits
            fields = {"values": ((0, B, H, D, -(-groups * kg // per)), torch.uint8),
                      "scale": ((0, B, H, D, groups), meta), "zero_point": ((0, B, H, D, groups), meta)}
        pool = PagePool(fields, axis=0, batch_axis=1, device=keys.device)
        if not fresh:
            self._key_pool = pool
        return pool

    def _pack_key_pages(self, keys: torch.Tensor) -> List[Segment]:
        """Quantize keys [B, H, T, D] along the tokens, one page per page_size tokens (the last may be
        short).  Full-shape pages go to the key pool, pages with another group count to an exact pool of
        their own.  A deferred value job rides with the last launch."""
        P = self.config.page_size
        T = keys.shape[-2]
        full, rest = divmod(T, P)
        launches = ([(0, P, full)] if full else []) + ([(full * P, rest, 1)] if rest else [])
        job, self._value_job = self._value_job, None
        out: List[Segment] = []
        for i, (start, tokens, n_pages) in enumerate(launches):
            ride = job if i == len(launches) - 1 else None
            out.extend(self._key_launch(keys[..., start:start + n_pages * tokens, :], tokens, n_pages, ride))
        return out

    def _key_launch(self, src: torch.Tensor, tokens: int, n_pages: int, job) -> List[Segment]:
        c = self.config
        H, D = src.shape[1], src.shape[3]
        kg, meta = c.resolved_key_group_size, c.metadata_dtype
        groups = -(-tokens // kg)
        fresh = groups != -(-c.page_size // kg)
        pool = self._key_pool_for(src, groups, fresh)
        slot = pool.reserve(n_pages, headroom=0 if fresh else (max(2, n_pages // 16) if pool.used == 0 else None))
        t = {name: pool.ref(name) for name in pool.shapes}  # page-major: the launch writes pages [slot, slot + n_pages)
        values = None if job is None else job[0]
        flag = self._flag_ptr(0)
        if c.promote_ratio > 0.0:
            K = promoted_count(D, c.promote_ratio)
            selection = {"magnitude": _lib.SELECT_MAGNITUDE, "variance": _lib.SELECT_VARIANCE,
                         "random": _lib.SELECT_GIVEN}[c.channel_selection]
            given = None
            if c.channel_selection == "random" and 0 < K < D:
                # one randperm per KV head per page, shared across the batch (reference mixed.py:145-153)
                given = torch.stack([random_channels(H, D, K, src.device) for _ in range(n_pages)], 0).to(torch.int32)
            common = dict(key_mode=_lib.KEY_MIXED, bits=2, group=kg, promoted=K, selection=selection, meta=meta,
                          nonfinite=flag)
            if given is not None and n_pages > 1:
                for p in range(n_pages):
                    launch_key_pages(src[..., p * tokens:(p + 1) * tokens, :], page_tokens=tokens, n_pages=1,
                                     given_idx=given[p].contiguous(), low=t["low_values"], high=t["high_values"],
                                     idx=t["channel_indices"], scale=t["scale"], zero=t["zero_point"],
                                     values=values if p == n_pages - 1 else None, slot=slot + p, **common)
            else:
                launch_key_pages(src, page_tokens=tokens, n_pages=n_pages,
                                 given_idx=None if given is None else given[0].contiguous(), low=t["low_values"],
                                 high=t["high_values"], idx=t["channel_indices"], scale=t["scale"],
                                 zero=t["zero_point"], values=values, slot=slot, **common)
            return [PoolMixedKey(pool, slot + p, tokens, D, groups * kg, kg, c.promote_bits, src.dtype)
                    for p in range(n_pages)]
        bits = c.resolved_key_bits
        launch_key_pages(src, page_tokens=tokens, n_pages=n_pages, key_mode=_lib.KEY_UNIFORM, bits=bits, group=kg,
                         promoted=0, selection=0, given_idx=None, meta=meta, low=t["values"], high=None, idx=None,
                         scale=t["scale"], zero=t["zero_point"], values=values, nonfinite=flag, slot=slot)
        packed = pool.shapes["values"][4]
        return [PoolKeys(pool, slot + p, tokens, D, groups * kg, packed * (8 // bits), kg, bits, src.dtype)
                for p in range(n_pages)]

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
        if self._tail_count_dev is not None:
            return  # already on: a second call keeps the count tensor captured graphs read
        if self._tail_key is None:
            B, H, D = self._shape
            cap = self._tail_capacity()
            self._tail_key = _storage((B, H, cap, D), self._dtype, self._device)
            self._tail_value = _storage((B, H, cap, D), self._dtype, self._device)
        if self._pending_key is not None and not self._pending_in_tail():
            self._store_pending(self._pending_key, self._pending_value)
            if not self._pending_in_tail():
                raise RuntimeError("the held tail does not fit the tail buffer")
        self._tail_count_dev = _storage((1,), torch.int64, self._device)
        self._tail_count_dev.zero_()
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
                self._sealed_version += 1
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
        sealed = self._sealed_pairs()
        tail_is_pending = self._tail_resident() or self._tail_count_dev is not None
        keepalive: list = [dict(p.tensors) for p in self._pools()]  # storage outlives the table
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
        plan.host_table = descs if sealed else None
        self._decode_plan_cache = plan
        return plan


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------

def _union_pairs(keys: list, values: list) -> list:
    """Cut two segment tracks that cover the same tokens at every boundary of either one; a piece that
    covers part of a segment becomes that part, dequantized."""
    if not keys or not values:
        return []
    k_len = [_segment_tokens(s) for s in keys]
    v_len = [_segment_tokens(s) for s in values]
    if min(k_len + v_len) <= 0:
        raise RuntimeError("DartKVCache contains an empty logical segment")
    k_ends, v_ends = list(accumulate(k_len)), list(accumulate(v_len))
    if k_ends[-1] != v_ends[-1]:
        raise RuntimeError("DartKVCache key/value logical lengths diverged")
    pairs, start, ki, vi = [], 0, 0, 0
    for stop in sorted(set(k_ends).union(v_ends)):
        k0, v0 = k_ends[ki] - k_len[ki], v_ends[vi] - v_len[vi]
        pairs.append((_piece(keys[ki], start - k0, stop - k0), _piece(values[vi], start - v0, stop - v0)))
        ki += stop == k_ends[ki]
        vi += stop == v_ends[vi]
        start = stop
    return pairs


def _piece(segment: Segment, start: int, stop: int) -> Segment:
    if start == 0 and stop == _segment_tokens(segment):
        return segment
    return _materialize(segment)[..., start:stop, :].contiguous()


def _page_mode(segment: Segment) -> int:
    """DENSE_PAGE 0, QUANTIZED_PAGE 1, MIXED_PAGE 2 (reference page_table.py:19-21)."""
    if isinstance(segment, torch.Tensor):
        return 0
    return 2 if isinstance(segment, MixedQuantizedKey) else 1


def _full_uniform(kseg: Segment, vseg: Segment, page: int) -> bool:
    return (isinstance(kseg, QuantizedTensor) and isinstance(vseg, QuantizedTensor)
            and kseg.original_shape[-2] == page and vseg.original_shape[-2] == page)


def _same_run_layout(a: tuple, b: tuple) -> bool:
    """Two full uniform pages whose packed fields stack into one page-major run."""
    return all(x.original_shape == y.original_shape and x.bits == y.bits and x.group_size == y.group_size
               and x.packed_dim == y.packed_dim and x.padded_dim == y.padded_dim for x, y in zip(a, b))


def _run_fields(segments: list, names: tuple, page_major: bool) -> list:
    """Page-major [n, ...] tensors of ``names`` over ``segments``: a slice of the pool when the segments
    are consecutive slots (keys) or consecutive equal-length row runs (values), else a stacked copy."""
    first = segments[0]
    pool = getattr(first, "_pool", None)
    n = len(segments)
    step = 1 if page_major else first._rows if pool is not None else 0
    if pool is not None and all(getattr(s, "_pool", None) is pool and s._at == first._at + i * step
                                and (page_major or s._rows == step) for i, s in enumerate(segments)):
        if page_major:
            return [pool.field(name, first._at, n) for name in names]
        # [B, H, n * rows, ...] -> [n, B, H, rows, ...]
        return [pool.field(name, first._at, n * step).unflatten(2, (n, step)).movedim(2, 0) for name in names]
    return [torch.stack([getattr(s, name) for s in segments], 0) for name in names]


def _tail_copy_job(tk: torch.Tensor, tv: torch.Tensor) -> tuple:
    """A two-block dkv_copy_token_blocks description that writes tokens into the tail buffers ``tk`` and
    ``tv`` ([B, H, capacity, D], one dtype): (tk, tv, blocks, key block, value block, element size, token
    stride in bytes, tk address, tv address).  Per call only the sources, the first row and the token
    count change."""
    blocks = (_lib.CopyBlock * 2)()
    e = tk.element_size()
    for blk, t in zip(blocks, (tk, tv)):
        blk.B, blk.H, _, D = t.shape
        blk.row_bytes = D * e
        blk.dst_sb, blk.dst_sh, blk.dst_st = t.stride(0) * e, t.stride(1) * e, t.stride(2) * e
    return (tk, tv, blocks, blocks[0], blocks[1], e, tk.stride(2) * e, tk.data_ptr(), tv.data_ptr())


def _value_rows_job(src: torch.Tensor, bits: int, group: int, meta: torch.dtype, pool: Optional[PagePool],
                    row0: int, nonfinite: int = 0, out: Optional[tuple] = None):
    """The C description of quantizing [B,H,T,D] value rows along head_dim into value pool rows
    [row0, row0 + T) (or, with ``out`` = (values, scale, zero) contiguous [B,H,T,...] tensors, into those).

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
    if out is not None:
        values, scale, zero = out
        out_rows, row0 = T, 0
    else:
        values, scale, zero = pool.ref("values"), pool.ref("scale"), pool.ref("zero_point")
        out_rows = pool.capacity
    job = _lib.ValueRowsArgs(src=src.data_ptr(), src_dtype=_lib.dtype_code(src.dtype), blocks=blocks,
                             block_stride=block_stride, block_rows=T, n=D, row_stride=D, bits=bits, group=group,
                             values=values.data_ptr(), scale=scale.data_ptr(), zero=zero.data_ptr(),
                             meta_dtype=_lib.dtype_code(meta), nonfinite=nonfinite or None,
                             out_block_rows=out_rows, out_row0=row0)
    return job, src


def _launch_value_rows(src: torch.Tensor, bits: int, group: int, meta: torch.dtype, values: torch.Tensor,
                       scale: torch.Tensor, zero: torch.Tensor, nonfinite: int = 0) -> None:
    """Quantize [B,H,T,D] value rows along head_dim into contiguous [B,H,T,...] outputs
    (dkv_quantize_value_rows)."""
    job, src = _value_rows_job(src, bits, group, meta, None, 0, nonfinite, out=(values, scale, zero))
    lib = _lib.load()
    _lib.check(lib.dkv_quantize_value_rows(job, _lib.stream_ptr(src.device)), "dkv_quantize_value_rows")


def _materialize(segment: Segment) -> torch.Tensor:
    return segment if isinstance(segment, torch.Tensor) else segment.dequantize()


def _segment_tokens(segment: Segment) -> int:
    return segment.shape[-2] if isinstance(segment, torch.Tensor) else segment.original_shape[-2]


def _segment_layout(segment: Segment) -> DartSegmentLayout:
    if isinstance(segment, torch.Tensor):
        return DartSegmentLayout("dense", tuple(segment.shape), (("values", tuple(segment.shape), tuple(segment.stride())),))
    if isinstance(segment, MixedQuantizedKey):
        kind, names = "mixed_key", ("low_values", "high_values", "channel_indices", "scale", "zero_point")
    else:
        kind, names = "quantized", ("values", "scale", "zero_point")
    fields = tuple((name, tuple(t.shape), tuple(t.stride())) for name, t in ((n, getattr(segment, n)) for n in names))
    return DartSegmentLayout(kind, tuple(segment.original_shape), fields)


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
    """(address, (batch, head) stride) of a segment field; a pool segment's comes from the pool's layout
    without making a view.  Empty fields give (0, 0)."""
    pool = getattr(seg, "_pool", None)
    if pool is not None:
        shape = pool.shapes[name]
        if 0 in shape[:pool.axis] + shape[pool.axis + 1:]:
            return 0, 0
        return seg.block(name)
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


def tail_segment(cache: DartKVCache, with_dense_check: bool = False):
    """Descriptor of the held tail (pending tokens in the tail buffer).

    With device-side tail counts the descriptor spans the whole tail buffer
    (its capacity) and the kernels read the live count from the device.  The
    descriptor of a tail is kept while its tensors keep their addresses and
    strides (one-token appends only change the token count), and the same
    object is returned while the token count stays too: do not modify it.
    ``with_dense_check`` returns (descriptor, True when it has no tokens or the
    dense decode kernel can read it: ``_dense16_ok``).
    """
    if cache._tail_count_dev is not None:
        pk, pv = cache._tail_key, cache._tail_value
    elif cache._pending_key is None:
        desc = _lib.Segment()
        return (desc, True) if with_dense_check else desc
    else:
        pk, pv = cache._pending_key, cache._pending_value
    key = (pk.data_ptr(), pv.data_ptr(), pk.stride(), pv.stride())
    tokens = pk.shape[-2]
    held = cache._tail_desc
    if held is None or held[0] != key:
        base = _lib.Segment()
        base.key_kind = _lib.KEY_DENSE
        base.value_kind = _lib.VALUE_DENSE
        keep: list = []
        base.key[0], base.key_bh[0] = _dense_block(pk, keep)
        base.value[0], base.value_bh[0] = _dense_block(pv, keep)
        if keep:
            raise RuntimeError("held tail is not in the tail buffer layout")
        held = cache._tail_desc = [key, base, _dense16_ok(base), -1, None]
    if held[3] != tokens:
        desc = _lib.Segment.from_buffer_copy(held[1])
        desc.tokens = tokens
        held[3], held[4] = tokens, desc
    return (held[4], tokens == 0 or held[2]) if with_dense_check else held[4]


__all__ = ["DartKVCache", "DartKVCacheConfig", "DartPageMetadata", "DartSegmentLayout"]

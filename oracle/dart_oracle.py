"""CPU oracle for the DartKV compressed-KV path.  TEST INFRASTRUCTURE ONLY.

This module restates the reference algorithm (PyTorch eager ops on CPU) so
the HIP kernels can be checked against it.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as a checker or as the timed CPU baseline.  The product
package (``dartkv_amd``) never imports or calls it.

Every function names the reference file:line it follows.  The op sequence is
kept identical on purpose: the reference quantizes in the source dtype one op
at a time, and the oracle must round exactly where the reference rounds.

Pinning (how each part is known to equal the reference):
* ``pack``/``unpack``: closed form (LSB-first bit fields), golden vectors.
* ``quantize``/``quantize_key_mixed``/``select_key_channels``: golden vectors
  written by ``tests/golden/make_golden.py`` from the reference itself, plus
  invariants (codes in range, group min -> code 0, round trip bound).
* ``OracleCache`` lifecycle: the reference tests' literal page layouts and the
  golden lifecycle vectors (non-held pages, value merging, Kitty modes).
* ``streamed_attention``: golden outputs of the reference's
  ``streamed_dart_attention`` plus the closed form ``dense_attention`` on the
  materialized cache.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional, Tuple, Union

import torch

SUPPORTED_BITS = (2, 4, 8)


# ---------------------------------------------------------------------------
# bit packing  (reference src/dart/quantization.py:25-45)
# ---------------------------------------------------------------------------

def pack(codes: torch.Tensor, bits: int, packed_dim: int) -> torch.Tensor:
    """LSB-first packing of uint8 codes along the last dim (quantization.py:25-35)."""
    per_byte = 8 // bits
    extra = packed_dim - codes.shape[-1]
    if extra:
        codes = torch.nn.functional.pad(codes, (0, extra))
    codes = codes.reshape(*codes.shape[:-1], -1, per_byte)
    shifts = torch.arange(per_byte, dtype=torch.uint8) * bits
    return torch.sum(codes << shifts, dim=-1, dtype=torch.uint8)


def unpack(packed: torch.Tensor, bits: int, length: int) -> torch.Tensor:
    """Inverse of :func:`pack` (quantization.py:38-45)."""
    per_byte = 8 // bits
    shifts = torch.arange(per_byte, dtype=torch.uint8) * bits
    fields = (packed.unsqueeze(-1) >> shifts) & ((1 << bits) - 1)
    return fields.reshape(*packed.shape[:-1], packed.shape[-1] * per_byte)[..., :length]


def _meta_dtype(data: torch.Tensor, requested: Optional[torch.dtype]) -> torch.dtype:
    """quantization.py:48-53."""
    if requested is not None:
        if requested not in (torch.float16, torch.bfloat16, torch.float32, torch.float64):
            raise TypeError(f"metadata dtype must be floating point, got {requested}")
        return requested
    return data.dtype if data.dtype in (torch.float16, torch.bfloat16) else torch.float32


def _numel(shape) -> int:
    n = 1
    for s in shape:
        n *= s
    return n


# ---------------------------------------------------------------------------
# uniform quantization  (reference src/dart/quantization.py:56-223)
# ---------------------------------------------------------------------------

@dataclass
class OQuantized:
    """Same fields as the reference ``QuantizedTensor`` (quantization.py:56-124)."""

    values: torch.Tensor
    scale: torch.Tensor
    zero_point: torch.Tensor
    original_shape: Tuple[int, ...]
    original_dim: int
    padded_dim: int
    packed_dim: int
    group_size: int
    bits: int
    output_dtype: torch.dtype
    axis: int = -1

    @property
    def groups(self) -> int:
        return (self.padded_dim + self.group_size - 1) // self.group_size

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.values, self.scale, self.zero_point))

    def dequantize(self, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """quantization.py:96-109: code*scale + zero in the metadata dtype."""
        codes = unpack(self.values, self.bits, self.packed_dim)[..., : self.padded_dim]
        axis = self.axis if self.axis >= 0 else len(self.original_shape) + self.axis
        moved = tuple(s for i, s in enumerate(self.original_shape) if i != axis) + (self.original_shape[axis],)
        outer = moved[:-1]
        grouped = codes.reshape(*outer, self.groups, self.group_size).to(self.scale.dtype)
        out = grouped * self.scale.unsqueeze(-1) + self.zero_point.unsqueeze(-1)
        out = out.reshape(*outer, self.padded_dim)[..., : self.original_dim]
        out = out.to(dtype or self.output_dtype)
        if axis != len(self.original_shape) - 1:
            out = out.movedim(-1, axis)
        return out


def quantize(data: torch.Tensor, *, bits: int = 2, group_size: int = 64,
             metadata_dtype: Optional[torch.dtype] = None, axis: int = -1) -> OQuantized:
    """quantization.py:134-204 (same op order, same dtype at every step)."""
    if bits not in SUPPORTED_BITS:
        raise ValueError(f"bits must be one of {SUPPORTED_BITS}, got {bits}")
    if not isinstance(group_size, int) or group_size <= 0:
        raise ValueError(f"group_size must be a positive integer, got {group_size}")
    if data.ndim == 0:
        raise ValueError("quantize expects a tensor with at least one dimension")
    if not torch.is_floating_point(data):
        raise TypeError(f"quantize expects a floating-point tensor, got {data.dtype}")
    if data.shape[-1] == 0:
        raise ValueError("quantize does not support an empty final dimension")
    if not torch.isfinite(data).all():
        raise ValueError("quantize expects all values to be finite")
    original_shape = tuple(data.shape)
    if not isinstance(axis, int) or not -data.ndim <= axis < data.ndim:
        raise ValueError(f"axis must be in [-{data.ndim}, {data.ndim}), got {axis}")
    axis = axis % data.ndim
    data = data.movedim(axis, -1).contiguous()
    n = data.shape[-1]
    groups = (n + group_size - 1) // group_size
    padded = groups * group_size
    rows = data.reshape(-1, n)
    if padded > n:  # replicate the last element (quantization.py:174-177)
        rows = torch.cat((rows, rows[..., -1:].expand(-1, padded - n)), dim=-1)
    g = rows.reshape(-1, groups, group_size)
    lo = g.amin(dim=-1)
    hi = g.amax(dim=-1)
    qmax = float((1 << bits) - 1)
    eps = 1e-4 if data.dtype in (torch.float16, torch.bfloat16) else 1e-6
    scale = (hi - lo).clamp(min=eps) / qmax
    q = ((g - lo.unsqueeze(-1)) / scale.unsqueeze(-1)).round()
    q = q.clamp_(0, qmax).to(torch.uint8).reshape(*data.shape[:-1], padded)
    per_byte = 8 // bits
    packed_dim = ((padded + per_byte - 1) // per_byte) * per_byte
    meta = _meta_dtype(data, metadata_dtype)
    return OQuantized(
        values=pack(q, bits, packed_dim),
        scale=scale.reshape(*data.shape[:-1], groups).to(meta),
        zero_point=lo.reshape(*data.shape[:-1], groups).to(meta),
        original_shape=original_shape, original_dim=n, padded_dim=padded,
        packed_dim=packed_dim, group_size=group_size, bits=bits,
        output_dtype=data.dtype, axis=axis,
    )


# ---------------------------------------------------------------------------
# Dart promotion  (reference src/dart/mixed.py:13-244)
# ---------------------------------------------------------------------------

@dataclass
class OMixedKey:
    """Same fields as the reference ``MixedQuantizedKey`` (mixed.py:13-116)."""

    low_values: torch.Tensor
    high_values: torch.Tensor
    channel_indices: torch.Tensor
    scale: torch.Tensor
    zero_point: torch.Tensor
    original_shape: Tuple[int, ...]
    padded_tokens: int
    group_size: int
    low_bits: int
    promote_bits: int
    output_dtype: torch.dtype

    @property
    def groups(self) -> int:
        return self.padded_tokens // self.group_size

    @property
    def nbytes(self) -> int:
        ts = (self.low_values, self.high_values, self.channel_indices, self.scale, self.zero_point)
        return sum(t.numel() * t.element_size() for t in ts)

    def dequantize(self, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """mixed.py:72-94: low | high<<2, scattered back by channel index."""
        nb = self.low_values.shape[-1]
        low = unpack(self.low_values, self.low_bits, nb * (8 // self.low_bits))[..., : self.group_size]
        hb = self.promote_bits - self.low_bits
        high = unpack(self.high_values, hb, self.high_values.shape[-1] * (8 // hb))[..., : self.group_size]
        B, H, _, D = self.original_shape
        full = torch.zeros((B, H, D, self.groups, self.group_size), dtype=low.dtype)
        K = self.channel_indices.shape[-1]
        if K:
            idx = self.channel_indices.long()[..., None, None].expand(B, H, K, self.groups, self.group_size)
            full.scatter_(2, idx, high)
        codes = low | (full << self.low_bits)
        out = codes.to(self.scale.dtype) * self.scale.unsqueeze(-1) + self.zero_point.unsqueeze(-1)
        out = out.reshape(B, H, D, self.padded_tokens)[..., : self.original_shape[-2]].transpose(-1, -2)
        return out.to(dtype or self.output_dtype)


def select_key_channels(keys: torch.Tensor, promote_ratio: float, *, strategy: str = "magnitude",
                        random_indices: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """mixed.py:119-163.  ``random_indices`` ([H, K]) replaces the reference's
    per-head ``torch.randperm`` draws so a checker can feed both sides the same
    random selection."""
    if keys.ndim != 4:
        raise ValueError("key_states must have shape [B, H, T, D]")
    if not 0.0 <= promote_ratio <= 1.0:
        raise ValueError("promote_ratio must be in [0, 1]")
    if strategy not in {"magnitude", "random", "variance"}:
        raise ValueError("strategy must be 'magnitude', 'random', or 'variance'")
    B, H, _, D = keys.shape
    count = min(D, int(D * promote_ratio + 1e-6))
    mask = torch.zeros(B, H, D, dtype=torch.bool)
    if count == 0:
        return mask, torch.empty(B, H, 0, dtype=torch.long)
    if count == D:
        return torch.ones_like(mask), torch.arange(D).view(1, 1, -1).expand(B, H, -1)
    if strategy == "random":
        if random_indices is None:
            random_indices = torch.stack([torch.randperm(D)[:count] for _ in range(H)], dim=0)
        idx = random_indices.long().unsqueeze(0).expand(B, -1, -1)
    elif strategy == "magnitude":
        idx = keys.abs().mean(dim=-2).topk(count, dim=-1, sorted=True).indices
    else:
        centered = keys - keys.mean(dim=-2, keepdim=True)
        idx = centered.square().mean(dim=-2).topk(count, dim=-1, sorted=True).indices
    mask.scatter_(-1, idx, True)
    return mask, idx


def quantize_key_mixed(keys: torch.Tensor, *, group_size: int = 128, promote_ratio: float = 0.25,
                       promote_bits: int = 4, strategy: str = "magnitude",
                       metadata_dtype: Optional[torch.dtype] = None,
                       random_indices: Optional[torch.Tensor] = None) -> OMixedKey:
    """mixed.py:166-244 (same op order and dtypes)."""
    if keys.ndim != 4:
        raise ValueError("key_states must have shape [B, H, T, D]")
    if not torch.is_floating_point(keys):
        raise TypeError("key_states must be floating point")
    if keys.shape[-2] == 0 or keys.shape[-1] == 0:
        raise ValueError("key_states sequence and head dimensions must be non-empty")
    if not isinstance(group_size, int) or group_size <= 0:
        raise ValueError("group_size must be a positive integer")
    if promote_bits != 4:
        raise ValueError("the reference mixed representation currently supports promote_bits=4")
    if not torch.isfinite(keys).all():
        raise ValueError("key_states must contain finite values")
    mask, idx = select_key_channels(keys, promote_ratio, strategy=strategy, random_indices=random_indices)
    B, H, T, D = keys.shape
    G = (T + group_size - 1) // group_size
    padded = G * group_size
    data = keys.transpose(-1, -2).contiguous()
    if padded > T:
        data = torch.cat((data, data[..., -1:].expand(-1, -1, -1, padded - T)), dim=-1)
    g = data.reshape(B, H, D, G, group_size)
    lo = g.amin(dim=-1)
    hi = g.amax(dim=-1)
    promoted = mask.unsqueeze(-1)
    qmax = torch.where(promoted, torch.full_like(lo, (1 << promote_bits) - 1), torch.full_like(lo, 3.0))
    eps = 1e-4 if keys.dtype in (torch.float16, torch.bfloat16) else 1e-6
    scale = (hi - lo).clamp(min=eps) / qmax
    q = ((g - lo.unsqueeze(-1)) / scale.unsqueeze(-1)).round()
    q = torch.minimum(torch.maximum(q, torch.zeros_like(q)), qmax.unsqueeze(-1)).to(torch.uint8)
    nb = (group_size + 3) // 4
    low = pack(q & 0x3, 2, nb * 4)
    hb = promote_bits - 2
    if idx.shape[-1]:
        sel = q.gather(2, idx[..., None, None].expand(B, H, idx.shape[-1], G, group_size)) >> 2
        high = pack(sel, hb, nb * (8 // hb))
    else:
        high = torch.empty(B, H, 0, G, nb * (8 // hb), dtype=torch.uint8)
    meta = metadata_dtype or (keys.dtype if keys.dtype in (torch.float16, torch.bfloat16) else torch.float32)
    return OMixedKey(
        low_values=low, high_values=high, channel_indices=idx.to(torch.int32),
        scale=scale.to(meta), zero_point=lo.to(meta), original_shape=tuple(keys.shape),
        padded_tokens=padded, group_size=group_size, low_bits=2, promote_bits=promote_bits,
        output_dtype=keys.dtype,
    )


# ---------------------------------------------------------------------------
# cache lifecycle  (reference src/dart/cache.py:45-613)
# ---------------------------------------------------------------------------

Segment = Union[torch.Tensor, OQuantized, OMixedKey]


@dataclass(frozen=True)
class OracleConfig:
    """Fields and defaults of the reference ``DartKVCacheConfig`` (cache.py:45-112)."""

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

    @property
    def kbits(self) -> int:
        return self.key_bits if self.key_bits is not None else self.bits

    @property
    def vbits(self) -> int:
        return self.value_bits if self.value_bits is not None else self.bits

    @property
    def kgroup(self) -> int:
        return self.key_group_size if self.key_group_size is not None else self.group_size

    @property
    def vgroup(self) -> int:
        return self.value_group_size if self.value_group_size is not None else self.group_size


def seg_tokens(seg: Segment) -> int:
    return seg.shape[-2] if isinstance(seg, torch.Tensor) else seg.original_shape[-2]


def materialize(seg: Segment) -> torch.Tensor:
    return seg if isinstance(seg, torch.Tensor) else seg.dequantize()


class OracleCache:
    """Restatement of ``DartKVCache`` append/segment logic (cache.py:115-542)."""

    def __init__(self, config: Optional[OracleConfig] = None, random_indices=None) -> None:
        self.config = config or OracleConfig()
        self.keys: List[Segment] = []
        self.values: List[Segment] = []
        self.pending_key: Optional[torch.Tensor] = None
        self.pending_value: Optional[torch.Tensor] = None
        self.shape = None
        self.dtype = None
        self.seen = 0
        # per-head random channel sets for the "random" strategy, shared with the GPU side
        self.random_indices = random_indices

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """cache.py:168-190."""
        if self.shape is None:
            self.shape = (k.shape[0], k.shape[1], k.shape[3])
            self.dtype = k.dtype
        k = k.detach().contiguous()
        v = v.detach().contiguous()
        T = k.shape[-2]
        sink = min(max(0, self.config.sink_tokens - self.seen), T)
        if sink:
            self.keys.append(k[..., :sink, :].clone())
            self.values.append(v[..., :sink, :].clone())
        if sink < T:
            self._remainder(k[..., sink:, :], v[..., sink:, :])
        self.seen += T

    def _remainder(self, k, v) -> None:
        """cache.py:403-422."""
        c = self.config
        if c.value_local_tokens:
            self._key_remainder(k)
            self._value_remainder(v)
            return
        if c.hold_partial_pages or c.local_tokens:
            if self.pending_key is not None:
                k = torch.cat((self.pending_key, k), dim=-2)
                v = torch.cat((self.pending_value, v), dim=-2)
            avail = max(0, k.shape[-2] - c.local_tokens)
            full = (avail // c.page_size) * c.page_size
            if full:
                self._pages(k[..., :full, :], v[..., :full, :])
            self.pending_key = k[..., full:, :].clone() if full < k.shape[-2] else None
            self.pending_value = v[..., full:, :].clone() if full < v.shape[-2] else None
            return
        for s in range(0, k.shape[-2], c.page_size):
            e = min(s + c.page_size, k.shape[-2])
            self._pages(k[..., s:e, :], v[..., s:e, :])

    def _key_remainder(self, k) -> None:
        """cache.py:424-455 (Kitty key Q-buffer lifecycle)."""
        c = self.config
        if (self.seen > 0 and self.pending_key is None and c.local_tokens == 1 and k.shape[-2] == 1
                and self.keys and not isinstance(self.keys[-1], torch.Tensor)):
            last = materialize(self.keys.pop())
            self._key_pages(last)
        if self.pending_key is not None:
            k = torch.cat((self.pending_key, k), dim=-2)
        local = 0 if self.seen == 0 else c.local_tokens
        avail = max(0, k.shape[-2] - local)
        full = (avail // c.page_size) * c.page_size
        if full:
            self._key_pages(k[..., :full, :])
        self.pending_key = k[..., full:, :].clone() if full < k.shape[-2] else None

    def _value_remainder(self, v) -> None:
        """cache.py:457-470."""
        c = self.config
        if self.pending_value is not None:
            v = torch.cat((self.pending_value, v), dim=-2)
        q = max(0, v.shape[-2] - c.value_local_tokens)
        for s in range(0, q, c.page_size):
            self._value_seg(v[..., s:min(s + c.page_size, q), :])
        self.pending_value = v[..., q:, :].clone() if q < v.shape[-2] else None

    def _pages(self, k, v) -> None:
        """cache.py:472-479."""
        P = self.config.page_size
        for s in range(0, k.shape[-2], P):
            e = min(s + P, k.shape[-2])
            self._key_pages(k[..., s:e, :])
            self._value_seg(v[..., s:e, :])

    def _key_pages(self, k) -> None:
        """cache.py:481-503."""
        c = self.config
        for s in range(0, k.shape[-2], c.page_size):
            page = k[..., s:s + c.page_size, :]
            if c.promote_ratio > 0.0:
                seg = quantize_key_mixed(page, group_size=c.kgroup, metadata_dtype=c.metadata_dtype,
                                         promote_ratio=c.promote_ratio, promote_bits=c.promote_bits,
                                         strategy=c.channel_selection, random_indices=self.random_indices)
            else:
                seg = quantize(page, axis=-2, bits=c.kbits, group_size=c.kgroup, metadata_dtype=c.metadata_dtype)
            self.keys.append(seg)

    def _value_seg(self, v) -> None:
        """cache.py:505-542 (token-wise values merged up to one page)."""
        c = self.config
        seg = quantize(v, bits=c.vbits, group_size=c.vgroup, metadata_dtype=c.metadata_dtype)
        if not self.values or isinstance(self.values[-1], torch.Tensor):
            self.values.append(seg)
            return
        prev = self.values[-1]
        if prev.original_shape[-2] == c.page_size:
            self.values.append(seg)
            return
        merged = _merge_values([prev, seg])
        n = merged.original_shape[-2]
        self.values[-1] = _slice_values(merged, 0, min(c.page_size, n))
        if n > c.page_size:
            self.values.append(_slice_values(merged, c.page_size, n))

    def segments(self) -> List[Tuple[Segment, Segment]]:
        """cache.py:229-274: union of K/V boundaries; straddled pieces go dense."""
        ks = list(self.keys)
        vs = list(self.values)
        if self.pending_key is not None:
            ks.append(self.pending_key)
            vs.append(self.pending_value)
        out = []
        ki = vi = ko = vo = 0
        while ki < len(ks) and vi < len(vs):
            kl, vl = seg_tokens(ks[ki]), seg_tokens(vs[vi])
            take = min(kl - ko, vl - vo)
            out.append((_slice_seg(ks[ki], ko, ko + take), _slice_seg(vs[vi], vo, vo + take)))
            ko += take
            vo += take
            if ko == kl:
                ki, ko = ki + 1, 0
            if vo == vl:
                vi, vo = vi + 1, 0
        return out

    def get(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """cache.py:192-199."""
        ks = [materialize(s) for s in self.keys] + ([self.pending_key] if self.pending_key is not None else [])
        vs = [materialize(s) for s in self.values] + ([self.pending_value] if self.pending_value is not None else [])
        return torch.cat(ks, dim=-2), torch.cat(vs, dim=-2)

    def page_ranges(self) -> List[Tuple[int, int, int, int]]:
        """(start, count, key mode, value mode) per segment; modes as page_table.py:24-27."""
        out, start = [], 0
        for k, v in self.segments():
            n = seg_tokens(k)
            out.append((start, n, _mode(k), _mode(v)))
            start += n
        return out


def _mode(seg: Segment) -> int:
    if isinstance(seg, torch.Tensor):
        return 0
    return 2 if isinstance(seg, OMixedKey) else 1


def _slice_seg(seg: Segment, a: int, b: int) -> Segment:
    """cache.py:557-560."""
    if a == 0 and b == seg_tokens(seg):
        return seg
    return materialize(seg)[..., a:b, :].contiguous()


def _slice_values(seg: OQuantized, a: int, b: int) -> OQuantized:
    """cache.py:563-578."""
    shape = list(seg.original_shape)
    shape[-2] = b - a
    return OQuantized(seg.values[..., a:b, :], seg.scale[..., a:b, :], seg.zero_point[..., a:b, :],
                      tuple(shape), seg.original_dim, seg.padded_dim, seg.packed_dim, seg.group_size,
                      seg.bits, seg.output_dtype, seg.axis)


def _merge_values(segs: List[OQuantized]) -> OQuantized:
    """cache.py:581-613."""
    r = segs[0]
    shape = list(r.original_shape)
    shape[-2] = sum(s.original_shape[-2] for s in segs)
    return OQuantized(torch.cat([s.values for s in segs], dim=-2), torch.cat([s.scale for s in segs], dim=-2),
                      torch.cat([s.zero_point for s in segs], dim=-2), tuple(shape), r.original_dim,
                      r.padded_dim, r.packed_dim, r.group_size, r.bits, r.output_dtype, r.axis)


# ---------------------------------------------------------------------------
# attention  (reference src/dart/attention.py:14-87)
# ---------------------------------------------------------------------------

def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: Optional[float] = None) -> torch.Tensor:
    """attention.py:14-29."""
    f = scale if scale is not None else 1.0 / math.sqrt(q.shape[-1])
    logits = torch.matmul(q.float(), k.float().transpose(-1, -2)) * f
    return torch.matmul(torch.softmax(logits, dim=-1), v.float()).to(q.dtype)


def streamed_attention(q: torch.Tensor, cache: OracleCache, *, scale: Optional[float] = None,
                       return_fp32: bool = False):
    """attention.py:32-87: per query head, online softmax over segments.

    Returns the output in ``q.dtype``; with ``return_fp32`` also returns the
    fp32 tensor the reference holds just before its final cast (attention.py:86).
    """
    B, Hkv, D = cache.shape
    Hq = q.shape[1]
    groups = Hq // Hkv
    f = scale if scale is not None else 1.0 / math.sqrt(D)
    qf = q.float()
    out = torch.zeros_like(qf)
    segs = cache.segments()
    deq = [(materialize(k), materialize(v)) for k, v in segs]  # CPU: triton_dequantize == .dequantize()
    for h in range(Hq):
        kv = h // groups
        qh = qf[:, h]
        m = torch.full((B, q.shape[-2]), -torch.inf, dtype=torch.float32)
        l = torch.zeros_like(m)
        acc = torch.zeros((B, q.shape[-2], D), dtype=torch.float32)
        for keys, values in deq:
            keys = keys[:, kv].float()
            values = values[:, kv].float()
            logits = torch.matmul(qh, keys.transpose(-1, -2)) * f
            new_m = torch.maximum(m, logits.amax(dim=-1))
            old_w = torch.exp(m - new_m)
            w = torch.exp(logits - new_m.unsqueeze(-1))
            acc = acc * old_w.unsqueeze(-1) + torch.matmul(w, values)
            l = l * old_w + w.sum(dim=-1)
            m = new_m
        out[:, h] = acc / l.clamp_min(1e-20).unsqueeze(-1)
    if return_fp32:
        return out.to(q.dtype), out
    return out.to(q.dtype)


def algorithmic_page_bytes(D: int, page: int, key_mode: int, key_bits: int, value_bits: int,
                           kg: int, vg: int, promoted: int, meta_bytes: int) -> int:
    """Bytes one (page, kv-head) block occupies: packed codes + metadata."""
    if key_mode == 2:
        G = (page + kg - 1) // kg
        nb = (kg + 3) // 4
        kbytes = D * G * nb + promoted * G * nb + 4 * promoted + 2 * D * G * meta_bytes
    else:
        G = (page + kg - 1) // kg
        per = 8 // key_bits
        kbytes = D * ((G * kg + per - 1) // per) + 2 * D * G * meta_bytes
    gv = (D + vg - 1) // vg
    per = 8 // value_bits
    vbytes = page * ((gv * vg + per - 1) // per) + 2 * page * gv * meta_bytes
    return kbytes + vbytes

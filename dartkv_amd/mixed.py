"""Dart mixed-precision keys: 2-bit codes for every channel, upper 2 bits for
promoted channels (HIP-backed).

Public surface and validation follow the reference ``dart.mixed``
(reference src/dart/mixed.py:13-247).  Channel scores, the top-k selection
(including torch's tie order), codes and packing run in
``dkv_quantize_key_pages``.
"""

from __future__ import annotations

import ctypes

from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _lib


@dataclass
class MixedQuantizedKey:
    """Packed keys (fields as reference mixed.py:13-35).

    ``low_values`` [B,H,D,G,nb], ``high_values`` [B,H,K,G,nb] (top-k order),
    ``channel_indices`` [B,H,K] int32, ``scale``/``zero_point`` [B,H,D,G].
    """

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
    def promoted_channels(self) -> int:
        return self.channel_indices.shape[-1]

    @property
    def head_dim(self) -> int:
        return self.original_shape[-1]

    @property
    def shape(self) -> Tuple[int, ...]:
        return self.original_shape

    @property
    def nbytes(self) -> int:
        tensors = (self.low_values, self.high_values, self.channel_indices, self.scale, self.zero_point)
        return sum(t.numel() * t.element_size() for t in tensors)

    @property
    def dense_nbytes(self) -> int:
        n = 1
        for s in self.original_shape:
            n *= s
        return n * torch.tensor([], dtype=self.output_dtype).element_size()

    @property
    def compression_ratio(self) -> float:
        return self.dense_nbytes / self.nbytes if self.nbytes else 1.0

    @property
    def promote_mask(self) -> torch.Tensor:
        mask = torch.zeros((*self.original_shape[:2], self.head_dim), dtype=torch.bool,
                           device=self.channel_indices.device)
        if self.promoted_channels:
            mask.scatter_(-1, self.channel_indices.long(), True)
        return mask

    def dequantize(self, *, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """Materialize [B,H,T,D] on the device (reference mixed.py:72-94 semantics)."""
        out_dtype = dtype or self.output_dtype
        if self.low_values.device.type == "cpu":
            # host-resident pages (a cache moved with .to("cpu")): dequantized on the current GPU
            gpu = torch.device("cuda", torch.cuda.current_device())
            return self.to(gpu).dequantize(dtype=dtype).cpu()
        _lib.require_device(self.low_values)
        B, H, T, D = self.original_shape
        kernel_dtype = out_dtype if out_dtype in _lib.FLOAT_DTYPES else torch.float32
        out = torch.empty(B, H, T, D, dtype=kernel_dtype, device=self.low_values.device)
        fields = [t.contiguous() for t in (self.low_values, self.high_values, self.channel_indices, self.scale,
                                           self.zero_point)]
        lib = _lib.load()
        rc = lib.dkv_dequantize_mixed(*(f.data_ptr() for f in fields), _lib.dtype_code(self.scale.dtype), B, H, D, T,
                                      self.group_size, self.promoted_channels, out.data_ptr(),
                                      _lib.dtype_code(kernel_dtype), _lib.stream_ptr(out.device))
        _lib.check(rc, "dkv_dequantize_mixed")
        return out.to(out_dtype)

    def to(self, device: torch.device | str) -> "MixedQuantizedKey":
        return MixedQuantizedKey(
            low_values=self.low_values.to(device), high_values=self.high_values.to(device),
            channel_indices=self.channel_indices.to(device), scale=self.scale.to(device),
            zero_point=self.zero_point.to(device), original_shape=self.original_shape,
            padded_tokens=self.padded_tokens, group_size=self.group_size, low_bits=self.low_bits,
            promote_bits=self.promote_bits, output_dtype=self.output_dtype,
        )


def promoted_count(head_dim: int, promote_ratio: float) -> int:
    """Number of promoted channels (reference mixed.py:138)."""
    return min(head_dim, int(head_dim * promote_ratio + 1e-6))


def random_channels(heads: int, head_dim: int, count: int, device: torch.device) -> torch.Tensor:
    """One randperm per KV head, shared across the batch (reference mixed.py:145-153)."""
    return torch.stack([torch.randperm(head_dim, device=device)[:count] for _ in range(heads)], dim=0)


def _selection_code(strategy: str) -> int:
    return {"magnitude": _lib.SELECT_MAGNITUDE, "variance": _lib.SELECT_VARIANCE, "random": _lib.SELECT_GIVEN}[strategy]


def select_key_channels(
    key_states: torch.Tensor,
    promote_ratio: float,
    *,
    strategy: str = "magnitude",
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Mask [B,H,D] and indices [B,H,K] of promoted channels (reference mixed.py:119-163)."""
    if key_states.ndim != 4:
        raise ValueError("key_states must have shape [B, H, T, D]")
    if not 0.0 <= promote_ratio <= 1.0:
        raise ValueError("promote_ratio must be in [0, 1]")
    if strategy not in {"magnitude", "random", "variance"}:
        raise ValueError("strategy must be 'magnitude', 'random', or 'variance'")
    batch, heads, _, head_dim = key_states.shape
    count = promoted_count(head_dim, promote_ratio)
    mask = torch.zeros(batch, heads, head_dim, dtype=torch.bool, device=key_states.device)
    if count == 0:
        return mask, torch.empty(batch, heads, 0, dtype=torch.long, device=key_states.device)
    if count == head_dim:
        indices = torch.arange(head_dim, device=key_states.device).view(1, 1, -1).expand(batch, heads, -1)
        return torch.ones_like(mask), indices
    mixed = quantize_key_mixed(key_states, group_size=max(1, key_states.shape[-2]), promote_ratio=promote_ratio,
                               strategy=strategy)
    indices = mixed.channel_indices.long()
    mask.scatter_(-1, indices, True)
    return mask, indices


def quantize_key_mixed(
    key_states: torch.Tensor,
    *,
    group_size: int = 128,
    promote_ratio: float = 0.25,
    promote_bits: int = 4,
    strategy: str = "magnitude",
    metadata_dtype: Optional[torch.dtype] = None,
    channel_indices: Optional[torch.Tensor] = None,
) -> MixedQuantizedKey:
    """Quantize a key chunk [B,H,T,D] with channel promotion (reference mixed.py:166-244).

    ``channel_indices`` ([H, K]) supplies the "random" strategy's per-head
    channel sets; when omitted they are drawn with ``torch.randperm`` like the
    reference.
    """
    if key_states.ndim != 4:
        raise ValueError("key_states must have shape [B, H, T, D]")
    if not torch.is_floating_point(key_states):
        raise TypeError("key_states must be floating point")
    if key_states.shape[-2] == 0 or key_states.shape[-1] == 0:
        raise ValueError("key_states sequence and head dimensions must be non-empty")
    if not isinstance(group_size, int) or group_size <= 0:
        raise ValueError("group_size must be a positive integer")
    if promote_bits != 4:
        raise ValueError("the reference mixed representation currently supports promote_bits=4")
    if not 0.0 <= promote_ratio <= 1.0:
        raise ValueError("promote_ratio must be in [0, 1]")
    if strategy not in {"magnitude", "random", "variance"}:
        raise ValueError("strategy must be 'magnitude', 'random', or 'variance'")
    if not bool(torch.isfinite(key_states).all()):
        raise ValueError("key_states must contain finite values")
    meta = metadata_dtype or (key_states.dtype if key_states.dtype in (torch.float16, torch.bfloat16) else torch.float32)
    if meta not in (torch.float16, torch.bfloat16, torch.float32, torch.float64):
        raise TypeError("metadata_dtype must be floating point")
    _lib.require_device(key_states)
    B, H, T, D = key_states.shape
    K = promoted_count(D, promote_ratio)
    G = (T + group_size - 1) // group_size
    nb = (group_size + 3) // 4
    dev = key_states.device
    low = torch.empty(B, H, D, G, nb, dtype=torch.uint8, device=dev)
    # with no promoted channels the reference allocates nb*4 bytes per group (mixed.py:220-227)
    high = torch.empty(B, H, K, G, nb if K else nb * 4, dtype=torch.uint8, device=dev)
    idx = torch.empty(B, H, K, dtype=torch.int32, device=dev)
    scale = torch.empty(B, H, D, G, dtype=meta, device=dev)
    zero = torch.empty(B, H, D, G, dtype=meta, device=dev)
    given = None
    selection = _selection_code(strategy)
    if strategy == "random" and 0 < K < D:
        given = channel_indices if channel_indices is not None else random_channels(H, D, K, dev)
        given = given.to(device=dev, dtype=torch.int32).contiguous()
    launch_key_pages(key_states, page_tokens=T, n_pages=1, key_mode=_lib.KEY_MIXED, bits=2, group=group_size,
                     promoted=K, selection=selection, given_idx=given, meta=meta,
                     low=low, high=high, idx=idx, scale=scale, zero=zero)
    return MixedQuantizedKey(low_values=low, high_values=high, channel_indices=idx, scale=scale, zero_point=zero,
                             original_shape=tuple(key_states.shape), padded_tokens=G * group_size,
                             group_size=group_size, low_bits=2, promote_bits=promote_bits,
                             output_dtype=key_states.dtype)


def launch_key_pages(src: torch.Tensor, *, page_tokens: int, n_pages: int, key_mode: int, bits: int, group: int,
                     promoted: int, selection: int, given_idx: Optional[torch.Tensor], meta: torch.dtype,
                     low: torch.Tensor, high: Optional[torch.Tensor], idx: Optional[torch.Tensor],
                     scale: torch.Tensor, zero: torch.Tensor, values=None, nonfinite: int = 0,
                     slot: int = 0) -> None:
    """Quantize ``n_pages`` pages of keys from ``src`` [B,H,T,D] into page-major outputs.

    Each output tensor has the page index as its leading dim when n_pages > 1
    (and may omit it when n_pages == 1 and ``slot`` is 0); page strides are
    taken from dim 0, and the pages written are [slot, slot + n_pages).
    ``values`` (a ``_lib.ValueRowsArgs``) adds the same tokens' value rows to
    the call: the library quantizes them alongside the key path.  ``nonfinite`` is
    the address of a device uint32 the kernels set on a NaN or an infinity (0: no check).
    """
    B, H, _, D = src.shape

    def page_stride(t: Optional[torch.Tensor]) -> int:
        if t is None or n_pages <= 1:
            return 0
        return t.stride(0) * t.element_size()

    def page(t: Optional[torch.Tensor]) -> int:
        if t is None:
            return 0
        return t.data_ptr() + (slot * t.stride(0) * t.element_size() if slot else 0)

    a = _lib.KeyPagesArgs()
    a.src = src.data_ptr()
    a.src_dtype = _lib.dtype_code(src.dtype)
    a.B, a.H, a.D = B, H, D
    a.page_tokens, a.n_pages = page_tokens, n_pages
    a.sb, a.sh, a.st, a.sd = src.stride()
    a.key_mode, a.bits, a.group = key_mode, bits, group
    a.promoted, a.selection = promoted, selection
    a.given_idx = _lib.ptr(given_idx)
    a.meta_dtype = _lib.dtype_code(meta)
    a.low, a.low_page_stride = page(low), page_stride(low)
    a.high, a.high_page_stride = page(high), page_stride(high)
    a.idx, a.idx_page_stride = page(idx), page_stride(idx)
    a.scale, a.scale_page_stride = page(scale), page_stride(scale)
    a.zero, a.zero_page_stride = page(zero), page_stride(zero)
    a.values = 0 if values is None else ctypes.addressof(values)
    a.nonfinite = nonfinite or None
    lib = _lib.load()
    _lib.check(lib.dkv_quantize_key_pages(a, _lib.stream_ptr(src.device)), "dkv_quantize_key_pages")


__all__ = ["MixedQuantizedKey", "quantize_key_mixed", "select_key_channels"]

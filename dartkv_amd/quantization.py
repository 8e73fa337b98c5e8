"""Group-wise affine quantization with LSB-first bit packing (HIP-backed).

Same public surface, field layout, validation order and error messages as the
reference ``dart.quantization`` (reference src/dart/quantization.py:17-226);
the arithmetic runs in ``dkv_quantize_rows`` / ``dkv_dequantize_rows``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _lib

_SUPPORTED_BITS = (2, 4, 8)


def _validate_bits(bits: int) -> None:
    if bits not in _SUPPORTED_BITS:
        raise ValueError(f"bits must be one of {_SUPPORTED_BITS}, got {bits}")


def _metadata_dtype(data: torch.Tensor, requested: Optional[torch.dtype]) -> torch.dtype:
    """reference quantization.py:48-53."""
    if requested is not None:
        if requested not in (torch.float16, torch.bfloat16, torch.float32, torch.float64):
            raise TypeError(f"metadata dtype must be floating point, got {requested}")
        return requested
    return data.dtype if data.dtype in (torch.float16, torch.bfloat16) else torch.float32


def _numel(shape: Tuple[int, ...]) -> int:
    result = 1
    for size in shape:
        result *= size
    return result


@dataclass
class QuantizedTensor:
    """A bit-packed affine-quantized tensor (fields as reference quantization.py:56-76).

    ``zero_point`` stores the floating-point group minimum.  ``values`` holds
    ``packed_dim // (8 // bits)`` bytes per row of the quantized axis.
    """

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
    def shape(self) -> Tuple[int, ...]:
        return self.original_shape

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.values, self.scale, self.zero_point))

    @property
    def dense_nbytes(self) -> int:
        return _numel(self.original_shape) * torch.tensor([], dtype=self.output_dtype).element_size()

    @property
    def compression_ratio(self) -> float:
        return self.dense_nbytes / self.nbytes if self.nbytes else 1.0

    def dequantize(self, *, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """Materialize on the device (reference quantization.py:96-109 semantics)."""
        out_dtype = dtype or self.output_dtype
        if self.values.device.type == "cpu":
            # host-resident pages (a cache moved with .to("cpu")): dequantized on the current GPU
            gpu = torch.device("cuda", torch.cuda.current_device())
            return self.to(gpu).dequantize(dtype=dtype).cpu()
        _lib.require_device(self.values)
        ndim = len(self.original_shape)
        axis = self.axis if self.axis >= 0 else ndim + self.axis
        moved = tuple(s for i, s in enumerate(self.original_shape) if i != axis) + (self.original_shape[axis],)
        rows = _numel(moved[:-1])
        n = self.original_dim
        values = self.values.reshape(rows, -1)
        scale = self.scale.reshape(rows, -1)
        zero = self.zero_point.reshape(rows, -1)
        if not (values.is_contiguous() and scale.is_contiguous() and zero.is_contiguous()):
            values, scale, zero = values.contiguous(), scale.contiguous(), zero.contiguous()
        kernel_dtype = out_dtype if out_dtype in _lib.FLOAT_DTYPES else torch.float32
        out = torch.empty(rows, n, dtype=kernel_dtype, device=self.values.device)
        lib = _lib.load()
        rc = lib.dkv_dequantize_rows(values.data_ptr(), scale.data_ptr(), zero.data_ptr(),
                                     _lib.dtype_code(self.scale.dtype), rows, n, self.bits, self.group_size,
                                     out.data_ptr(), _lib.dtype_code(kernel_dtype), n,
                                     _lib.stream_ptr(out.device))
        _lib.check(rc, "dkv_dequantize_rows")
        out = out.reshape(moved).to(out_dtype)
        if axis != ndim - 1:
            out = out.movedim(-1, axis)
        return out

    def to(self, device: torch.device | str) -> "QuantizedTensor":
        return QuantizedTensor(
            values=self.values.to(device), scale=self.scale.to(device), zero_point=self.zero_point.to(device),
            original_shape=self.original_shape, original_dim=self.original_dim, padded_dim=self.padded_dim,
            packed_dim=self.packed_dim, group_size=self.group_size, bits=self.bits,
            output_dtype=self.output_dtype, axis=self.axis,
        )


def _check_finite(data: torch.Tensor, message: str) -> None:
    if not bool(torch.isfinite(data).all()):
        raise ValueError(message)


def quantize(
    data: torch.Tensor,
    *,
    bits: int = 2,
    group_size: int = 64,
    metadata_dtype: Optional[torch.dtype] = None,
    axis: int = -1,
) -> QuantizedTensor:
    """Quantize ``data`` along ``axis`` (reference quantization.py:134-204).

    Groups are asymmetric min/max affine ranges; the last group is padded by
    repeating the final element.  Codes, scales and zero points are
    bit-identical to the reference on the same input.
    """
    _validate_bits(bits)
    if not isinstance(group_size, int) or group_size <= 0:
        raise ValueError(f"group_size must be a positive integer, got {group_size}")
    if data.ndim == 0:
        raise ValueError("quantize expects a tensor with at least one dimension")
    if not torch.is_floating_point(data):
        raise TypeError(f"quantize expects a floating-point tensor, got {data.dtype}")
    if data.shape[-1] == 0:
        raise ValueError("quantize does not support an empty final dimension")
    _check_finite(data, "quantize expects all values to be finite")
    original_shape = tuple(data.shape)
    if not isinstance(axis, int) or not -data.ndim <= axis < data.ndim:
        raise ValueError(f"axis must be in [-{data.ndim}, {data.ndim}), got {axis}")
    axis = axis % data.ndim
    _lib.require_device(data)
    moved = data.movedim(axis, -1).contiguous()
    n = moved.shape[-1]
    groups = (n + group_size - 1) // group_size
    padded = groups * group_size
    per_byte = 8 // bits
    packed_dim = ((padded + per_byte - 1) // per_byte) * per_byte
    meta = _metadata_dtype(moved, metadata_dtype)
    outer = moved.shape[:-1]
    rows = _numel(outer)
    dev = data.device
    values = torch.empty(*outer, packed_dim // per_byte, dtype=torch.uint8, device=dev)
    scale = torch.empty(*outer, groups, dtype=meta, device=dev)
    zero = torch.empty(*outer, groups, dtype=meta, device=dev)
    if rows:
        lib = _lib.load()
        rc = lib.dkv_quantize_rows(moved.data_ptr(), _lib.dtype_code(moved.dtype), rows, n, n, 1, bits, group_size,
                                   values.data_ptr(), scale.data_ptr(), zero.data_ptr(), _lib.dtype_code(meta),
                                   _lib.stream_ptr(dev))
        _lib.check(rc, "dkv_quantize_rows")
    return QuantizedTensor(values=values, scale=scale, zero_point=zero, original_shape=original_shape,
                           original_dim=n, padded_dim=padded, packed_dim=packed_dim, group_size=group_size,
                           bits=bits, output_dtype=data.dtype, axis=axis)


def dequantize(data: QuantizedTensor, *, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Functional alias for :meth:`QuantizedTensor.dequantize`."""
    return data.dequantize(dtype=dtype)


def quantize_axis(
    data: torch.Tensor,
    axis: int,
    *,
    bits: int = 2,
    group_size: int = 64,
    metadata_dtype: Optional[torch.dtype] = None,
) -> QuantizedTensor:
    """Explicit spelling for quantization along a non-last axis (reference quantization.py:213-223)."""
    return quantize(data, bits=bits, group_size=group_size, metadata_dtype=metadata_dtype, axis=axis)


__all__ = ["QuantizedTensor", "dequantize", "quantize", "quantize_axis"]

"""Compatibility names for the reference's Triton helpers (reference src/dart/triton_ops.py:310-327).

This build has no Triton: ``TRITON_AVAILABLE`` is False and
``triton_dequantize`` runs the HIP dequantize kernels (the same result the
reference's ``.dequantize()`` gives, bit for bit).
"""

from __future__ import annotations

from typing import Optional

import torch

from .mixed import MixedQuantizedKey
from .quantization import QuantizedTensor

TRITON_AVAILABLE = False


def triton_available() -> bool:
    return TRITON_AVAILABLE


def triton_dequantize(data: QuantizedTensor | MixedQuantizedKey, *, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Dequantize on the device with the HIP kernels."""
    return data.dequantize(dtype=dtype)


__all__ = ["TRITON_AVAILABLE", "triton_available", "triton_dequantize"]

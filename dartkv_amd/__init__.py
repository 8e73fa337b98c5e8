"""dartkv_amd: MI355X-native (HIP, gfx950) compressed-KV path with the DartKV Python API.

The public names match the reference package ``dart`` (reference
src/dart/__init__.py:3-34), so ``import dartkv_amd as dart`` is a drop-in for
the compressed-KV path.  Compute runs in ``libdartkv_hip.so`` (C ABI in
include/dartkv.h); there is no CPU fallback.
"""

from .attention import decode_attention, dense_attention, streamed_dart_attention
from .cache import DartKVCache, DartKVCacheConfig, DartPageMetadata, DartSegmentLayout
from .fused_attention import fused_dart_attention
from .mixed import MixedQuantizedKey, quantize_key_mixed, select_key_channels
from .page_table import DENSE_PAGE, MIXED_PAGE, QUANTIZED_PAGE, DartPageRun, DartPageTable
from .quantization import QuantizedTensor, dequantize, quantize, quantize_axis
from .triton_ops import TRITON_AVAILABLE, triton_available, triton_dequantize
from . import torch_ops  # registers torch.ops.dartkv.*

__all__ = [
    "DartKVCache",
    "DartKVCacheConfig",
    "DartPageMetadata",
    "DartSegmentLayout",
    "dense_attention",
    "decode_attention",
    "fused_dart_attention",
    "DENSE_PAGE",
    "MIXED_PAGE",
    "QUANTIZED_PAGE",
    "DartPageTable",
    "DartPageRun",
    "QuantizedTensor",
    "MixedQuantizedKey",
    "dequantize",
    "quantize",
    "quantize_axis",
    "quantize_key_mixed",
    "select_key_channels",
    "streamed_dart_attention",
    "TRITON_AVAILABLE",
    "triton_available",
    "triton_dequantize",
]

__version__ = "0.1.0"

"""ctypes binding of libdartkv_hip.so (the C ABI declared in include/dartkv.h).

The library is loaded on first use.  There is no CPU fallback: compute entry
points raise if the library is missing or a tensor is not on a ROCm device.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdartkv_hip.so")

DKV_OK = 0
DKV_ERR_INVALID = 1
DKV_ERR_UNSUPPORTED = 2
DKV_ERR_DTYPE = 3
DKV_ERR_HIP = 4

KEY_DENSE, KEY_UNIFORM, KEY_MIXED = 0, 1, 2
VALUE_DENSE, VALUE_UNIFORM = 0, 1
SELECT_MAGNITUDE, SELECT_VARIANCE, SELECT_GIVEN = 0, 1, 2

ABI_VERSION = 13

_DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.float64: 3}
# element types the kernels read and write (sources, outputs, metadata)
FLOAT_DTYPES = (torch.float64, torch.float32, torch.float16, torch.bfloat16)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}") from None


class ValueRowsArgs(ctypes.Structure):
    _fields_ = [
        ("src", ctypes.c_void_p), ("src_dtype", ctypes.c_int64),
        ("blocks", ctypes.c_int64), ("block_stride", ctypes.c_int64), ("block_rows", ctypes.c_int64),
        ("n", ctypes.c_int64), ("row_stride", ctypes.c_int64),
        ("bits", ctypes.c_int64), ("group", ctypes.c_int64),
        ("values", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("zero", ctypes.c_void_p),
        ("meta_dtype", ctypes.c_int64), ("nonfinite", ctypes.c_void_p),
        ("out_block_rows", ctypes.c_int64), ("out_row0", ctypes.c_int64),
    ]


class KeyPagesArgs(ctypes.Structure):
    _fields_ = [
        ("src", ctypes.c_void_p), ("src_dtype", ctypes.c_int64),
        ("B", ctypes.c_int64), ("H", ctypes.c_int64), ("D", ctypes.c_int64),
        ("page_tokens", ctypes.c_int64), ("n_pages", ctypes.c_int64),
        ("sb", ctypes.c_int64), ("sh", ctypes.c_int64), ("st", ctypes.c_int64), ("sd", ctypes.c_int64),
        ("key_mode", ctypes.c_int64), ("bits", ctypes.c_int64), ("group", ctypes.c_int64),
        ("promoted", ctypes.c_int64), ("selection", ctypes.c_int64),
        ("given_idx", ctypes.c_void_p), ("meta_dtype", ctypes.c_int64),
        ("low", ctypes.c_void_p), ("low_page_stride", ctypes.c_int64),
        ("high", ctypes.c_void_p), ("high_page_stride", ctypes.c_int64),
        ("idx", ctypes.c_void_p), ("idx_page_stride", ctypes.c_int64),
        ("scale", ctypes.c_void_p), ("scale_page_stride", ctypes.c_int64),
        ("zero", ctypes.c_void_p), ("zero_page_stride", ctypes.c_int64),
        ("values", ctypes.c_void_p),  # const dkv_value_rows_args* (optional)
        ("nonfinite", ctypes.c_void_p),  # uint32_t* (optional)
        ("copies", ctypes.c_void_p), ("n_copies", ctypes.c_int64),  # const dkv_copy_block* (optional)
    ]


class Segment(ctypes.Structure):
    _fields_ = [
        ("tokens", ctypes.c_int32), ("key_kind", ctypes.c_int32), ("value_kind", ctypes.c_int32),
        ("key_bits", ctypes.c_int32), ("key_group", ctypes.c_int32), ("promoted", ctypes.c_int32),
        ("value_bits", ctypes.c_int32), ("value_group", ctypes.c_int32),
        ("key", ctypes.c_uint64 * 5), ("key_bh", ctypes.c_int64 * 5),
        ("value", ctypes.c_uint64 * 3), ("value_bh", ctypes.c_int64 * 3),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("query", ctypes.c_void_p), ("q_dtype", ctypes.c_int64), ("q_sb", ctypes.c_int64), ("q_sh", ctypes.c_int64),
        ("out", ctypes.c_void_p), ("out_sb", ctypes.c_int64), ("out_sh", ctypes.c_int64),
        ("out_f32", ctypes.c_void_p),
        ("segments", ctypes.c_void_p), ("n_segments", ctypes.c_int64),
        ("tail", Segment),
        ("B", ctypes.c_int64), ("Hq", ctypes.c_int64), ("Hkv", ctypes.c_int64), ("D", ctypes.c_int64),
        ("cache_dtype", ctypes.c_int64), ("meta_dtype", ctypes.c_int64),
        ("scale", ctypes.c_double),
        ("n_splits", ctypes.c_int64),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
        ("fast_first", ctypes.c_int64), ("fast_count", ctypes.c_int64), ("fast_promoted", ctypes.c_int64),
        ("fast_value_group", ctypes.c_int64), ("fast_splits", ctypes.c_int64),
        ("rest_dense_tokens", ctypes.c_int64),
        ("fast_events", ctypes.c_void_p * 2),
        ("tail_tokens_dev", ctypes.c_void_p),
        ("fast_key_bits", ctypes.c_int64), ("fast_value_bits", ctypes.c_int64),
        ("segments_host", ctypes.c_void_p),
    ]


assert ctypes.sizeof(Segment) == 160


class DecodePrepArgs(ctypes.Structure):
    _fields_ = [
        ("qkv", ctypes.c_void_p), ("qkv_sb", ctypes.c_int64),
        ("q_weight", ctypes.c_void_p), ("k_weight", ctypes.c_void_p), ("eps", ctypes.c_double),
        ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p), ("q_out", ctypes.c_void_p),
        ("tail_key", ctypes.c_void_p), ("tail_value", ctypes.c_void_p), ("tail_pos", ctypes.c_void_p),
        ("B", ctypes.c_int64), ("Hq", ctypes.c_int64), ("Hkv", ctypes.c_int64), ("D", ctypes.c_int64),
        ("cap", ctypes.c_int64), ("dtype", ctypes.c_int64),
    ]


class CopyBlock(ctypes.Structure):
    _fields_ = [
        ("src", ctypes.c_void_p), ("dst", ctypes.c_void_p),
        ("B", ctypes.c_int64), ("H", ctypes.c_int64), ("T", ctypes.c_int64), ("row_bytes", ctypes.c_int64),
        ("src_sb", ctypes.c_int64), ("src_sh", ctypes.c_int64), ("src_st", ctypes.c_int64),
        ("dst_sb", ctypes.c_int64), ("dst_sh", ctypes.c_int64), ("dst_st", ctypes.c_int64),
    ]


COPY_MAX_BLOCKS = 8

EXPORTED = (
    "dkv_last_error", "dkv_abi_version", "dkv_quantize_rows", "dkv_quantize_row_blocks", "dkv_quantize_value_rows",
    "dkv_quantize_key_pages",
    "dkv_dequantize_rows",
    "dkv_dequantize_mixed", "dkv_decode_workspace_bytes", "dkv_decode_attention", "dkv_decode_attention_noalloc",
    "dkv_decode_scratch_bytes", "dkv_decode_prep", "dkv_copy_token_blocks",
)

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load libdartkv_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing; build it with `python -m dartkv_amd.build` "
                "(dartkv_amd has no CPU fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        lib.dkv_last_error.restype = ctypes.c_char_p
        lib.dkv_abi_version.restype = ctypes.c_int
        lib.dkv_quantize_rows.argtypes = [vp, i32, i64, i64, i64, i64, i32, i64, vp, vp, vp, i32, vp]
        lib.dkv_quantize_row_blocks.argtypes = [vp, i32, i64, i64, i64, i64, i64, i32, i64, vp, vp, vp, i32, vp]
        lib.dkv_quantize_value_rows.argtypes = [ctypes.POINTER(ValueRowsArgs), vp]
        lib.dkv_quantize_key_pages.argtypes = [ctypes.POINTER(KeyPagesArgs), vp]
        lib.dkv_dequantize_rows.argtypes = [vp, vp, vp, i32, i64, i64, i32, i64, vp, i32, i64, vp]
        lib.dkv_dequantize_mixed.argtypes = [vp, vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, i64, vp, i32, vp]
        lib.dkv_decode_workspace_bytes.argtypes = [i64, i64, i64, i64]
        lib.dkv_decode_workspace_bytes.restype = i64
        lib.dkv_decode_attention.argtypes = [ctypes.POINTER(DecodeArgs), vp]
        lib.dkv_decode_attention_noalloc.argtypes = [ctypes.POINTER(DecodeArgs), vp]
        lib.dkv_decode_scratch_bytes.argtypes = []
        lib.dkv_decode_scratch_bytes.restype = i64
        lib.dkv_decode_prep.argtypes = [ctypes.POINTER(DecodePrepArgs), vp]
        lib.dkv_copy_token_blocks.argtypes = [ctypes.POINTER(CopyBlock), i64, vp]
        for name in ("dkv_quantize_rows", "dkv_quantize_row_blocks", "dkv_quantize_value_rows", "dkv_quantize_key_pages",
                     "dkv_dequantize_rows",
                     "dkv_dequantize_mixed", "dkv_decode_attention", "dkv_decode_attention_noalloc",
                     "dkv_decode_prep", "dkv_copy_token_blocks"):
            getattr(lib, name).restype = ctypes.c_int
        if lib.dkv_abi_version() != ABI_VERSION:
            raise RuntimeError("libdartkv_hip.so ABI version mismatch; rebuild it")
        _lib = lib
    return _lib


def check(rc: int, where: str) -> None:
    """Map a C status code to the Python exception the reference raises."""
    if rc == DKV_OK:
        return
    msg = load().dkv_last_error().decode(errors="replace")
    if rc == DKV_ERR_DTYPE:
        raise TypeError(msg)
    if rc in (DKV_ERR_INVALID, DKV_ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(f"{where}: {msg}")


def require_device(*tensors: torch.Tensor) -> None:
    """All compute runs on the ROCm device; CPU tensors are an error, not a fallback."""
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(
                f"dartkv_amd computes on a ROCm GPU; got a tensor on {t.device}. "
                "Move the tensors to the GPU (there is no CPU fallback).")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device) -> int:
    """The current HIP stream of ``device`` (what torch.cuda.current_stream(device).cuda_stream gives,
    read without building a Stream object)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


def ptr(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else t.data_ptr()


def copy_token_blocks(pairs, device: torch.device) -> None:
    """dst.copy_(src) for each (dst, src) pair of [B, H, T, D] tensors of one dtype on ``device``, up to
    COPY_MAX_BLOCKS pairs per launch (dkv_copy_token_blocks); the last dimension must be contiguous."""
    for dst, src in pairs:
        if dst.shape != src.shape or dst.dtype != src.dtype or dst.dim() != 4:
            raise ValueError("copy_token_blocks: pairs must be [B, H, T, D] tensors of one shape and dtype")
        if dst.stride(3) != 1 or src.stride(3) != 1:
            raise ValueError("copy_token_blocks: the last dimension must be contiguous")
    lib = load()
    stream = stream_ptr(device)
    for at in range(0, len(pairs), COPY_MAX_BLOCKS):
        chunk = pairs[at:at + COPY_MAX_BLOCKS]
        blocks = (CopyBlock * len(chunk))()
        for blk, (dst, src) in zip(blocks, chunk):
            e = src.element_size()
            blk.src, blk.dst = src.data_ptr(), dst.data_ptr()
            blk.B, blk.H, blk.T, _ = src.shape
            blk.row_bytes = src.shape[3] * e
            blk.src_sb, blk.src_sh, blk.src_st = src.stride(0) * e, src.stride(1) * e, src.stride(2) * e
            blk.dst_sb, blk.dst_sh, blk.dst_st = dst.stride(0) * e, dst.stride(1) * e, dst.stride(2) * e
        check(lib.dkv_copy_token_blocks(blocks, len(chunk), stream), "dkv_copy_token_blocks")

"""Attention over DartKV caches (reference src/dart/attention.py:1-90).

* ``dense_attention``: eager fp32 attention on dense tensors (a plain
  reference for tests and the materialized path).
* ``streamed_dart_attention``: attention over the packed cache without
  materializing it.  One query token runs the HIP split-K decode kernel;
  several query tokens dequantize one segment at a time with the HIP
  dequantize kernels and keep an online softmax on the GPU.
* ``decode_attention``: the single-token kernel entry used by both
  ``streamed_dart_attention`` and ``fused_dart_attention``.
"""

from __future__ import annotations

import collections
import ctypes
import math
import os
from typing import Optional, Tuple

import torch

from . import _lib
from .cache import DartKVCache, _dense16_ok, _materialize, tail_segment

# The HIP decode kernels take at most this many query heads per KV head and this head_dim
# (decode.hip kMaxGroup / kMaxDim); larger shapes run segment_attention.
MAX_GROUP, MAX_HEAD_DIM = 16, 512


def dense_attention(query: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, *,
                    scale: Optional[float] = None) -> torch.Tensor:
    """Eager attention for [B, H, Q/T, D] tensors (reference attention.py:14-29)."""
    if query.ndim != 4 or keys.ndim != 4 or values.ndim != 4:
        raise ValueError("query, keys, and values must have shape [B, H, T, D]")
    if keys.shape != values.shape or query.shape[0] != keys.shape[0] or query.shape[-1] != keys.shape[-1]:
        raise ValueError("query/key/value batch, head_dim, and key/value shapes must be compatible")
    factor = scale if scale is not None else 1.0 / math.sqrt(query.shape[-1])
    logits = torch.matmul(query.float(), keys.float().transpose(-1, -2)) * factor
    return torch.matmul(torch.softmax(logits, dim=-1), values.float()).to(query.dtype)


def _check_query(query: torch.Tensor, cache: DartKVCache):
    if cache.get_seq_length() == 0 or cache.shape is None:
        raise ValueError("cache is empty")
    batch, kv_heads, _, head_dim = cache.shape
    if query.shape[0] != batch or query.shape[-1] != head_dim:
        raise ValueError("query batch and head_dim must match the cache")
    if query.shape[1] % kv_heads:
        raise ValueError("query heads must be divisible by cache KV heads")
    return batch, kv_heads, head_dim


def default_splits(batch: int, kv_heads: int, n_segments: int, target: int = 4096) -> int:
    """Split count that gives the 256-CU device a few thousand workers."""
    return max(1, min(n_segments, -(-target // max(1, batch * kv_heads))))


def page_kernel_splits(batch: int, kv_heads: int, pages: int) -> int:
    """Split count of the MFMA page kernel.

    One wave per split.  About 2,048 waves fill the device once (256 CUs x 8
    resident waves); beyond that, up to 16 splits of at least 4 pages each
    still help, since each split pays a fixed prologue.  Measured optimum at
    C5 (512 (batch, kv head) pairs x 255 pages) and C4 (128 x 63): 16.
    """
    bh = max(1, batch * kv_heads)
    return max(1, min(pages, max(-(-2048 // bh), min(16, -(-pages // 4)))))


_FAST_ENABLED: Optional[bool] = None
_NO_TAIL = _lib.Segment()  # the descriptor of no held tail (read only)


def _fast_enabled() -> bool:
    """False when the environment sets DKV_FORCE_GENERAL (read on first use: a decode call does not pay
    for an environment lookup)."""
    global _FAST_ENABLED
    if _FAST_ENABLED is None:
        _FAST_ENABLED = os.environ.get("DKV_FORCE_GENERAL", "0") in ("", "0")
    return _FAST_ENABLED


_workspaces: "collections.OrderedDict[tuple, torch.Tensor]" = collections.OrderedDict()
_MAX_WORKSPACES = 8  # (device, stream) pairs whose workspace is kept; the least recently used goes first


def _workspace(device: torch.device, nbytes: int, stream: Optional[int] = None) -> torch.Tensor:
    """A decode workspace for the split records: one per device and stream, kept and grown as needed (calls
    on one stream run in order, so they can share it).  At most ``_MAX_WORKSPACES`` are kept (least recently
    used dropped first; the caching allocator reuses a dropped one once the stream's work has run) and
    ``release_workspaces`` drops them all.  Under graph capture a fresh one, which the graph keeps."""
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    key = (device.index, _lib.stream_ptr(device) if stream is None else stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = _workspaces[key] = torch.empty(nbytes, dtype=torch.uint8, device=device)
        while len(_workspaces) > _MAX_WORKSPACES:
            _workspaces.popitem(last=False)
    _workspaces.move_to_end(key)
    return ws


def release_workspaces() -> None:
    """Drop the kept decode workspaces (their memory returns to torch's caching allocator, so
    ``torch.cuda.empty_cache`` can free it)."""
    _workspaces.clear()


def _call_layout(plan, cache: DartKVCache, q3: torch.Tensor, kv_heads: int, head_dim: int, tail, use_fast: bool,
                 dense_ok: bool, n_splits: Optional[int], factor: float):
    """The parts of a decode call's arguments that depend only on the plan and the call's shape: split
    counts, the kernels' descriptors and options (a ``DecodeArgs`` without the per-call pointers), and the
    workspace size.  Kept per plan and call shape."""
    batch, Hq = q3.shape[0], q3.shape[1]
    group = Hq // kv_heads
    fast_count = plan.fast_count if use_fast else 0
    rest = plan.count - fast_count + (1 if tail.tokens > 0 else 0)
    # the dense kernel takes the non-page segments (sink, tail) when they are
    # all dense: one record per 32-token chunk of each
    dense_tokens = 0
    # (more than 8 heads per KV head only as waves of the Dart page kernel's launch)
    if (use_fast and rest and (group <= 8 or (fast_count and plan.fast_promoted)) and plan.rest_dense >= 0
            and dense_ok):
        dense_tokens = max(plan.rest_dense, tail.tokens)
    if fast_count:
        # the uniform page kernel splits over half pages
        units = fast_count if plan.fast_promoted else 2 * fast_count
        fast_splits = n_splits or page_kernel_splits(batch, kv_heads, units)
        fast_splits = max(1, min(fast_splits, units))
        splits = rest * -(-dense_tokens // 32) if dense_tokens else (max(1, min(rest, 4)) if rest else 0)
    else:
        fast_splits = 0
        splits = n_splits or default_splits(batch, kv_heads, rest)
        splits = max(1, min(splits, max(1, rest)))
    a = _lib.DecodeArgs()
    a.q_dtype = _lib.dtype_code(q3.dtype)
    a.q_sb, a.q_sh = q3.stride(0), q3.stride(1)
    a.segments = 0 if plan.table is None else plan.table.data_ptr()
    a.n_segments = plan.count
    a.segments_host = None if plan.host_table is None else ctypes.addressof(plan.host_table)
    a.B, a.Hq, a.Hkv, a.D = batch, Hq, kv_heads, head_dim
    a.cache_dtype = _lib.dtype_code(cache.dtype)
    a.meta_dtype = _lib.dtype_code(cache.config.metadata_dtype)
    a.scale = float(factor)
    a.n_splits = splits
    a.workspace_bytes = _lib.load().dkv_decode_workspace_bytes(batch, Hq, head_dim, splits + fast_splits)
    if fast_count:
        a.fast_first, a.fast_count = plan.fast_first, fast_count
        a.fast_promoted, a.fast_value_group, a.fast_splits = plan.fast_promoted, plan.fast_value_group, fast_splits
        a.fast_key_bits, a.fast_value_bits = plan.fast_key_bits, plan.fast_value_bits
    # a whole number of chunks: valid for every tail length with this chunk count
    a.rest_dense_tokens = 32 * -(-dense_tokens // 32)
    return a, a.workspace_bytes


def decode_attention(query: torch.Tensor, cache: DartKVCache, *, scale: Optional[float] = None,
                     n_splits: Optional[int] = None, out_f32: Optional[torch.Tensor] = None,
                     fast: Optional[bool] = None, fast_events=None, out: Optional[torch.Tensor] = None,
                     static_scratch: bool = False) -> torch.Tensor:
    """Single-token decode over the packed cache with the HIP split-K kernel.

    ``query`` is [B, Hq, 1, D] (or [B, Hq, D]) on the cache's device.  Returns
    [B, Hq, 1, D] in ``query.dtype``.  If ``out_f32`` ([B, Hq, D] fp32) is
    given it receives the result before the final cast.  ``fast`` selects
    the MFMA page kernel for the pages it supports (default: on unless the
    environment sets DKV_FORCE_GENERAL=1, read at the first call); ``n_splits`` overrides the split
    count of the page kernel (or of the general kernel when it does all work).
    ``fast_events`` (two recorded ``torch.cuda.Event`` objects) are recorded
    again right before and after the page kernel, to time it alone.  ``out``
    ([B, Hq, 1, D] in ``query.dtype``) receives the result instead of a new
    tensor.  ``static_scratch`` keeps the split records in the library's static
    device scratch (``dkv_decode_attention_noalloc``) instead of a workspace
    tensor, so with ``out`` given the call allocates nothing.
    """
    _lib.require_device(query)
    batch, kv_heads, head_dim = _check_query(query, cache)
    # q3: the query as [B, Hq, D] (a [B, Hq, 1, D] query is read through its own strides 0, 1 and 3)
    q3 = query.reshape(query.shape[0], query.shape[1], query.shape[-1]) if query.ndim == 4 and query.shape[2] != 1 \
        else query
    if q3.stride(-1) != 1:
        q3 = q3.contiguous()
    device = query.device
    if device != cache.device:
        raise ValueError("query and cache must be on the same device")
    factor = scale if scale is not None else 1.0 / math.sqrt(head_dim)
    plan = cache.decode_plan(device)
    if plan.tail_is_pending:
        tail, dense_ok = tail_segment(cache, with_dense_check=True)
    else:
        tail, dense_ok = _NO_TAIL, True
    Hq = q3.shape[1]
    use_fast = ((_fast_enabled() if fast is None else fast) and plan.fast_count > 0
                and Hq // kv_heads in _fast_rows(plan))
    chunks = -(-max(plan.rest_dense, tail.tokens) // 32)
    key = (Hq, q3.dtype, q3.stride(0), q3.stride(1), use_fast, n_splits, factor, static_scratch, tail.tokens > 0,
           dense_ok, chunks)
    layout = plan.call_layouts.get(key)
    if layout is None:
        layout = plan.call_layouts[key] = _call_layout(plan, cache, q3, kv_heads, head_dim, tail, use_fast, dense_ok,
                                                       n_splits, factor)
    template, ws_bytes = layout
    if out is None:
        out = torch.empty(batch, Hq, 1, head_dim, dtype=query.dtype, device=query.device)
    elif out.shape != (batch, Hq, 1, head_dim) or out.dtype != query.dtype or out.device != query.device \
            or out.stride(-1) != 1:
        raise ValueError("out must be a [B, Hq, 1, D] tensor of the query's dtype and device, unit stride in D")
    lib = _lib.load()
    stream = _lib.stream_ptr(device)
    workspace = None if static_scratch else _workspace(device, ws_bytes, stream)
    a = _lib.DecodeArgs.from_buffer_copy(template)
    a.query = q3.data_ptr()
    a.out = out.data_ptr()
    a.out_sb, a.out_sh = out.stride(0), out.stride(1)
    if out_f32 is not None:
        if out_f32.shape != (batch, Hq, head_dim) or out_f32.dtype != torch.float32 or not out_f32.is_contiguous():
            raise ValueError("out_f32 must be a contiguous float32 [B, Hq, D] tensor")
        a.out_f32 = out_f32.data_ptr()
    a.tail = tail
    a.workspace = _lib.ptr(workspace)
    if cache.device_tail is not None and plan.tail_is_pending:
        a.tail_tokens_dev = cache.device_tail.data_ptr()
    if fast_events is not None:
        a.fast_events[0], a.fast_events[1] = fast_events[0].cuda_event, fast_events[1].cuda_event
    if static_scratch:
        _lib.check(lib.dkv_decode_attention_noalloc(a, stream), "dkv_decode_attention_noalloc")
    else:
        _lib.check(lib.dkv_decode_attention(a, stream), "dkv_decode_attention")
    return out


def streamed_dart_attention(query: torch.Tensor, cache: DartKVCache, *, scale: Optional[float] = None) -> torch.Tensor:
    """Attend to packed pages without materializing the cache (reference attention.py:32-87).

    GQA maps query head h to KV head h // (Hq / Hkv).
    """
    if query.ndim != 4:
        raise ValueError("query must have shape [B, Hq, Q, D]")
    if cache.get_seq_length() == 0:
        raise ValueError("cache is empty")
    batch, kv_heads, head_dim = _check_query(query, cache)
    _lib.require_device(query)
    if query.shape[1] // kv_heads > MAX_GROUP or head_dim > MAX_HEAD_DIM:
        return segment_attention(query, cache, scale=scale)
    if query.shape[-2] == 1:
        return decode_attention(query, cache, scale=scale)
    return _multi_token_attention(query, cache, scale=scale)


def segment_attention(query: torch.Tensor, cache: DartKVCache, *, scale: Optional[float] = None,
                      out_f32: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Attention over the cache one segment at a time, for shapes the HIP decode kernels do not take
    (more than MAX_GROUP query heads per KV head, head_dim above MAX_HEAD_DIM): each segment is
    dequantized by the HIP dequantize kernels and attended with fp32 logits and an online softmax on
    the GPU, the reference's streamed algorithm (attention.py:32-87).  ``out_f32`` ([B, Hq, Q, D]
    float32) receives the result before the final cast."""
    batch, kv_heads, head_dim = _check_query(query, cache)
    group = query.shape[1] // kv_heads
    factor = scale if scale is not None else 1.0 / math.sqrt(head_dim)
    q = query.float()
    shape = (*query.shape[:3], 1)
    m = torch.full(shape, float("-inf"), device=query.device)
    l = torch.zeros(shape, device=query.device)
    acc = torch.zeros(query.shape, dtype=torch.float32, device=query.device)
    for kseg, vseg in cache.iter_segments():
        k = _materialize(kseg).float().repeat_interleave(group, dim=1)
        v = _materialize(vseg).float().repeat_interleave(group, dim=1)
        logits = torch.matmul(q, k.transpose(-1, -2).contiguous()) * factor
        m_new = torch.maximum(m, logits.amax(dim=-1, keepdim=True))
        p = torch.exp(logits - m_new)
        correction = torch.exp(m - m_new)
        l = l * correction + p.sum(dim=-1, keepdim=True)
        acc = acc * correction + torch.matmul(p, v)
        m = m_new
    out = acc / l.clamp_min(1e-20)
    if out_f32 is not None:
        out_f32.copy_(out)
    return out.to(query.dtype)


def _fast_rows(plan) -> Tuple[int, ...]:
    """Query rows per KV head the MFMA page kernels take: up to 16 on Dart pages, 8 on uniform pages."""
    return (1, 2, 4, 8, 16) if plan.fast_promoted else (1, 2, 4, 8)


def _multi_token_attention(query: torch.Tensor, cache: DartKVCache, *, scale: Optional[float] = None,
                           out_f32: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Several query tokens per head over the packed cache.

    The reference attends every query token to every cached token, with no
    mask (attention.py:67-87), so token i of query head h is one more query
    row of h's KV group.  A [B, Hq, c, D] slice of the query read as a
    [B, Hq * c, D] query keeps that grouping (row h * c + i belongs to KV head
    h // G), and the single-token HIP decode path runs it unchanged: the MFMA
    page kernel while G * c fits its rows per KV head (8, or 16 on Dart pages:
    the dequantized pages serve all rows of a launch), the general kernel up to
    16.  ``out_f32`` ([B, Hq, Q, D] float32) receives the result before the cast.
    """
    batch, kv_heads, head_dim = cache.shape[0], cache.shape[1], cache.shape[3]
    Hq, Q = query.shape[1], query.shape[-2]
    groups = Hq // kv_heads
    plan = cache.decode_plan(query.device)
    rows = _fast_rows(plan) if plan.fast_count > 0 and _fast_enabled() else (1, 2, 4)
    fits = [c for c in range(1, Q + 1) if groups * c in rows]  # token counts a page-kernel launch takes
    if out_f32 is not None and (out_f32.shape != (batch, Hq, Q, head_dim) or out_f32.dtype != torch.float32):
        raise ValueError("out_f32 must be a float32 [B, Hq, Q, D] tensor")
    out = torch.empty(batch, Hq, Q, head_dim, dtype=query.dtype, device=query.device)
    start = 0
    while start < Q:
        left = [c for c in fits if c <= Q - start]
        c = max(left) if left else min(Q - start, max(1, 16 // groups))
        q_rows = query[:, :, start:start + c].reshape(batch, Hq * c, head_dim)
        o32 = None if out_f32 is None else torch.empty(batch, Hq * c, head_dim, dtype=torch.float32,
                                                       device=query.device)
        o = decode_attention(q_rows, cache, scale=scale, out_f32=o32)
        out[:, :, start:start + c] = o.reshape(batch, Hq, c, head_dim)
        if out_f32 is not None:
            out_f32[:, :, start:start + c] = o32.reshape(batch, Hq, c, head_dim)
        start += c
    return out


__all__ = ["dense_attention", "streamed_dart_attention", "decode_attention"]

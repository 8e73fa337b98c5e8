"""dkv_decode_attention_noalloc (static device scratch, no allocation) against dkv_decode_attention (GPU).

Both entry points run the same kernels with the same split counts; only the
address of the split records differs, so outputs must agree bit for bit.  Two
calls in a row (the second smaller) check that records left by the first call
do not leak into the second; Dart pages, uniform pages and an fp32 cache (the
general kernel) cover every decode kernel.
"""

from __future__ import annotations

import pytest
import torch

from tests.golden_util import bits_equal

DEV = "cuda"


def _cache(B, T, dtype, **over):
    import dartkv_amd as dart
    from dartkv_amd import synthetic
    cfg = dict(bits=2, page_size=128, key_group_size=128, value_group_size=64, promote_ratio=0.25, sink_tokens=32,
               hold_partial_pages=True, metadata_dtype=torch.float16)
    cfg.update(over)
    k, v, q = synthetic.outlier_kv(B, 8, T, 128, query_heads=32, dtype=dtype, seed=B * 1000 + T, device=DEV)
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    cache.append(k, v)
    return cache, q


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["dart_pages", "uniform_pages", "fp32_general"])
def test_noalloc_decode_equals_the_workspace_entry_point(kind):
    import dartkv_amd as dart
    over = {"dart_pages": {}, "uniform_pages": dict(bits=4, promote_ratio=0.0),
            "fp32_general": dict(metadata_dtype=torch.float32)}[kind]
    dtype = torch.float32 if kind == "fp32_general" else torch.bfloat16
    for B, T in ((6, 3000), (2, 700)):  # the second call is smaller than the first
        print("case", kind, B, T, flush=True)
        cache, q = _cache(B, T, dtype, **over)
        ref32 = torch.empty(B, 32, 128, dtype=torch.float32, device=DEV)
        ref = dart.decode_attention(q, cache, out_f32=ref32)
        out = torch.full((B, 32, 1, 128), float("nan"), dtype=dtype, device=DEV)
        out32 = torch.full((B, 32, 128), float("nan"), dtype=torch.float32, device=DEV)
        got = dart.decode_attention(q, cache, out_f32=out32, out=out, static_scratch=True)
        torch.cuda.synchronize()
        assert got.data_ptr() == out.data_ptr()
        assert bits_equal(out32.cpu(), ref32.cpu()), kind
        assert bits_equal(out.cpu(), ref.cpu()), kind


def test_noalloc_decode_rejects_records_beyond_the_scratch():
    """Host-side check (no device work): records beyond the static scratch are an error, not an allocation."""
    from dartkv_amd import _lib
    lib = _lib.load()
    assert lib.dkv_decode_scratch_bytes() == 32 << 20
    a = _lib.DecodeArgs()
    a.B, a.Hq, a.Hkv, a.D = 64, 32, 8, 128
    a.n_segments, a.segments = 1, 16  # never read: the size check comes first
    a.n_splits = 8000  # 8000 * 64 * 32 * 130 * 4 bytes of records
    assert lib.dkv_decode_workspace_bytes(64, 32, 128, 8000) > lib.dkv_decode_scratch_bytes()
    assert lib.dkv_decode_attention_noalloc(a, None) == _lib.DKV_ERR_INVALID
    assert b"static scratch" in lib.dkv_last_error()

"""Parity at the benchmarked sizes (GPU): the caches and decode calls bench.py times.

* C5 (batch 64, 32,768-token context, 8 KV / 32 query heads, head_dim 128):
  one layer of the 2-bit + 25 % cache and one of the 4-bit uniform cache.
  The 2-bit + 25 % prefill (130,560 key pages) takes the separate
  channel-selection launch used above 8,192 pages.  Sequences 0 and 63 are
  compared with the CPU oracle fed those sequences alone: every packed field
  of every page bit for bit, and the decode output (fp32, before the final
  cast) within max|a-b| / max|b| <= 2e-3 per (batch, head) at the split count
  bench.py uses.
* C3 (batch 8, 16,384 tokens): the one-shot prefill append (8,128 key pages,
  selection and value rows in one launch), then 256 one-token appends; the
  pages sealed by those appends and the decode afterwards against the oracle
  for sequences 0 and 7.

Size-independent checks cover the sequences the oracle does not replay: the
page count and token coverage of every sequence's table, and finite outputs.
"""

from __future__ import annotations

import pytest
import torch

from tests.golden_util import bits_equal

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _seg_fields(seg):
    if isinstance(seg, torch.Tensor):
        return {"dense": seg}
    if hasattr(seg, "low_values"):
        return {"low": seg.low_values, "high": seg.high_values, "idx": seg.channel_indices,
                "scale": seg.scale, "zero": seg.zero_point}
    return {"values": seg.values, "scale": seg.scale, "zero": seg.zero_point}


def _compare_sequence(cache_pairs, oracle_pairs, b: int, first: int = 0) -> int:
    """Every field of cache segments [first:] for sequence b equals the single-sequence oracle's."""
    assert len(cache_pairs) == len(oracle_pairs)
    checked = 0
    for i in range(first, len(cache_pairs)):
        (ks, vs), (oks, ovs) = cache_pairs[i], oracle_pairs[i]
        for side, seg, oseg in (("key", ks, oks), ("value", vs, ovs)):
            fa, fb = _seg_fields(seg), _seg_fields(oseg)
            assert set(fa) == set(fb), (i, side)
            for name in fa:
                a = fa[name][b:b + 1].cpu()
                assert bits_equal(a, fb[name]), (b, i, side, name)
        checked += 1
    return checked


def _rel_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    a = actual.detach().float().cpu().flatten(1)
    e = expected.detach().float().cpu().flatten(1)
    return float(((a - e).abs().amax(-1) / e.abs().amax(-1).clamp_min(1e-30)).max())


def _config(bits_mode: str) -> dict:
    cfg = dict(page_size=128, key_group_size=128, value_group_size=64, sink_tokens=32, hold_partial_pages=True,
               metadata_dtype=torch.float16)
    cfg.update(dict(bits=2, promote_ratio=0.25) if bits_mode == "2b25" else dict(bits=4, promote_ratio=0.0))
    return cfg


@pytest.mark.parametrize("bits_mode", ["2b25", "4b"])
def test_c5_layer_pages_and_decode_vs_oracle(bits_mode):
    import dartkv_amd as dart
    from dartkv_amd import synthetic
    from dartkv_amd.attention import page_kernel_splits
    from oracle import dart_oracle as O
    B, H, Hq, T, D = 64, 8, 32, 32768, 128
    cfg = _config(bits_mode)
    print("case C5", bits_mode, (B, H, T, D), flush=True)
    keys, values, query = synthetic.outlier_kv(B, H, T, D, query_heads=Hq, dtype=torch.bfloat16, device=DEV)
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    cache.append(keys, values)
    plan = cache.decode_plan(torch.device(DEV))
    pages = (T - 32) // 128
    assert plan.fast_count == pages and plan.count == pages + 1
    units = pages if plan.fast_promoted else 2 * pages
    out32 = torch.empty(B, Hq, D, dtype=torch.float32, device=DEV)
    out = dart.decode_attention(query, cache, out_f32=out32, n_splits=page_kernel_splits(B, H, units))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out32).all()) and out.shape == (B, Hq, 1, D)
    table = cache.page_table().validate()
    assert table.page_count == pages + 2 and table.seen_tokens == T
    pairs = cache.iter_segments()
    for b in (0, B - 1):
        print("sequence", b, flush=True)
        oc = O.OracleCache(O.OracleConfig(**cfg))
        oc.append(keys[b:b + 1].cpu(), values[b:b + 1].cpu())
        assert _compare_sequence(pairs, oc.segments(), b) == pages + 2
        _, ref32 = O.streamed_attention(query[b:b + 1].cpu(), oc, return_fp32=True)
        err = _rel_err(out32[b:b + 1], ref32.reshape(1, Hq, D))
        print("decode rel err", b, err, flush=True)
        assert err <= 2e-3


def test_c3_prefill_then_one_token_appends_vs_oracle():
    import dartkv_amd as dart
    from dartkv_amd import synthetic
    from oracle import dart_oracle as O
    B, H, T, D, extra = 8, 8, 16384, 128, 256
    cfg = _config("2b25")
    print("case C3", (B, H, T, D), "+", extra, "one-token appends", flush=True)
    keys, values, query = synthetic.outlier_kv(B, H, T + extra, D, query_heads=32, dtype=torch.bfloat16, device=DEV)
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    cache.append(keys[:, :, :T].contiguous(), values[:, :, :T].contiguous())
    prefill_pairs = len(cache.iter_segments())
    assert prefill_pairs == 1 + (T - 32) // 128 + 1  # sink, 127 pages, 96-token tail
    for i in range(extra):
        cache.append(keys[:, :, T + i:T + i + 1], values[:, :, T + i:T + i + 1])
    out32 = torch.empty(B, 32, D, dtype=torch.float32, device=DEV)
    dart.decode_attention(query, cache, out_f32=out32)
    torch.cuda.synchronize()
    pairs = cache.iter_segments()
    assert len(pairs) == prefill_pairs + 2  # two pages sealed by the one-token appends
    for b in (0, B - 1):
        print("sequence", b, flush=True)
        oc = O.OracleCache(O.OracleConfig(**cfg))
        kb, vb = keys[b:b + 1].cpu(), values[b:b + 1].cpu()
        oc.append(kb[:, :, :T], vb[:, :, :T])
        for i in range(extra):
            oc.append(kb[:, :, T + i:T + i + 1], vb[:, :, T + i:T + i + 1])
        assert _compare_sequence(pairs, oc.segments(), b) == len(pairs)
        _, ref32 = O.streamed_attention(query[b:b + 1].cpu(), oc, return_fp32=True)
        err = _rel_err(out32[b:b + 1], ref32.reshape(1, 32, D))
        print("decode rel err", b, err, flush=True)
        assert err <= 2e-3

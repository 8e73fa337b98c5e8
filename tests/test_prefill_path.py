"""The first append of an empty cache (DartKVCache._prefill: one library call that quantizes the pages and
copies the dense sink and held tail, its outputs planned per configuration and input layout) against the
general append path on the same inputs: the same segments, byte for byte, the same held tail, pool
capacities and versions, and the same state after later appends (reference lifecycle: cache.py:168-190,
:403-542).

The host-side plan is checked on the CPU (token split, pool capacities, the cases it leaves to the
general path); the rest runs on the GPU.
"""

from __future__ import annotations

import pytest
import torch

from tests.golden_util import bits_equal

DEV = "cuda"

BASE = dict(bits=2, page_size=128, key_group_size=128, value_group_size=64, promote_ratio=0.25, sink_tokens=32,
            hold_partial_pages=True, metadata_dtype=torch.float16)

CASES = [
    ("dart_sink_held", dict(BASE), (2, 4, 700)),
    ("dart_variance", dict(BASE, channel_selection="variance"), (2, 4, 600)),
    ("dart_no_sink", dict(BASE, sink_tokens=0), (3, 2, 512)),
    ("dart_sink_exact_pages", dict(BASE, sink_tokens=32), (1, 4, 32 + 3 * 128)),
    ("uniform2", dict(BASE, promote_ratio=0.0), (2, 4, 700)),
    ("uniform4_g64", dict(BASE, promote_ratio=0.0, bits=4, key_group_size=64, value_group_size=32), (2, 3, 450)),
    ("uniform8", dict(BASE, promote_ratio=0.0, bits=8, sink_tokens=5), (2, 4, 333)),
    ("local_window", dict(BASE, local_tokens=16, sink_tokens=8), (2, 4, 600)),
    ("seal_all_exact", dict(BASE, hold_partial_pages=False, sink_tokens=0), (2, 4, 512)),
    ("page64", dict(BASE, page_size=64, key_group_size=32, value_group_size=32, sink_tokens=5), (3, 4, 300)),
    ("mixed_bits", dict(BASE, promote_ratio=0.0, key_bits=4, value_bits=2), (2, 4, 400)),
    ("f32_meta", dict(BASE, metadata_dtype=torch.float32), (2, 2, 400)),
    ("batch1_head1", dict(BASE), (1, 1, 400)),
]


def _fields(seg):
    if isinstance(seg, torch.Tensor):
        return [seg]
    if hasattr(seg, "low_values"):
        return [seg.low_values, seg.high_values, seg.channel_indices, seg.scale, seg.zero_point]
    return [seg.values, seg.scale, seg.zero_point]


def _state(cache):
    pools = [(p.capacity, p.used, p.shapes) for p in (cache._key_pool, cache._value_pool) if p is not None]
    pend = None if cache._pending_key is None else (cache._pending_key.clone(), cache._pending_value.clone(),
                                                      cache._tail_key.shape, cache._tail_key.stride())
    return dict(keys=[(type(s).__name__, [t.clone() for t in _fields(s)]) for s in cache._keys],
                values=[(type(s).__name__, [t.clone() for t in _fields(s)]) for s in cache._values],
                pools=pools, pending=pend, seen=cache._seen_tokens, layout=cache._layout_version,
                sealed=cache._sealed_version)


def _assert_same(a, b):
    for track in ("keys", "values"):
        assert len(a[track]) == len(b[track]), track
        for (na, fa), (nb, fb) in zip(a[track], b[track]):
            assert na == nb
            for x, y in zip(fa, fb):
                assert x.shape == y.shape and x.dtype == y.dtype
                assert bits_equal(x.cpu(), y.cpu())
    assert a["pools"] == b["pools"]
    assert (a["pending"] is None) == (b["pending"] is None)
    if a["pending"] is not None:
        assert bits_equal(a["pending"][0].cpu(), b["pending"][0].cpu())
        assert bits_equal(a["pending"][1].cpu(), b["pending"][1].cpu())
        assert a["pending"][2:] == b["pending"][2:]
    assert (a["seen"], a["layout"], a["sealed"]) == (b["seen"], b["layout"], b["sealed"])


def _pair(cfg, monkeypatch):
    """(prefill-path cache, general-path cache) factories and a counter of prefill-path appends."""
    import dartkv_amd as dart
    taken = []
    real = dart.DartKVCache._prefill

    def spy(self, k, v):
        done = real(self, k, v) if not getattr(self, "_force_general", False) else False
        if done:
            taken.append(1)
        return done

    monkeypatch.setattr(dart.DartKVCache, "_prefill", spy)
    fast = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    slow = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    slow._force_general = True
    return fast, slow, taken


@pytest.mark.gpu
@pytest.mark.parametrize("name,cfg,shape", CASES, ids=[c[0] for c in CASES])
def test_prefill_matches_general_path(name, cfg, shape, monkeypatch):
    """Prefill-path and general-path first appends leave the same state, and so do the same later
    appends (one-token appends across a page seal, then a chunk); decode reads them identically."""
    import dartkv_amd as dart
    from dartkv_amd import synthetic
    B, H, T = shape
    extra = 150
    k, v, q = synthetic.outlier_kv(B, H, T + extra, 128, query_heads=4 * H, dtype=torch.bfloat16, seed=T + B,
                                   device=DEV)
    fast, slow, taken = _pair(cfg, monkeypatch)
    fast.append(k[:, :, :T], v[:, :, :T])
    slow.append(k[:, :, :T], v[:, :, :T])
    torch.cuda.synchronize()
    assert taken == [1], "the first append should take the prefill path"
    _assert_same(_state(fast), _state(slow))
    for i in range(T, T + 130):
        fast.append(k[:, :, i:i + 1], v[:, :, i:i + 1])
        slow.append(k[:, :, i:i + 1], v[:, :, i:i + 1])
    fast.append(k[:, :, T + 130:], v[:, :, T + 130:])
    slow.append(k[:, :, T + 130:], v[:, :, T + 130:])
    torch.cuda.synchronize()
    _assert_same(_state(fast), _state(slow))
    a = dart.decode_attention(q, fast)
    b = dart.decode_attention(q, slow)
    torch.cuda.synchronize()
    assert bits_equal(a.cpu(), b.cpu())


@pytest.mark.gpu
def test_prefill_strided_inputs_and_fallbacks(monkeypatch):
    """Sliced (non-contiguous) inputs take the prefill path where the value rows can be read in place and
    the general path otherwise; both give the general path's state."""
    from dartkv_amd import synthetic
    k, v, _ = synthetic.outlier_kv(2, 4, 900, 128, query_heads=16, dtype=torch.bfloat16, seed=5, device=DEV)
    token_major_k = k.transpose(1, 2).contiguous().transpose(1, 2)
    token_major_v = v.transpose(1, 2).contiguous().transpose(1, 2)
    for ks, vs, expect_fast in ((k[:, :, 100:800], v[:, :, 100:800], True),
                                (token_major_k[:, :, 100:800], v[:, :, 100:800], True),
                                (k[:, :, 100:800], token_major_v[:, :, 100:800], False),
                                (k[:, 1:3, :700], v[:, 1:3, :700], False)):
        fast, slow, taken = _pair(dict(BASE), monkeypatch)
        fast.append(ks, vs)
        slow.append(ks, vs)
        torch.cuda.synchronize()
        assert taken == ([1] if expect_fast else [])
        _assert_same(_state(fast), _state(slow))


@pytest.mark.gpu
def test_prefill_nonfinite_input_leaves_cache_empty():
    """A NaN in a prefill raises the general path's ValueError; the cache stays empty and takes a later
    prefill as a fresh cache does."""
    import dartkv_amd as dart
    from dartkv_amd import synthetic
    k, v, q = synthetic.outlier_kv(2, 4, 600, 128, query_heads=16, dtype=torch.bfloat16, seed=9, device=DEV)
    for target, cfg, msg in ((k, dict(BASE), "key_states must contain finite values"),
                             (v, dict(BASE), "quantize expects all values to be finite"),
                             (k, dict(BASE, promote_ratio=0.0), "quantize expects all values to be finite")):
        cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
        bad = target.clone()
        bad[1, 2, 300, 7] = float("nan")
        with pytest.raises(ValueError, match=msg):
            if target is k:
                cache.append(bad, v)
            else:
                cache.append(k, bad)
        assert cache.seen_tokens == 0 and not cache._keys and not cache._values and cache._pending_key is None
        cache.append(k, v)
        ref = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
        ref.append(k, v)
        torch.cuda.synchronize()
        a, b = dart.decode_attention(q, cache), dart.decode_attention(q, ref)
        torch.cuda.synchronize()
        assert bits_equal(a.cpu(), b.cpu())


@pytest.mark.gpu
def test_prefill_under_inference_mode_then_outside():
    """Storage made by a prefill inside inference_mode stays writable by later appends outside it."""
    import dartkv_amd as dart
    from dartkv_amd import synthetic
    k, v, q = synthetic.outlier_kv(2, 4, 800, 128, query_heads=16, dtype=torch.bfloat16, seed=3, device=DEV)
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**BASE))
    ref = dart.DartKVCache(dart.DartKVCacheConfig(**BASE))
    with torch.inference_mode():
        cache.append(k[:, :, :600], v[:, :, :600])
    ref.append(k[:, :, :600], v[:, :, :600])
    for i in range(600, 800):
        cache.append(k[:, :, i:i + 1], v[:, :, i:i + 1])
        ref.append(k[:, :, i:i + 1], v[:, :, i:i + 1])
    torch.cuda.synchronize()
    _assert_same(_state(cache), _state(ref))


def _split(cfg, T):
    """The general path's token split of a first append: (sink, sealed, held)."""
    P, local = cfg.page_size, cfg.local_tokens
    sink = min(cfg.sink_tokens, T)
    rest = T - sink
    if cfg.hold_partial_pages or local:
        sealed = (max(0, rest - local) // P) * P
    else:
        sealed = rest
    return sink, sealed, rest - sealed


@pytest.mark.parametrize("T", [1, 31, 32, 33, 160, 161, 287, 288, 700])
@pytest.mark.parametrize("over", [{}, dict(sink_tokens=0), dict(local_tokens=16), dict(hold_partial_pages=False),
                                  dict(hold_partial_pages=False, sink_tokens=0), dict(value_local_tokens=4),
                                  dict(channel_selection="random"), dict(channel_selection="random",
                                                                         promote_ratio=0.0)])
def test_prefill_plan_split_and_capacities(T, over):
    """CPU: the plan's token split is the general path's; the pools' capacities are those its first reserve
    calls give; Kitty value windows, random channel choices, short last pages and appends that seal nothing
    are left to the general path."""
    from dartkv_amd.cache import DartKVCacheConfig, _PrefillPlan
    from dartkv_amd.pool import PagePool
    cfg = DartKVCacheConfig(**dict(BASE, **over))
    k = torch.zeros(2, 3, T, 128, dtype=torch.bfloat16)
    plan = _PrefillPlan.build(cfg, k, k)
    sink, sealed, held = _split(cfg, T)
    applies = not (cfg.value_local_tokens or sealed == 0 or sealed % cfg.page_size
                   or (cfg.channel_selection == "random" and cfg.promote_ratio > 0))
    assert (plan is not False) == applies
    if plan is False:
        return
    assert (plan.sink, plan.sealable, plan.pending, plan.n_pages) == (sink, sealed, held, sealed // cfg.page_size)
    kpool = PagePool(plan.key_fields, axis=0, batch_axis=1, device=k.device)
    kpool.reserve(plan.n_pages, headroom=max(2, plan.n_pages // 16))
    vpool = PagePool(plan.value_fields, axis=2, batch_axis=0, device=k.device, align=64)
    vpool.reserve(sealed, headroom=max(64, sealed // 16))
    assert (plan.key_capacity, plan.value_capacity) == (kpool.capacity, vpool.capacity)
    assert plan.key_layout == kpool._layout and plan.value_layout == vpool._layout
    assert plan.tail_capacity == (cfg.page_size + cfg.local_tokens if held else 0)

"""Seeded random cache configurations and append sequences: the HIP path against the oracle (GPU).

Each case draws a configuration (key and value bit widths, group sizes, page size, sink tokens,
held pages, Kitty key and value windows, promotion ratio and strategy, metadata dtype), a shape
(batch, KV heads, query heads per KV head, head_dim), a cache dtype (bf16, fp16, fp32, float64) and
a sequence of append lengths, then checks every packed segment bit for bit against the oracle and
the one- and two-token attention on the fp32 output within the parity bar: max|a-b| / max|b| per
(batch, head) of 2e-3 for 16-bit caches and 1e-5 for fp32 and float64 caches.  The "random"
channel strategy draws its channels on the device, so it is covered by its own given-channel test.
"""

from __future__ import annotations

import random

import pytest
import torch

from tests.golden_util import bits_equal

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _case(seed: int) -> dict:
    r = random.Random(seed)
    dtype = r.choice([torch.bfloat16, torch.float16, torch.float32, torch.float64])
    D = r.choice([16, 32, 64, 128])
    page = r.choice([4, 8, 16, 32, 128])
    cfg = dict(bits=r.choice([2, 4, 8]), key_bits=r.choice([None, 2, 4, 8]), value_bits=r.choice([None, 2, 4, 8]),
               group_size=r.choice([4, 8, 16, 32, 64]), key_group_size=r.choice([None, 3, 4, 8, page]),
               value_group_size=r.choice([None, 4, 6, 8, 16, D]), page_size=page,
               sink_tokens=r.choice([0, 1, 3, 32]), hold_partial_pages=r.random() < 0.5,
               promote_ratio=r.choice([0.0, 0.0, 0.25, 0.5]), channel_selection=r.choice(["magnitude", "variance"]),
               metadata_dtype=r.choice([torch.float16, torch.bfloat16, torch.float32, torch.float64]))
    if r.random() < 0.2:
        cfg["local_tokens"] = r.choice([1, 2, 4])
    if r.random() < 0.1:
        cfg["value_local_tokens"] = r.choice([1, 2])
    total = r.randint(page + 1, min(400, 6 * page + 40))
    updates, left = [], total
    while left:
        n = min(left, r.choice([1, 1, 2, 5, page, 3 * page + 1]))
        updates.append(n)
        left -= n
    return dict(B=r.choice([1, 2]), Hkv=r.choice([1, 2, 4]), G=r.choice([1, 2, 4, 8]), D=D, dtype=dtype, cfg=cfg,
                updates=updates)


def _fields(seg):
    if isinstance(seg, torch.Tensor):
        return [seg]
    if hasattr(seg, "low_values"):
        return [seg.low_values, seg.high_values, seg.channel_indices, seg.scale, seg.zero_point]
    return [seg.values, seg.scale, seg.zero_point]


def _rel_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    a = actual.detach().float().cpu().flatten(2)
    b = expected.detach().float().cpu().flatten(2)
    return float(((a - b).abs().amax(dim=-1) / b.abs().amax(dim=-1).clamp_min(1e-30)).max())


@pytest.mark.parametrize("seed", range(64))
def test_random_lifecycle_vs_oracle(seed):
    import dartkv_amd as dart
    from dartkv_amd import _lib, synthetic
    from dartkv_amd.attention import _multi_token_attention
    from oracle import dart_oracle as O
    _lib.load()
    c = _case(seed)
    B, Hkv, D, dtype, cfg = c["B"], c["Hkv"], c["D"], c["dtype"], c["cfg"]
    Hq = Hkv * c["G"]
    total = sum(c["updates"])
    print("case", seed, B, Hkv, Hq, D, dtype, cfg, c["updates"], flush=True)
    k, v, _ = synthetic.outlier_kv(B, Hkv, total, D, query_heads=Hq, dtype=torch.float32, seed=1000 + seed,
                                   outliers=min(8, D // 4))
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, 2, D, generator=g)
    if dtype == torch.float64:
        k, v, q = (t.double() * (1 + 1e-9 * torch.randn(t.shape, generator=g, dtype=torch.float64)) for t in (k, v, q))
    k, v, q = k.to(dtype), v.to(dtype), q.to(dtype)
    oc = O.OracleCache(O.OracleConfig(**cfg))
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    kd, vd = k.to(DEV), v.to(DEV)
    start = 0
    for n in c["updates"]:
        oc.append(k[..., start:start + n, :], v[..., start:start + n, :])
        cache.append(kd[..., start:start + n, :], vd[..., start:start + n, :])
        start += n
    torch.cuda.synchronize()
    segs, osegs = cache.iter_segments(), oc.segments()
    assert len(segs) == len(osegs)
    for i, ((ks, vs), (oks, ovs)) in enumerate(zip(segs, osegs)):
        for side, a, b in (("key", ks, oks), ("value", vs, ovs)):
            fa, fb = _fields(a), _fields(b)
            assert len(fa) == len(fb), (seed, i, side)
            for x, y in zip(fa, fb):
                assert bits_equal(x.cpu(), y), (seed, i, side)
    tol = 2e-3 if dtype in (torch.float16, torch.bfloat16) else 1e-5
    ref1 = O.streamed_attention(q[:, :, :1], oc, return_fp32=True)[1]
    out1 = torch.empty(B, Hq, D, dtype=torch.float32, device=DEV)
    dart.decode_attention(q[:, :, :1].contiguous().to(DEV), cache, out_f32=out1)
    ref2 = O.streamed_attention(q, oc, return_fp32=True)[1]
    out2 = torch.empty(B, Hq, 2, D, dtype=torch.float32, device=DEV)
    _multi_token_attention(q.to(DEV), cache, out_f32=out2)
    torch.cuda.synchronize()
    e1, e2 = _rel_err(out1.unsqueeze(2), ref1), _rel_err(out2, ref2)
    print("rel err one token", e1, "two tokens", e2, flush=True)
    assert e1 <= tol and e2 <= tol, (seed, e1, e2)


def _fast_case(seed: int) -> dict:
    r = random.Random(7000 + seed)
    uniform = r.random() < 0.4
    cfg = dict(page_size=128, key_group_size=128, value_group_size=r.choice([16, 32, 64, 128]),
               sink_tokens=r.choice([0, 32]), hold_partial_pages=r.random() < 0.7, metadata_dtype=torch.float16)
    if uniform:
        cfg.update(bits=r.choice([2, 4, 8]), key_bits=r.choice([2, 4, 8]), value_bits=r.choice([2, 4, 8]),
                   promote_ratio=0.0)
    else:
        cfg.update(bits=2, promote_ratio=r.choice([0.125, 0.25, 0.375, 0.5]),
                   channel_selection=r.choice(["magnitude", "variance"]))
    B, Hkv = r.choice([(1, 1), (1, 2), (1, 4), (2, 2), (2, 4), (1, 8)])
    total = r.randint(300, 1000)
    first = r.randint(1, total)
    updates = [first] + [1] * min(total - first, 3)
    updates += [total - sum(updates)] if total > sum(updates) else []
    return dict(B=B, Hkv=Hkv, G=r.choice([1, 2, 4, 8]), Q=r.choice([1, 1, 2, 3]),
                dtype=r.choice([torch.bfloat16, torch.float16]), cfg=cfg, updates=updates)


@pytest.mark.parametrize("seed", range(32))
def test_random_page_kernel_caches_vs_oracle(seed):
    """Caches in the page kernels' layout (head_dim 128, 128-token pages, one key group per page, fp16
    metadata, 16-bit K/V): random Dart promotion counts or uniform bit widths, value groups, GQA ratios,
    sinks, held pages, lengths and query token counts; the page kernels must take the page run."""
    import dartkv_amd as dart
    from dartkv_amd import _lib, synthetic
    from dartkv_amd.attention import _multi_token_attention
    from oracle import dart_oracle as O
    _lib.load()
    c = _fast_case(seed)
    B, Hkv, dtype, cfg, Q = c["B"], c["Hkv"], c["dtype"], c["cfg"], c["Q"]
    Hq, D = Hkv * c["G"], 128
    total = sum(c["updates"])
    print("case", seed, B, Hkv, Hq, Q, dtype, cfg, c["updates"], flush=True)
    k, v, _ = synthetic.outlier_kv(B, Hkv, total, D, query_heads=Hq, dtype=dtype, seed=2000 + seed)
    q = torch.randn(B, Hq, Q, D, generator=torch.Generator().manual_seed(seed)).to(dtype)
    oc = O.OracleCache(O.OracleConfig(**cfg))
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    kd, vd = k.to(DEV), v.to(DEV)
    start = 0
    for n in c["updates"]:
        oc.append(k[..., start:start + n, :], v[..., start:start + n, :])
        cache.append(kd[..., start:start + n, :], vd[..., start:start + n, :])
        start += n
    torch.cuda.synchronize()
    segs, osegs = cache.iter_segments(), oc.segments()
    assert len(segs) == len(osegs)
    for i, ((ks, vs), (oks, ovs)) in enumerate(zip(segs, osegs)):
        for side, a, b in (("key", ks, oks), ("value", vs, ovs)):
            for x, y in zip(_fields(a), _fields(b)):
                assert bits_equal(x.cpu(), y), (seed, i, side)
    plan = cache.decode_plan(torch.device(DEV))
    full_pages = sum(1 for s, _ in osegs if not isinstance(s, torch.Tensor) and O.seg_tokens(s) == 128)
    # the page kernels take the longest run of full pages (partial pages of unheld appends split runs)
    assert 0 < plan.fast_count <= full_pages if full_pages else plan.fast_count == 0, (plan.fast_count, full_pages)
    ref = O.streamed_attention(q, oc, return_fp32=True)[1]
    out = torch.empty(B, Hq, Q, D, dtype=torch.float32, device=DEV)
    if Q == 1:
        o1 = torch.empty(B, Hq, D, dtype=torch.float32, device=DEV)
        dart.decode_attention(q.to(DEV), cache, out_f32=o1)
        out = o1.unsqueeze(2)
    else:
        _multi_token_attention(q.to(DEV), cache, out_f32=out)
    torch.cuda.synchronize()
    err = _rel_err(out, ref)
    print("rel err", err, "fast pages", plan.fast_count, flush=True)
    assert err <= 2e-3, (seed, err)

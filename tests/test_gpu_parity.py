"""HIP kernels vs the reference's golden vectors and the CPU oracle (GPU).

Bar: packed codes, channel indices, scales and zero points bit-exact;
attention within max|a-b| / max|b| per (batch, head) of 2e-3 for bf16/fp16
caches and 1e-5 for fp32 and float64 caches, on the fp32 output before the
final cast.
"""

from __future__ import annotations

import pytest
import torch

from tests.golden_util import DTYPES, bits_equal

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _dkv():
    import dartkv_amd
    from dartkv_amd import _lib
    _lib.load()
    return dartkv_amd


def rel_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    """max over (batch, head) of max|a-b| / max|b| on [B, H, ..., D] tensors."""
    a = actual.detach().float().cpu().flatten(2)
    b = expected.detach().float().cpu().flatten(2)
    num = (a - b).abs().amax(dim=-1)
    den = b.abs().amax(dim=-1).clamp_min(1e-30)
    return float((num / den).max())


def tolerance(dtype: torch.dtype) -> float:
    """fp32 attention over 16-bit inputs: 2e-3; over fp32 and float64 caches (whose
    attention also computes in fp32): 1e-5."""
    return 2e-3 if dtype in (torch.float16, torch.bfloat16) else 1e-5


def test_uniform_quantize_bit_exact_vs_golden(golden):
    dart = _dkv()
    for e in golden.manifest["uniform"]:
        data = golden.get(e["input"]).to(DEV)
        print("case", e["tag"], tuple(data.shape), data.dtype, e["bits"], e["group"], e["axis"], flush=True)
        q = dart.quantize(data, bits=e["bits"], group_size=e["group"], metadata_dtype=DTYPES[e["meta"]], axis=e["axis"])
        torch.cuda.synchronize()
        assert golden.matches(e["values"], q.values.cpu()), e["tag"]
        assert golden.matches(e["scale"], q.scale.cpu()), e["tag"]
        assert golden.matches(e["zero"], q.zero_point.cpu()), e["tag"]
        assert golden.matches(e["deq"], q.dequantize().cpu().contiguous()), e["tag"]


@pytest.mark.parametrize("layout", ["token_slice", "batch1", "head1", "tokens_major", "one_token"])
def test_value_rows_read_in_place_equal_the_contiguous_copy(layout):
    """dkv_quantize_row_blocks on a strided token slice == dkv_quantize_rows on its copy, bit for bit."""
    dart = _dkv()
    from dartkv_amd.cache import _launch_value_rows
    g = torch.Generator().manual_seed(7)
    B, H, D = {"batch1": (1, 4), "head1": (3, 1)}.get(layout, (2, 3)) + (128,)
    if layout == "tokens_major":
        full = torch.randn(B, 200, H, D, generator=g).transpose(1, 2)  # [B, H, 200, D], not row blocks
    else:
        full = torch.randn(B, H, 200, D, generator=g)
    t0, T = (37, 1) if layout == "one_token" else (37, 130)
    for dtype in (torch.bfloat16, torch.float16, torch.float32):
        src = full.to(dtype).to(DEV)[:, :, t0:t0 + T]
        for bits, group, meta in ((2, 64, torch.float16), (4, 128, torch.bfloat16), (8, 32, torch.float32),
                                  (2, 48, torch.float16)):
            print("case", layout, dtype, bits, group, meta, flush=True)
            G = -(-D // group)
            values = torch.empty(B, H, T, -(-G * group // (8 // bits)), dtype=torch.uint8, device=DEV)
            scale = torch.empty(B, H, T, G, dtype=meta, device=DEV)
            zero = torch.empty_like(scale)
            _launch_value_rows(src, bits, group, meta, values, scale, zero)
            q = dart.quantize(src.contiguous(), bits=bits, group_size=group, metadata_dtype=meta, axis=-1)
            torch.cuda.synchronize()
            assert torch.equal(values, q.values.reshape(values.shape))
            assert bits_equal(scale.cpu(), q.scale.reshape(scale.shape).cpu())
            assert bits_equal(zero.cpu(), q.zero_point.reshape(zero.shape).cpu())


def test_mixed_key_bit_exact_vs_golden_including_tie_order(golden):
    dart = _dkv()
    from tests.test_oracle_golden import _input
    for e in golden.manifest["mixed"]:
        keys = _input(golden, e, DTYPES[e["dtype"]]).to(DEV)
        print("case", e["tag"], tuple(keys.shape), keys.dtype, e["group"], e["ratio"], e["strategy"], flush=True)
        mk = dart.quantize_key_mixed(keys, group_size=e["group"], promote_ratio=e["ratio"], strategy=e["strategy"],
                                     metadata_dtype=DTYPES[e["meta"]])
        torch.cuda.synchronize()
        for field, actual in (("low", mk.low_values), ("high", mk.high_values), ("idx", mk.channel_indices),
                              ("scale", mk.scale), ("zero", mk.zero_point), ("deq", mk.dequantize())):
            assert golden.matches(e[field], actual.cpu()), (e["tag"], field)


def _config(cfg: dict):
    import dartkv_amd
    kw = dict(cfg)
    if "metadata_dtype" in kw:
        kw["metadata_dtype"] = DTYPES[kw["metadata_dtype"]]
    return dartkv_amd.DartKVCacheConfig(**kw)


def _seg_fields(seg):
    if isinstance(seg, torch.Tensor):
        return {"dense": seg}
    if hasattr(seg, "low_values"):
        return {"low": seg.low_values, "high": seg.high_values, "idx": seg.channel_indices,
                "scale": seg.scale, "zero": seg.zero_point}
    return {"values": seg.values, "scale": seg.scale, "zero": seg.zero_point}


@pytest.mark.parametrize("Hkv,Hq,Q,dtype,uniform", [
    (8, 32, 3, torch.bfloat16, False),   # G 4: two tokens (8 rows), then one (4 rows)
    (8, 32, 4, torch.bfloat16, False),   # G 4: four tokens in one launch (16 rows)
    (8, 32, 8, torch.float16, False),    # G 4: two launches of four tokens
    (4, 16, 3, torch.bfloat16, True),    # G 4 on uniform 4-bit pages: two tokens, then one
    (4, 16, 4, torch.bfloat16, True),    # G 4 on uniform pages: two launches of two tokens
    (4, 16, 8, torch.float16, True),     # G 4 on uniform pages: four launches of two tokens
    (2, 4, 5, torch.float16, True),      # G 2 on uniform pages: four tokens, then one
])
def test_multi_token_attention_vs_oracle_by_page_kind(Hkv, Hq, Q, dtype, uniform):
    """As below, on Dart pages and on uniform pages (promote ratio 0, 4-bit keys and values)."""
    dart = _dkv()
    from dartkv_amd.attention import _multi_token_attention
    from oracle import dart_oracle as O
    from dartkv_amd import synthetic
    k, v, _ = synthetic.outlier_kv(2, Hkv, 700, 128, query_heads=Hq, dtype=dtype, seed=60 + Q)
    cfg = dict(bits=4 if uniform else 2, page_size=128, key_group_size=128, value_group_size=64,
               promote_ratio=0.0 if uniform else 0.25, sink_tokens=32, hold_partial_pages=True,
               metadata_dtype=torch.float16)
    oc = O.OracleCache(O.OracleConfig(**cfg))
    oc.append(k, v)
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    cache.append(k.to(DEV), v.to(DEV))
    assert cache.decode_plan(torch.device(DEV)).fast_count == (700 - 32) // 128
    q = torch.randn(2, Hq, Q, 128, generator=torch.Generator().manual_seed(Q + 20)).to(dtype)
    _, ref32 = O.streamed_attention(q, oc, return_fp32=True)
    print("case", Hkv, Hq, Q, dtype, uniform, flush=True)
    out32 = torch.empty(2, Hq, Q, 128, dtype=torch.float32, device=DEV)
    _multi_token_attention(q.to(DEV), cache, out_f32=out32)
    torch.cuda.synchronize()
    err = rel_err(out32, ref32)
    print("rel err", err, flush=True)
    assert err <= tolerance(dtype)


@pytest.mark.parametrize("Hkv,Hq,Q,dtype", [
    (8, 32, 3, torch.bfloat16),   # G 4: two tokens (8 rows), then one (4 rows)
    (8, 32, 4, torch.float16),    # G 4: four tokens in one launch (16 rows)
    (8, 32, 5, torch.bfloat16),   # G 4: four tokens, then one (16 and 4 rows)
    (4, 8, 5, torch.bfloat16),    # G 2: four tokens (8 rows), then one
    (4, 4, 4, torch.float16),     # G 1: four tokens in one launch
    (2, 16, 3, torch.bfloat16),   # G 8: two tokens per launch (16 rows), then one (8 rows)
    (2, 32, 1, torch.bfloat16),   # G 16: one token, the 16-row page kernel
    (2, 6, 2, torch.bfloat16),    # G 3: general kernel
])
def test_multi_token_attention_vs_oracle(Hkv, Hq, Q, dtype):
    """Several query tokens attend to every cached token (reference attention.py:67-87, no mask)."""
    dart = _dkv()
    from dartkv_amd.attention import _multi_token_attention
    from oracle import dart_oracle as O
    from dartkv_amd import synthetic
    k, v, _ = synthetic.outlier_kv(2, Hkv, 900, 128, query_heads=Hq, dtype=dtype, seed=40 + Q)
    cfg = dict(bits=2, page_size=128, key_group_size=128, value_group_size=64, promote_ratio=0.25, sink_tokens=32,
               hold_partial_pages=True, metadata_dtype=torch.float16)
    oc = O.OracleCache(O.OracleConfig(**cfg))
    oc.append(k, v)
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    cache.append(k.to(DEV), v.to(DEV))
    q = torch.randn(2, Hq, Q, 128, generator=torch.Generator().manual_seed(Q)).to(dtype)
    _, ref32 = O.streamed_attention(q, oc, return_fp32=True)
    print("case", Hkv, Hq, Q, dtype, flush=True)
    qd = q.to(DEV)
    out32 = torch.empty(2, Hq, Q, 128, dtype=torch.float32, device=DEV)
    out = _multi_token_attention(qd, cache, out_f32=out32)
    fused = dart.fused_dart_attention(qd, cache)
    torch.cuda.synchronize()
    err = rel_err(out32, ref32)
    print("rel err", err, flush=True)
    assert err <= tolerance(dtype)
    assert out.shape == (2, Hq, Q, 128) and bits_equal(fused.cpu(), out.cpu())


@pytest.mark.parametrize("selection", ["magnitude", "variance"])
def test_large_append_pages_bit_exact_vs_oracle(selection):
    """An append of more than 256 key pages takes the separate selection pass
    (scores, one wave per page, codes) with the value rows in the selection's
    launch; every packed field, channel order included, equals the oracle's."""
    dart = _dkv()
    from dartkv_amd import synthetic
    from oracle import dart_oracle as O
    k, v, _ = synthetic.outlier_kv(2, 8, 3000, 128, query_heads=32, dtype=torch.bfloat16, seed=11)
    cfg = dict(bits=2, page_size=128, key_group_size=128, value_group_size=64, promote_ratio=0.25, sink_tokens=32,
               hold_partial_pages=True, metadata_dtype=torch.float16, channel_selection=selection)
    print("case", selection, "pages", 2 * 8 * ((3000 - 32) // 128), flush=True)
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    cache.append(k.to(DEV), v.to(DEV))
    oc = O.OracleCache(O.OracleConfig(**cfg))
    oc.append(k, v)
    torch.cuda.synchronize()
    assert len(cache.iter_segments()) == len(oc.segments())
    pairs = list(zip(cache.iter_segments(), oc.segments()))
    for (ks, vs), (oks, ovs) in pairs:
        for a, b in zip(_seg_fields(ks).values(), _seg_fields(oks).values()):
            assert bits_equal(a.cpu(), b)
        for a, b in zip(_seg_fields(vs).values(), _seg_fields(ovs).values()):
            assert bits_equal(a.cpu(), b)


@pytest.mark.parametrize("bits,dtype", [(2, torch.bfloat16), (4, torch.float16), (8, torch.bfloat16),
                                        (8, torch.float16)])
def test_uniform_append_pages_bit_exact_vs_oracle(bits, dtype):
    """Uniform 2/4/8-bit pages of head_dim 128 (the single-pass key page kernel, packed rows staged in LDS),
    with a partial held page and the value rows: every packed field equals the oracle's."""
    dart = _dkv()
    from dartkv_amd import synthetic
    from oracle import dart_oracle as O
    k, v, _ = synthetic.outlier_kv(2, 4, 1100, 128, query_heads=8, dtype=dtype, seed=5 + bits)
    cfg = dict(bits=bits, page_size=128, key_group_size=128, value_group_size=64, promote_ratio=0.0, sink_tokens=32,
               hold_partial_pages=False, metadata_dtype=torch.float16)
    print("case uniform", bits, dtype, flush=True)
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    cache.append(k.to(DEV), v.to(DEV))
    oc = O.OracleCache(O.OracleConfig(**cfg))
    oc.append(k, v)
    torch.cuda.synchronize()
    assert len(cache.iter_segments()) == len(oc.segments()) == 1 + -(-(1100 - 32) // 128)
    pairs = list(zip(cache.iter_segments(), oc.segments()))
    for (ks, vs), (oks, ovs) in pairs:
        for a, b in zip(_seg_fields(ks).values(), _seg_fields(oks).values()):
            assert bits_equal(a.cpu(), b)
        for a, b in zip(_seg_fields(vs).values(), _seg_fields(ovs).values()):
            assert bits_equal(a.cpu(), b)


@pytest.mark.parametrize("name", ["c2", "c1", "nonheld", "held_mixed", "kitty_local", "kitty_value_local",
                                  "uniform_mix_bits", "f64_mixed", "f64_uniform", "f64_meta16"])
def test_cache_pages_and_decode_vs_golden(golden, name):
    dart = _dkv()
    from tests.test_oracle_golden import _lifecycle_inputs
    e = next(x for x in golden.manifest["cache"] if x["name"] == name)
    keys, values, query = _lifecycle_inputs(golden, e)
    print("lifecycle", name, tuple(keys.shape), keys.dtype, e["updates"], flush=True)
    cache = dart.DartKVCache(_config(e["config"]))
    start = 0
    kd, vd = keys.to(DEV), values.to(DEV)
    for n in e["updates"]:
        cache.update(kd[..., start:start + n, :], vd[..., start:start + n, :])
        start += n
    table = cache.page_table().validate()
    assert table.sequence_ranges().tolist() == e["ranges"]
    assert table.key_modes.tolist() == e["key_modes"]
    assert table.value_modes.tolist() == e["value_modes"]
    assert cache.storage_bytes == e["storage_bytes"]
    segs = cache.iter_segments()
    assert len(segs) == len(e["segments"])
    for i, ((kseg, vseg), rec) in enumerate(zip(segs, e["segments"])):
        for side, seg in (("key", kseg), ("value", vseg)):
            fields = _seg_fields(seg)
            assert set(fields) == set(rec[side]), (name, i, side)
            for field, ref in rec[side].items():
                assert golden.matches(ref, fields[field].cpu().contiguous()), (name, i, side, field)
    ref32 = golden.get(e["attn_out_f32"])
    qd = query.to(DEV)
    if qd.shape[-2] == 1:
        out32 = torch.empty(qd.shape[0], qd.shape[1], qd.shape[-1], dtype=torch.float32, device=DEV)
        out = dart.decode_attention(qd, cache, out_f32=out32)
        torch.cuda.synchronize()
        err = rel_err(out32.unsqueeze(2), ref32)
        print("decode rel err", name, err, flush=True)
        assert err <= tolerance(keys.dtype), (name, err)
        fused = dart.fused_dart_attention(qd, cache, fallback=False)
        assert bits_equal(fused.cpu(), out.cpu())


@pytest.mark.parametrize("meta,ratio,strategy", [
    (torch.float16, 0.25, "magnitude"),
    (torch.float64, 0.25, "variance"),
    (torch.float32, 0.0, "magnitude"),
])
def test_float64_cache_vs_oracle(meta, ratio, strategy):
    """A float64 cache (the reference caches float64 tensors: quantized in float64, attention in fp32,
    output cast back): five 128-token pages per (batch, head) in one append, then one-token appends;
    pages and materialized K/V bit-exact, one- and three-token attention within 1e-5."""
    dart = _dkv()
    from oracle import dart_oracle as O
    from dartkv_amd import synthetic
    g = torch.Generator().manual_seed(64)
    k, v, q = synthetic.outlier_kv(2, 2, 703, 128, query_heads=8, dtype=torch.float64, seed=91)
    k, v = (t * (1 + 1e-9 * torch.randn(t.shape, generator=g, dtype=torch.float64)) for t in (k, v))
    q3 = torch.randn(2, 8, 3, 128, generator=g, dtype=torch.float64)
    cfg = dict(bits=4 if ratio == 0.0 else 2, page_size=128, key_group_size=128, value_group_size=64,
               promote_ratio=ratio, channel_selection=strategy, sink_tokens=32, hold_partial_pages=True,
               metadata_dtype=meta)
    oc = O.OracleCache(O.OracleConfig(**cfg))
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    kd, vd = k.to(DEV), v.to(DEV)
    print("float64 cache", meta, ratio, strategy, flush=True)
    for a, b in ((0, 700), (700, 701), (701, 702), (702, 703)):
        oc.append(k[..., a:b, :], v[..., a:b, :])
        cache.append(kd[..., a:b, :], vd[..., a:b, :])
    torch.cuda.synchronize()
    assert len(cache.iter_segments()) == len(oc.segments())
    for (ks, vs), (oks, ovs) in zip(cache.iter_segments(), oc.segments()):
        for x, y in zip(_seg_fields(ks).values(), _seg_fields(oks).values()):
            assert bits_equal(x.cpu(), y)
        for x, y in zip(_seg_fields(vs).values(), _seg_fields(ovs).values()):
            assert bits_equal(x.cpu(), y)
    mk, mv = cache.get()
    omk, omv = oc.get()
    assert bits_equal(mk.cpu(), omk) and bits_equal(mv.cpu(), omv)
    ref32 = O.streamed_attention(q, oc, return_fp32=True)[1]
    out32 = torch.empty(2, 8, 128, dtype=torch.float32, device=DEV)
    out = dart.decode_attention(q.to(DEV), cache, out_f32=out32)
    torch.cuda.synchronize()
    assert out.dtype == torch.float64
    err = rel_err(out32.unsqueeze(2), ref32)
    print("float64 decode rel err", err, flush=True)
    assert err <= 1e-5
    assert bits_equal(out.cpu(), out32.unsqueeze(2).cpu().double())
    ref3 = O.streamed_attention(q3, oc, return_fp32=True)[1]
    out3 = dart.streamed_dart_attention(q3.to(DEV), cache)
    torch.cuda.synchronize()
    assert out3.dtype == torch.float64
    err3 = rel_err(out3.float(), ref3)
    print("float64 three-token rel err", err3, flush=True)
    assert err3 <= 1e-5


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_config2_decode_vs_oracle(seed, dtype):
    """Config 2 (B1, T1024, Hkv 8, Hq 32, D 128, page 128, kg 128, vg 64, 2-bit + 25 %, sink 32, held tail)."""
    dart = _dkv()
    from oracle import dart_oracle as O
    from dartkv_amd import synthetic
    k, v, q = synthetic.outlier_kv(1, 8, 1024, 128, query_heads=32, dtype=dtype, seed=100 + seed)
    cfg = dict(bits=2, page_size=128, key_group_size=128, value_group_size=64, promote_ratio=0.25, sink_tokens=32,
               hold_partial_pages=True, metadata_dtype=torch.float16)
    oc = O.OracleCache(O.OracleConfig(**cfg))
    oc.append(k, v)
    _, ref32 = O.streamed_attention(q, oc, return_fp32=True)
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    cache.append(k.to(DEV), v.to(DEV))
    out32 = torch.empty(1, 32, 128, dtype=torch.float32, device=DEV)
    dart.decode_attention(q.to(DEV), cache, out_f32=out32)
    torch.cuda.synchronize()
    err = rel_err(out32.unsqueeze(2), ref32)
    print("config2", seed, dtype, "rel err", err, flush=True)
    assert err <= 2e-3
    # every packed page matches the oracle bit for bit
    assert len(cache.iter_segments()) == len(oc.segments())
    for (ks, vs), (oks, ovs) in zip(cache.iter_segments(), oc.segments()):
        for a, b in zip(_seg_fields(ks).values(), _seg_fields(oks).values()):
            assert bits_equal(a.cpu(), b)
        for a, b in zip(_seg_fields(vs).values(), _seg_fields(ovs).values()):
            assert bits_equal(a.cpu(), b)


@pytest.mark.parametrize("kb,vb,vg,dtype", [
    (2, 2, 64, torch.bfloat16),   # 16 value codes per lane
    (4, 4, 32, torch.bfloat16),
    (8, 8, 16, torch.float16),
    (2, 8, 8, torch.bfloat16),    # value group 8: 8 value codes per lane
    (4, 2, 8, torch.float16),
    (8, 4, 8, torch.bfloat16),
])
def test_uniform_pages_bit_exact_vs_oracle(kb, vb, vg, dtype):
    """Uniform key pages (one token group per 128-token page, the single-pass key kernel) and value rows
    of every width, bit for bit against the oracle, for value groups that give 16 and 8 codes per lane."""
    _dkv()
    from dartkv_amd import synthetic
    from oracle import dart_oracle as O
    import dartkv_amd as dart
    cfg = dict(bits=kb, key_bits=kb, value_bits=vb, page_size=128, key_group_size=128, value_group_size=vg,
               promote_ratio=0.0, sink_tokens=32, hold_partial_pages=True, metadata_dtype=torch.float16)
    k, v, _ = synthetic.outlier_kv(2, 4, 700, 128, dtype=dtype, seed=70 + kb + vb)
    print("uniform pages", kb, vb, vg, dtype, flush=True)
    oc = O.OracleCache(O.OracleConfig(**cfg))
    oc.append(k, v)
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    cache.append(k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    assert len(cache.iter_segments()) == len(oc.segments()) == 7
    for (ks, vs), (oks, ovs) in zip(cache.iter_segments(), oc.segments()):
        for x, y in zip(_seg_fields(ks).values(), _seg_fields(oks).values()):
            assert bits_equal(x.cpu(), y)
        for x, y in zip(_seg_fields(vs).values(), _seg_fields(ovs).values()):
            assert bits_equal(x.cpu(), y)


def _oracle_and_cache(B, Hkv, Hq, T, dtype, seed, **over):
    import dartkv_amd as dart
    from dartkv_amd import synthetic
    from oracle import dart_oracle as O
    cfg = dict(bits=2, page_size=128, key_group_size=128, value_group_size=64, promote_ratio=0.25, sink_tokens=32,
               hold_partial_pages=True, metadata_dtype=torch.float16)
    cfg.update(over)
    k, v, q = synthetic.outlier_kv(B, Hkv, T, 128, query_heads=Hq, dtype=dtype, seed=seed)
    oc = O.OracleCache(O.OracleConfig(**cfg))
    oc.append(k, v)
    _, ref32 = O.streamed_attention(q, oc, return_fp32=True)
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    cache.append(k.to(DEV), v.to(DEV))
    return cache, q.to(DEV), ref32


@pytest.mark.parametrize("B,Hkv,Hq,T,dtype,vg,ratio", [
    (1, 8, 32, 1024, torch.bfloat16, 64, 0.25),    # config 2
    (3, 4, 16, 2000, torch.bfloat16, 64, 0.25),
    (2, 2, 4, 1500, torch.float16, 32, 0.25),      # GQA 2, fp16 cache, value group 32
    (2, 4, 4, 700, torch.bfloat16, 128, 0.25),     # GQA 1, value group 128
    (2, 4, 32, 1300, torch.bfloat16, 64, 0.25),    # GQA 8: two row groups
    (1, 2, 16, 900, torch.float16, 32, 0.25),      # GQA 8, fp16 cache, value group 32
    (1, 2, 16, 800, torch.bfloat16, 64, 0.5),      # GQA 8, 64 promoted channels
    (2, 2, 16, 600, torch.bfloat16, 16, 0.125),    # GQA 8, 16 promoted channels, value group 16
])
def test_fast_page_kernel_vs_oracle_and_general(B, Hkv, Hq, T, dtype, vg, ratio):
    dart = _dkv()
    cache, q, ref32 = _oracle_and_cache(B, Hkv, Hq, T, dtype, seed=7 + T, value_group_size=vg, promote_ratio=ratio)
    plan = cache.decode_plan(q.device)
    print("case", B, Hkv, Hq, T, dtype, vg, ratio, "fast pages", plan.fast_count, "of", plan.count, flush=True)
    assert plan.fast_count == (T - 32) // 128
    out_fast = torch.empty(B, Hq, 128, dtype=torch.float32, device=DEV)
    out_gen = torch.empty_like(out_fast)
    dart.decode_attention(q, cache, out_f32=out_fast, fast=True)
    dart.decode_attention(q, cache, out_f32=out_gen, fast=False)
    torch.cuda.synchronize()
    e_fast = rel_err(out_fast.unsqueeze(2), ref32)
    e_gen = rel_err(out_gen.unsqueeze(2), ref32)
    print("rel err fast", e_fast, "general", e_gen, flush=True)
    assert e_gen <= 2e-3
    assert e_fast <= 2e-3


@pytest.mark.parametrize("B,Hkv,Hq,T,dtype,vg,ratio", [
    (1, 8, 32, 1024, torch.bfloat16, 64, 0.25),    # config 2
    (2, 2, 4, 1500, torch.float16, 32, 0.25),      # GQA 2, fp16 cache, value group 32
    (2, 4, 4, 700, torch.bfloat16, 128, 0.25),     # GQA 1, value group 128
    (2, 4, 32, 1300, torch.bfloat16, 64, 0.25),    # GQA 8: two row groups
    (1, 2, 16, 800, torch.bfloat16, 64, 0.5),      # GQA 8, 64 promoted channels
    (2, 2, 16, 600, torch.bfloat16, 16, 0.125),    # GQA 8, 16 promoted channels, value group 16
    (1, 2, 8, 900, torch.float16, 64, 0.375),      # 48 promoted channels
])
def test_channel_split_pages_agree_with_whole_pages(monkeypatch, B, Hkv, Hq, T, dtype, vg, ratio):
    """Pages shared by four waves (each a quarter of the channels, partial logits summed in LDS) give the
    oracle's answer, and the whole-page kernel's up to the fp16 rounding of the softmax weights."""
    dart = _dkv()
    cache, q, ref32 = _oracle_and_cache(B, Hkv, Hq, T, dtype, seed=11 + T, value_group_size=vg, promote_ratio=ratio)
    outs = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("DKV_SPLIT_PAGES", mode)
        for splits in (None, 1, 3):
            o = torch.empty(B, Hq, 128, dtype=torch.float32, device=DEV)
            dart.decode_attention(q, cache, out_f32=o, n_splits=splits, fast=True)
            torch.cuda.synchronize()
            outs[mode, splits] = o.cpu()
    for key, o in outs.items():
        e = rel_err(o.unsqueeze(2), ref32)
        d = rel_err(o.unsqueeze(2), outs["0", key[1]].unsqueeze(2))
        print("case", B, Hkv, Hq, T, dtype, vg, ratio, "split pages", key, "rel err", e, "vs whole pages", d,
              flush=True)
        assert e <= 2e-3
        assert d <= 1e-3


def test_fast_page_kernel_split_counts_agree():
    """Every split count gives the same answer.

    Splits normalise their softmax weights by their own running max before the
    weights are rounded to fp16 for the PV product, so results differ by that
    rounding (~1e-4), not by more.
    """
    dart = _dkv()
    cache, q, ref32 = _oracle_and_cache(2, 8, 32, 3000, torch.bfloat16, seed=3)
    outs = []
    for splits in (1, 2, 5, 22):
        o = torch.empty(2, 32, 128, dtype=torch.float32, device=DEV)
        dart.decode_attention(q, cache, out_f32=o, n_splits=splits, fast=True)
        outs.append(o.cpu())
    for o in outs:
        assert rel_err(o.unsqueeze(2), ref32) <= 2e-3
        assert rel_err(o.unsqueeze(2), outs[0].unsqueeze(2)) <= 1e-3


@pytest.mark.parametrize("kb,vb,B,Hkv,Hq,T,dtype,vg", [
    (4, 4, 1, 8, 32, 1024, torch.bfloat16, 64),   # config 5's 4-bit variant shape
    (2, 2, 3, 4, 16, 2000, torch.bfloat16, 64),
    (8, 8, 2, 2, 4, 1500, torch.float16, 32),     # GQA 2, fp16 cache
    (4, 2, 2, 4, 4, 700, torch.bfloat16, 128),    # GQA 1, mixed widths
    (2, 8, 1, 2, 8, 900, torch.float16, 16),
    (8, 4, 2, 3, 12, 1100, torch.bfloat16, 64),
    (4, 4, 2, 2, 16, 800, torch.bfloat16, 64),    # GQA 8: two row groups
    (8, 8, 1, 4, 32, 700, torch.float16, 32),     # GQA 8, 8-bit, fp16 cache
    (2, 2, 1, 2, 16, 900, torch.bfloat16, 16),    # GQA 8, 2-bit, value group 16
])
def test_uniform_page_kernel_vs_oracle_and_general(kb, vb, B, Hkv, Hq, T, dtype, vg):
    """Uniform pages (no promoted channels): the arithmetic page kernel against the oracle and the general
    kernel, with a sink and a held tail around the page run."""
    dart = _dkv()
    cache, q, ref32 = _oracle_and_cache(B, Hkv, Hq, T, dtype, seed=11 + T + kb, value_group_size=vg,
                                        promote_ratio=0.0, key_bits=kb, value_bits=vb)
    plan = cache.decode_plan(q.device)
    print("case", kb, vb, B, Hkv, Hq, T, dtype, vg, "fast pages", plan.fast_count, "of", plan.count, flush=True)
    assert plan.fast_count == (T - 32) // 128
    assert (plan.fast_promoted, plan.fast_key_bits, plan.fast_value_bits) == (0, kb, vb)
    out_fast = torch.empty(B, Hq, 128, dtype=torch.float32, device=DEV)
    out_gen = torch.empty_like(out_fast)
    dart.decode_attention(q, cache, out_f32=out_fast, fast=True)
    dart.decode_attention(q, cache, out_f32=out_gen, fast=False)
    torch.cuda.synchronize()
    e_fast = rel_err(out_fast.unsqueeze(2), ref32)
    e_gen = rel_err(out_gen.unsqueeze(2), ref32)
    print("rel err fast", e_fast, "general", e_gen, flush=True)
    assert e_gen <= 2e-3
    assert e_fast <= 2e-3


def test_uniform_page_kernel_split_counts_agree():
    """Splits over half pages: odd counts start and end mid-page; all agree within the fp16 rounding of
    the softmax weights."""
    dart = _dkv()
    cache, q, ref32 = _oracle_and_cache(2, 8, 32, 3000, torch.bfloat16, seed=5, promote_ratio=0.0, bits=4)
    pages = cache.decode_plan(q.device).fast_count
    outs = []
    for splits in (1, 3, 7, 2 * pages):
        o = torch.empty(2, 32, 128, dtype=torch.float32, device=DEV)
        dart.decode_attention(q, cache, out_f32=o, n_splits=splits, fast=True)
        outs.append(o.cpu())
    for o in outs:
        assert rel_err(o.unsqueeze(2), ref32) <= 2e-3
        assert rel_err(o.unsqueeze(2), outs[0].unsqueeze(2)) <= 1e-3


@pytest.mark.parametrize("kind", ["dart", "uniform"])
@pytest.mark.parametrize("factor", [3.0e4, 1.0e-6])
def test_page_kernels_take_queries_outside_fp16_range(kind, factor):
    """The page kernels round the query to fp16; each split first scales its query heads by a power of
    two (largest |q| into [2^14, 2^15)) and takes the inverse power into the logit scale.  A bf16 query
    with elements far above fp16's largest value (65504), or far below its normal range, then matches
    the oracle like any other; before, the first overflowed to inf (NaN output)."""
    from dartkv_amd import synthetic
    from oracle import dart_oracle as O
    dart = _dkv()
    cfg = dict(bits=2, page_size=128, key_group_size=128, value_group_size=64, promote_ratio=0.25, sink_tokens=32,
               hold_partial_pages=True, metadata_dtype=torch.float16)
    if kind == "uniform":
        cfg.update(promote_ratio=0.0, key_bits=4, value_bits=4)
    k, v, q = synthetic.outlier_kv(2, 2, 900, 128, query_heads=8, dtype=torch.bfloat16, seed=21)
    q = (q.float() * factor).to(torch.bfloat16)
    if factor > 1:
        assert float(q.float().abs().max()) > 65504.0
    oc = O.OracleCache(O.OracleConfig(**cfg))
    oc.append(k, v)
    _, ref32 = O.streamed_attention(q, oc, return_fp32=True)
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    cache.append(k.to(DEV), v.to(DEV))
    q = q.to(DEV)
    plan = cache.decode_plan(q.device)
    assert plan.fast_count == (900 - 32) // 128
    out = torch.empty(2, 8, 128, dtype=torch.float32, device=DEV)
    dart.decode_attention(q, cache, out_f32=out, fast=True)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    err = rel_err(out.unsqueeze(2), ref32)
    print("case", kind, factor, "rel err", err, flush=True)
    assert err <= 2e-3


def test_decode_checks_the_page_and_dense_contracts_against_the_host_descriptors():
    """dkv_decode_attention checks what it is told about the descriptor table against the host copy the
    caller passes (segments_host): a fast page range that starts on the dense sink, or a dense rest that
    holds a packed page, is an error naming the entry, not NaN or a fault."""
    dart = _dkv()
    cache, q, ref32 = _oracle_and_cache(1, 2, 8, 700, torch.bfloat16, seed=5)
    plan = cache.decode_plan(q.device)
    assert plan.fast_first == 1 and plan.fast_count == (700 - 32) // 128 and plan.rest_dense >= 0
    first, count = plan.fast_first, plan.fast_count
    try:  # (the plan keeps call layouts derived from these fields: they are dropped after each change)
        plan.fast_first = 0  # entry 0 is the dense sink
        plan.call_layouts.clear()
        with pytest.raises(ValueError, match="descriptor 0 is not a page the fast page kernel reads"):
            dart.decode_attention(q, cache, fast=True)
        plan.fast_first, plan.fast_count = first, count - 1  # the last page falls to the dense kernel
        plan.call_layouts.clear()
        with pytest.raises(ValueError, match=f"descriptor {first + count - 1} is not a dense segment"):
            dart.decode_attention(q, cache, fast=True)
    finally:
        plan.fast_first, plan.fast_count = first, count
        plan.call_layouts.clear()
    out = torch.empty(1, 8, 128, dtype=torch.float32, device=DEV)
    dart.decode_attention(q, cache, out_f32=out, fast=True)
    torch.cuda.synchronize()
    assert rel_err(out.unsqueeze(2), ref32) <= 2e-3


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_codes_round_half_to_even_on_exact_half_quotients(bits, dtype):
    """Groups whose scale is exactly 1 (min 0, max qmax) and whose elements are half-integers: every
    quotient is an exact tie, so the codes pin the kernels' rounding (half to even, then the clamp to
    [0, qmax]) against the oracle, for value rows, uniform key pages and Dart key pages."""
    from oracle import dart_oracle as O
    dart = _dkv()
    qmax = (1 << bits) - 1
    halves = torch.arange(0, qmax, dtype=torch.float32) + 0.5
    groups = 2 * -(-qmax // 62)
    body = halves.repeat(-(-groups * 62 // qmax))[: groups * 62].reshape(groups, 62)
    ends = torch.tensor([0.0, float(qmax)]).expand(groups, 2)
    x = torch.cat([ends, body], 1).to(dtype)  # each group of 64: min 0, max qmax (scale exactly 1), then ties
    q = dart.quantize(x.to(DEV), bits=bits, group_size=64, metadata_dtype=torch.float32)
    ref = O.quantize(x, bits=bits, group_size=64, metadata_dtype=torch.float32)
    torch.cuda.synchronize()
    assert bits_equal(q.values.cpu(), ref.values) and bits_equal(q.scale.cpu(), ref.scale)
    # keys along the tokens: a [1, 1, 128, 128] page whose channels each run through the same values
    keys = torch.cat([x[0], x[-1]])[:128].reshape(128, 1).expand(128, 128).contiguous().reshape(1, 1, 128, 128)
    kq = dart.quantize(keys.to(DEV), bits=bits, group_size=128, metadata_dtype=torch.float32, axis=2)
    kref = O.quantize(keys, bits=bits, group_size=128, metadata_dtype=torch.float32, axis=2)
    torch.cuda.synchronize()
    assert bits_equal(kq.values.cpu(), kref.values)
    if bits == 2:
        mk = dart.quantize_key_mixed(keys.to(DEV), group_size=128, promote_ratio=0.25)
        mref = O.quantize_key_mixed(keys, group_size=128, promote_ratio=0.25)
        torch.cuda.synchronize()
        assert bits_equal(mk.low_values.cpu(), mref.low_values) and bits_equal(mk.high_values.cpu(), mref.high_values)

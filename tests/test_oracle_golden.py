"""Pin the CPU oracle to the reference's golden vectors (CPU only)."""

from __future__ import annotations

import pytest
import torch

from dartkv_amd import synthetic
from oracle import dart_oracle as O
from tests.golden_util import DTYPES, bits_equal


def _input(golden, entry, dtype):
    t = golden.get(entry["input"])
    if t is not None:
        return t
    B, H, T, D = entry["shape"]
    keys, _, _ = synthetic.outlier_kv(B, H, T, D, dtype=torch.float32, seed=entry["seed"], outliers=entry["outliers"])
    keys = keys.to(dtype)
    assert golden.matches(entry["input"], keys), "synthetic input drifted from the golden digest"
    return keys


def test_uniform_quantize_matches_reference(golden):
    entries = golden.manifest["uniform"]
    assert len(entries) > 100
    for e in entries:
        data = golden.get(e["input"])
        q = O.quantize(data, bits=e["bits"], group_size=e["group"], metadata_dtype=DTYPES[e["meta"]], axis=e["axis"])
        assert golden.matches(e["values"], q.values), e["tag"]
        assert golden.matches(e["scale"], q.scale), e["tag"]
        assert golden.matches(e["zero"], q.zero_point), e["tag"]
        assert golden.matches(e["deq"], q.dequantize()), e["tag"]
        assert (q.padded_dim, q.packed_dim) == (e["padded_dim"], e["packed_dim"])


def test_mixed_key_matches_reference_including_tie_order(golden):
    entries = golden.manifest["mixed"]
    assert len(entries) == 29
    for e in entries:
        keys = _input(golden, e, DTYPES[e["dtype"]])
        mk = O.quantize_key_mixed(keys, group_size=e["group"], promote_ratio=e["ratio"],
                                  strategy=e["strategy"], metadata_dtype=DTYPES[e["meta"]])
        for field, actual in (("low", mk.low_values), ("high", mk.high_values), ("idx", mk.channel_indices),
                              ("scale", mk.scale), ("zero", mk.zero_point), ("deq", mk.dequantize())):
            assert golden.matches(e[field], actual), (e["tag"], field)
        assert mk.padded_tokens == e["padded_tokens"]


def _lifecycle_inputs(golden, e):
    dtype = DTYPES[e["dtype"]]
    if "keys" in e:
        return golden.get(e["keys"]), golden.get(e["values"]), golden.get(e["query"])
    total = sum(e["updates"])
    outliers = 0 if e["name"] == "c1" else (8 if e["D"] >= 64 else 2)
    k, v, q = synthetic.outlier_kv(e["B"], e["Hkv"], total, e["D"], query_heads=e["Hq"], dtype=dtype, outliers=outliers)
    from tests.golden_util import sha256
    assert sha256(k) == e["keys_sha256"] and sha256(v) == e["values_sha256"] and sha256(q) == e["query_sha256"]
    return k, v, q


def _oracle_config(cfg: dict) -> O.OracleConfig:
    kw = dict(cfg)
    if "metadata_dtype" in kw:
        kw["metadata_dtype"] = DTYPES[kw["metadata_dtype"]]
    return O.OracleConfig(**kw)


def _seg_fields(seg):
    if isinstance(seg, torch.Tensor):
        return {"dense": seg}
    if isinstance(seg, O.OMixedKey):
        return {"low": seg.low_values, "high": seg.high_values, "idx": seg.channel_indices,
                "scale": seg.scale, "zero": seg.zero_point}
    return {"values": seg.values, "scale": seg.scale, "zero": seg.zero_point}


@pytest.mark.parametrize("name", ["c2", "c1", "nonheld", "held_mixed", "kitty_local", "kitty_value_local",
                                  "uniform_mix_bits", "f64_mixed", "f64_uniform", "f64_meta16"])
def test_cache_lifecycle_and_streamed_attention_match_reference(golden, name):
    e = next(x for x in golden.manifest["cache"] if x["name"] == name)
    keys, values, query = _lifecycle_inputs(golden, e)
    cache = O.OracleCache(_oracle_config(e["config"]))
    start = 0
    for n in e["updates"]:
        cache.append(keys[..., start:start + n, :], values[..., start:start + n, :])
        start += n
    ranges = cache.page_ranges()
    assert [[s, s + n] for s, n, _, _ in ranges] == e["ranges"]
    assert [km for _, _, km, _ in ranges] == e["key_modes"]
    assert [vm for _, _, _, vm in ranges] == e["value_modes"]
    segs = cache.segments()
    assert len(segs) == len(e["segments"])
    for i, ((kseg, vseg), rec) in enumerate(zip(segs, e["segments"])):
        for side, seg in (("key", kseg), ("value", vseg)):
            fields = _seg_fields(seg)
            assert set(fields) == set(rec[side]), (name, i, side)
            for field, ref in rec[side].items():
                assert golden.matches(ref, fields[field]), (name, i, side, field)
    out, out32 = O.streamed_attention(query, cache, return_fp32=True)
    assert golden.matches(e["attn_out"], out)
    assert golden.matches(e["attn_out_f32"], out32)
    mk, mv = cache.get()
    g = e["Hq"] // e["Hkv"]
    dense = O.dense_attention(query, mk.repeat_interleave(g, dim=1), mv.repeat_interleave(g, dim=1))
    assert golden.matches(e["dense_attn"], dense)


def test_pack_unpack_closed_form():
    """LSB-first layout: element j of a byte sits at bits [j*b, (j+1)*b)."""
    for bits in (2, 4, 8):
        per = 8 // bits
        codes = torch.randint(0, 1 << bits, (3, 5 * per + 1), dtype=torch.uint8)
        packed = O.pack(codes, bits, ((codes.shape[-1] + per - 1) // per) * per)
        for j in range(codes.shape[-1]):
            assert torch.equal((packed[:, j // per] >> ((j % per) * bits)) & ((1 << bits) - 1), codes[:, j])
        assert torch.equal(O.unpack(packed, bits, codes.shape[-1]), codes)


def test_quantize_invariants_brute_force():
    """Codes in range, group min -> 0, round trip within scale/2 plus the source-dtype roundings.

    u is the unit roundoff of the source dtype: the scale itself is rounded
    (relative u, times up to qmax), the quotient is rounded before rint, and
    the restored value is rounded to the source dtype.
    """
    torch.manual_seed(0)
    unit = {torch.float32: 2.0 ** -24, torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        x = (torch.randn(4, 6, 33) * 3).to(dtype)
        u = unit[dtype]
        for bits in (2, 4, 8):
            qmax = (1 << bits) - 1
            q = O.quantize(x, bits=bits, group_size=8, metadata_dtype=torch.float32)
            codes = O.unpack(q.values, bits, q.packed_dim)[..., : q.padded_dim].reshape(4, 6, -1, 8)
            assert int(codes.max()) <= qmax
            assert int(codes.amin(dim=-1).max()) == 0
            restored = q.dequantize(dtype=torch.float32)
            err = (restored - x.float()).abs()
            scale = q.scale.float().repeat_interleave(8, dim=-1)[..., :33]
            bound = scale * (0.5 + 2 * qmax * u + 4 * u) + 2 * u * x.float().abs() + 1e-6
            assert bool((err <= bound).all()), (dtype, bits, float((err - bound).max()))


def test_streamed_attention_equals_dense_on_materialized_cache():
    """Online softmax over pages equals one softmax over the materialized cache."""
    torch.manual_seed(7)
    keys = torch.randn(1, 2, 19, 8)
    values = torch.randn_like(keys)
    query = torch.randn(1, 4, 3, 8)
    cache = O.OracleCache(O.OracleConfig(page_size=5, key_group_size=5, value_group_size=4, promote_ratio=0.25,
                                         sink_tokens=1, metadata_dtype=torch.float32))
    cache.append(keys, values)
    mk, mv = cache.get()
    expected = O.dense_attention(query, mk.repeat_interleave(2, dim=1), mv.repeat_interleave(2, dim=1))
    torch.testing.assert_close(O.streamed_attention(query, cache), expected, rtol=2e-3, atol=2e-3)


def test_reference_test_literals_page_layout():
    """Literals from the reference tests (tests/test_cache.py:76-123, :217-262)."""
    torch.manual_seed(51)
    keys = torch.randn(1, 2, 11, 12)
    cache = O.OracleCache(O.OracleConfig(page_size=4, hold_partial_pages=True, sink_tokens=2, key_group_size=4,
                                         value_group_size=6, promote_ratio=0.25, metadata_dtype=torch.float32))
    cache.append(keys, torch.randn_like(keys))
    assert [(s, n) for s, n, _, _ in cache.page_ranges()] == [(0, 2), (2, 4), (6, 4), (10, 1)]
    assert [km for _, _, km, _ in cache.page_ranges()] == [0, 2, 2, 0]
    assert [vm for _, _, _, vm in cache.page_ranges()] == [0, 1, 1, 0]
    keys = torch.randn(1, 1, 13, 8)
    cache = O.OracleCache(O.OracleConfig(page_size=4, local_tokens=4, key_group_size=4, value_group_size=4,
                                         metadata_dtype=torch.float32))
    cache.append(keys, keys)
    assert [(km, n) for _, n, km, _ in cache.page_ranges()] == [(1, 4), (1, 4), (0, 5)]
    cache.append(keys[..., :3, :], keys[..., :3, :])
    assert [(km, n) for _, n, km, _ in cache.page_ranges()] == [(1, 4), (1, 4), (1, 4), (0, 4)]


def test_storage_bytes_formula_matches_reference(golden):
    """Config-2 storage: 7 pages x 8 heads x 10,880 B + dense sink and tail = 1,133,568 B,
    the reference profile's figure (docs/PROFILE.md:101) and its cache.storage_bytes."""
    per_page = O.algorithmic_page_bytes(128, 128, 2, 2, 2, 128, 64, 32, 2)
    assert per_page == 10880
    dense_sink = 8 * 32 * 128 * 2 * 2
    dense_tail = 8 * 96 * 128 * 2 * 2
    total = 8 * 7 * per_page + dense_sink + dense_tail
    assert total == 1_133_568
    c2 = next(x for x in golden.manifest["cache"] if x["name"] == "c2")
    assert c2["storage_bytes"] == total

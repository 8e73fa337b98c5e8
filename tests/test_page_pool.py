"""The device page pool behind DartKVCache (GPU): byte-exact batch reordering, page runs as pool slices,
page tables as views of the page directory, and attention for shapes beyond the HIP decode kernels.

Reordering is checked against the cache's own bytes (every packed field of every segment, row by row)
and against the oracle on the reordered inputs; the reference re-quantizes reordered rows
(integrations/huggingface.py:117-127), which this build does not by default, so that oracle comparison
is of decode outputs, not of codes.  The adapter's opt-in ``requantize_on_reorder`` mode rebuilds the
layer as the reference does, and is checked bit for bit against the oracle doing the same.
"""

from __future__ import annotations

import pytest
import torch

from tests.golden_util import bits_equal

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _fields(seg):
    if isinstance(seg, torch.Tensor):
        return [seg]
    if hasattr(seg, "low_values"):
        return [seg.low_values, seg.high_values, seg.channel_indices, seg.scale, seg.zero_point]
    return [seg.values, seg.scale, seg.zero_point]


def _snapshot(cache):
    return [[t.detach().clone() for t in _fields(k) + _fields(v)] for k, v in cache.iter_segments()]


def _cache(B, T, **over):
    import dartkv_amd as dart
    from dartkv_amd import synthetic
    cfg = dict(bits=2, page_size=128, key_group_size=128, value_group_size=64, promote_ratio=0.25, sink_tokens=32,
               hold_partial_pages=True, metadata_dtype=torch.float16)
    cfg.update(over)
    k, v, q = synthetic.outlier_kv(B, 4, T, 128, query_heads=16, dtype=torch.bfloat16, seed=B * 7 + T, device=DEV)
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    cache.append(k, v)
    return cache, k, v, q


@pytest.mark.parametrize("index", [[2, 0, 1], [1, 1, 0], [0, 2], [2, 2, 1, 0, 0]])
@pytest.mark.parametrize("over", [{}, dict(promote_ratio=0.0, bits=4), dict(page_size=64, key_group_size=32,
                                                                              value_group_size=32, sink_tokens=5)])
def test_reorder_batch_gathers_packed_bytes(index, over):
    """Every packed field of every segment, batch row by row, is the old row the index names; the decode
    of the reordered cache is the reordered decode, bit for bit."""
    import dartkv_amd as dart
    cache, k, v, q = _cache(3, 700, **over)
    before = _snapshot(cache)
    out_before = dart.decode_attention(q, cache)
    idx = torch.tensor(index, device=DEV)
    cache.reorder_batch(idx)
    after = _snapshot(cache)
    assert len(after) == len(before)
    for seg_before, seg_after in zip(before, after):
        for a, b in zip(seg_before, seg_after):
            assert bits_equal(a.index_select(0, idx).cpu(), b.cpu())
    out_after = dart.decode_attention(q.index_select(0, idx), cache)
    torch.cuda.synchronize()
    expected = out_before.index_select(0, idx).cpu()
    if len(index) == 3:  # same batch size, same split counts: the same arithmetic
        assert bits_equal(out_after.cpu(), expected)
    else:  # another batch size may choose other split counts: held to the parity bar against the oracle
        from oracle import dart_oracle as O
        cfg = dict(bits=2, page_size=128, key_group_size=128, value_group_size=64, promote_ratio=0.25,
                   sink_tokens=32, hold_partial_pages=True, metadata_dtype=torch.float16)
        cfg.update(over)
        qi = q.index_select(0, idx)
        out32 = torch.empty(len(index), qi.shape[1], 128, dtype=torch.float32, device=DEV)
        dart.decode_attention(qi, cache, out_f32=out32)
        oc = O.OracleCache(O.OracleConfig(**cfg))
        oc.append(k.index_select(0, idx).cpu(), v.index_select(0, idx).cpu())
        _, ref32 = O.streamed_attention(qi.cpu(), oc, return_fp32=True)
        a, b = out32.cpu(), ref32.reshape(out32.shape)
        err = float(((a - b).abs().amax(-1) / b.abs().amax(-1)).max())
        assert err <= 2e-3, err
    assert cache.shape[0] == len(index)
    # appends after a reorder keep working: one token, then enough to seal a page
    nk, nv = k[:1, :, :200].expand(len(index), -1, -1, -1).contiguous(), v[:1, :, :200].expand(len(index), -1, -1, -1).contiguous()
    cache.append(nk[:, :, :1], nv[:, :, :1])
    cache.append(nk[:, :, 1:], nv[:, :, 1:])
    assert cache.get_seq_length() == 900
    assert bool(torch.isfinite(dart.decode_attention(q.index_select(0, idx), cache).float()).all())


def test_reordered_cache_decodes_like_the_oracle_on_reordered_inputs():
    import dartkv_amd as dart
    from oracle import dart_oracle as O
    cache, k, v, q = _cache(3, 900)
    idx = [2, 0, 1]
    cache.reorder_batch(idx)
    out32 = torch.empty(3, 16, 128, dtype=torch.float32, device=DEV)
    dart.decode_attention(q[idx], cache, out_f32=out32)
    cfg = dict(bits=2, page_size=128, key_group_size=128, value_group_size=64, promote_ratio=0.25, sink_tokens=32,
               hold_partial_pages=True, metadata_dtype=torch.float16)
    oc = O.OracleCache(O.OracleConfig(**cfg))
    oc.append(k[idx].cpu(), v[idx].cpu())
    _, ref32 = O.streamed_attention(q[idx].cpu(), oc, return_fp32=True)
    a, b = out32.cpu(), ref32.reshape(3, 16, 128)
    err = float(((a - b).abs().amax(-1) / b.abs().amax(-1)).max())
    assert err <= 2e-3, err


def test_hf_reorder_select_and_repeat_keep_bytes_and_length():
    import dartkv_amd as dart
    from dartkv_amd.integrations import DartHFCache
    from dartkv_amd import synthetic
    cfg = dart.DartKVCacheConfig(bits=2, page_size=16, key_group_size=16, value_group_size=16, promote_ratio=0.25,
                                 sink_tokens=3, hold_partial_pages=True, metadata_dtype=torch.float16)
    k, v, _ = synthetic.outlier_kv(4, 2, 50, 32, dtype=torch.bfloat16, seed=3, device=DEV)
    hf = DartHFCache(cfg)
    for layer in range(2):
        hf.update(k, v, layer)
    rows0 = [hf.layer_for_attention(i).get() for i in range(2)]
    epoch = hf.graph_epoch
    hf.reorder_cache(torch.tensor([3, 2, 1, 0]))
    assert hf.graph_epoch == epoch + 1 and hf.get_seq_length() == 50
    for i in range(2):
        kk, vv = hf.layer_for_attention(i).get()
        assert bits_equal(kk.cpu(), rows0[i][0].flip(0).cpu()) and bits_equal(vv.cpu(), rows0[i][1].flip(0).cpu())
    hf.batch_select_indices(torch.tensor([0, 2]))
    kk, _ = hf.layer_for_attention(0).get()
    assert kk.shape[0] == 2 and bits_equal(kk.cpu(), rows0[0][0][[3, 1]].cpu())
    hf.batch_repeat_interleave(2)
    kk, _ = hf.layer_for_attention(1).get()
    assert kk.shape[0] == 4 and bits_equal(kk.cpu(), rows0[1][0][[3, 3, 1, 1]].cpu())
    out_k, _ = hf.update(k[:4, :, :1], v[:4, :, :1], 0)
    assert out_k.shape == (4, 2, 51, 32)


def test_page_runs_are_pool_slices_and_tables_follow_the_tail():
    import dartkv_amd as dart
    cache, k, v, q = _cache(2, 1000, promote_ratio=0.0, bits=4)
    runs = cache.page_runs()
    assert len(runs) == 1 and runs[0].page_count == (1000 - 32) // 128
    run = runs[0].validate()
    pairs = cache.iter_segments()
    for p in range(run.page_count):
        ks, vs = pairs[1 + p]
        assert bits_equal(run.key_values[p].cpu(), ks.values.cpu())
        assert bits_equal(run.value_values[p].cpu(), vs.values.cpu())
        assert bits_equal(run.value_scale[p].cpu(), vs.scale.cpu())
    pool = cache._key_pool
    assert run.key_values.data_ptr() == pool.tensors["values"][pairs[1][0]._at].data_ptr()  # a view, not a copy
    assert run.value_values.untyped_storage().data_ptr() == cache._value_pool.tensors["values"].untyped_storage().data_ptr()
    table = cache.page_table()
    assert table.sequence_starts.untyped_storage().data_ptr() == table.token_counts.untyped_storage().data_ptr()
    last = table.token_counts[-1].item()
    cache.append(k[:, :, :1], v[:, :, :1])
    fresh = cache.page_table().validate()
    assert fresh is not table and fresh.token_counts[-1].item() == last + 1
    assert table.token_counts[-1].item() == last  # an old table keeps its snapshot
    assert fresh.page_count == table.page_count


@pytest.mark.parametrize("Hkv,Hq,D", [(1, 20, 64), (2, 4, 640)])
def test_shapes_beyond_the_decode_kernels_fall_back_to_segment_attention(Hkv, Hq, D):
    """More than 16 query heads per KV head, or head_dim above 512: fused (fallback=True) and streamed
    attention run segment_attention and match the oracle; fused with fallback=False raises."""
    import dartkv_amd as dart
    from dartkv_amd import synthetic
    from dartkv_amd.attention import segment_attention
    from oracle import dart_oracle as O
    cfg = dict(bits=2, page_size=32, key_group_size=32, value_group_size=32, promote_ratio=0.25, sink_tokens=4,
               hold_partial_pages=True, metadata_dtype=torch.float16)
    k, v, q = synthetic.outlier_kv(2, Hkv, 150, D, query_heads=Hq, dtype=torch.bfloat16, seed=D)
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    cache.append(k.to(DEV), v.to(DEV))
    oc = O.OracleCache(O.OracleConfig(**cfg))
    oc.append(k, v)
    _, ref32 = O.streamed_attention(q, oc, return_fp32=True)
    out32 = torch.empty(2, Hq, 1, D, dtype=torch.float32, device=DEV)
    segment_attention(q.to(DEV), cache, out_f32=out32)
    a, b = out32.cpu().flatten(2), ref32.flatten(2)
    err = float(((a - b).abs().amax(-1) / b.abs().amax(-1)).max())
    assert err <= 1e-5, err
    fused = dart.fused_dart_attention(q.to(DEV), cache)
    streamed = dart.streamed_dart_attention(q.to(DEV), cache)
    assert bits_equal(fused.cpu(), streamed.cpu())
    with pytest.raises(ValueError, match="query heads per KV head"):
        dart.fused_dart_attention(q.to(DEV), cache, fallback=False)


@pytest.mark.parametrize("start", [96, 100])
def test_one_token_appends_reach_decode_after_a_decode_at_any_tail_length(start):
    """Decode after each of several one-token appends, starting with an empty held tail (the prompt ends on
    a page boundary) or a partial one: the decode plan built for the sealed pages reads the tail per call,
    so every new token is attended (oracle on the same inputs, fp32 pre-cast output)."""
    import dartkv_amd as dart
    from dartkv_amd import synthetic
    from oracle import dart_oracle as O
    cfg = dict(bits=2, page_size=32, key_group_size=32, value_group_size=32, promote_ratio=0.25, sink_tokens=0,
               hold_partial_pages=True, metadata_dtype=torch.float16)
    k, v, q = synthetic.outlier_kv(2, 2, start + 6, 128, query_heads=8, dtype=torch.bfloat16, seed=start)
    cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
    cache.append(k[:, :, :start].to(DEV), v[:, :, :start].to(DEV))
    oc = O.OracleCache(O.OracleConfig(**cfg))
    oc.append(k[:, :, :start], v[:, :, :start])
    for t in range(start, start + 6):
        out = torch.empty(2, 8, 128, dtype=torch.float32, device=DEV)
        dart.decode_attention(q.to(DEV), cache, out_f32=out)
        _, ref = O.streamed_attention(q, oc, return_fp32=True)
        a, b = out.cpu(), ref.reshape(2, 8, 128)
        err = float(((a - b).abs().amax(-1) / b.abs().amax(-1)).max())
        assert err <= 2e-3, (t, err)
        cache.append(k[:, :, t:t + 1].to(DEV), v[:, :, t:t + 1].to(DEV))
        oc.append(k[:, :, t:t + 1], v[:, :, t:t + 1])
    assert cache.get_seq_length() == start + 6


def test_hf_requantize_on_reorder_rebuilds_like_the_reference():
    """Reference huggingface.py:117-127: each layer is rebuilt from index_select of its materialized rows,
    so the selected rows are quantized again from one prefill; every packed field and the materialized
    contents match an oracle cache rebuilt the same way, bit for bit."""
    import dartkv_amd as dart
    from dartkv_amd.integrations import DartHFCache
    from dartkv_amd import synthetic
    from oracle import dart_oracle as O
    cfg = dict(bits=2, page_size=16, key_group_size=16, value_group_size=16, promote_ratio=0.25, sink_tokens=3,
               hold_partial_pages=True, metadata_dtype=torch.float16)
    k, v, _ = synthetic.outlier_kv(4, 2, 53, 32, dtype=torch.bfloat16, seed=11)
    hf = DartHFCache(dart.DartKVCacheConfig(**cfg), requantize_on_reorder=True)
    oc = O.OracleCache(O.OracleConfig(**cfg))
    hf.update(k[:, :, :50].to(DEV), v[:, :, :50].to(DEV), 0)
    oc.append(k[:, :, :50], v[:, :, :50])
    for t in range(50, 53):  # one-token updates that leave a held tail
        hf.update(k[:, :, t:t + 1].to(DEV), v[:, :, t:t + 1].to(DEV), 0)
        oc.append(k[:, :, t:t + 1], v[:, :, t:t + 1])
    epoch = hf.graph_epoch
    for rows in ([3, 1, 1, 0], [2, 0]):
        if len(rows) == 4:
            hf.reorder_cache(torch.tensor(rows))
        else:
            hf.batch_select_indices(torch.tensor(rows))
        ok, ov = oc.get()
        idx = torch.tensor(rows)
        oc = O.OracleCache(O.OracleConfig(**cfg))
        oc.append(ok.index_select(0, idx), ov.index_select(0, idx))
        cache = hf.layer_for_attention(0)
        torch.cuda.synchronize()
        segs, osegs = cache.iter_segments(), oc.segments()
        assert len(segs) == len(osegs)
        for (ks, vs), (oks, ovs) in zip(segs, osegs):
            for a, b in ((ks, oks), (vs, ovs)):
                fa, fb = _fields(a), _fields(b)
                assert len(fa) == len(fb)
                for x, y in zip(fa, fb):
                    assert bits_equal(x.cpu(), y)
        kk, vv = cache.get()
        ek, ev = oc.get()
        assert bits_equal(kk.cpu(), ek) and bits_equal(vv.cpu(), ev)
        assert hf.get_seq_length() == 53
    assert hf.graph_epoch == epoch + 2


def test_shrinking_batch_selection_frees_the_old_pool_allocation():
    """Selecting fewer batch rows gathers every pool field into tensors of their own; the pool's old
    allocation (all fields of every row) is then released, not kept until the pool next grows."""
    cache, k, v, q = _cache(4, 700)
    kpool, vpool = cache._key_pool, cache._value_pool
    old_bytes = sum(p._buffer.numel() for p in (kpool, vpool) if p._buffer is not None)
    assert old_bytes > 0
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    cache.reorder_batch([2])
    torch.cuda.synchronize()
    after = torch.cuda.memory_allocated()
    assert kpool._buffer is None and vpool._buffer is None
    assert before - after >= old_bytes // 2, (before, after, old_bytes)
    import dartkv_amd as dart
    out = dart.decode_attention(q[[2]], cache)  # the selected row still decodes
    assert torch.isfinite(out.float()).all()

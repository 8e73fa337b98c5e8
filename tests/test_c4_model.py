"""BASELINE config C4 at its real shape on the GPU: a Qwen3-8B-shaped model (36 layers, hidden 4096,
32 query / 8 KV heads, head_dim 128, vocab 151936, random bf16 weights) with the fused adapter and
``DartHFCache`` (2-bit + 25 % key promotion, sink 32, page 128, key group 128, value group 64, fp16
metadata), batch 16, an 8,192-token random prompt, then 40 greedy steps through ``GraphDecodeStep``
(HIP-graph replays, one eager step that seals a page: the tail after the prefill holds
8,192 - 32 - 63 x 128 = 96 tokens).

Reference: examples/benchmark_kitty.py:297-342 runs this shape through ``generate()``; the decode
branch is src/dart/integrations/qwen3.py:72-84.

Checks, for batch rows 0 and 15 of layers 0 and 35:
* every decode call (graph replays included: the call's query and output are copied out by
  the captured graph) equals an eager call on the same cache state bit for bit, and its fp32
  output is within the parity bar (max|a-b| / max|b| per (batch, head) <= 2e-3) of fp32
  attention over the materialized cache;
* the packed pages, including the one sealed from tokens that ``dkv_decode_prep`` appended
  inside replayed steps, equal the oracle's pages bit for bit when the oracle is fed the same
  K/V (the prefill's and each step's token);
* the last step's output is within 2e-3 of the oracle's streamed attention;
* all logits are finite.
"""

from __future__ import annotations

import math

import pytest
import torch

from tests.golden_util import bits_equal

pytestmark = pytest.mark.gpu

DEV = "cuda"
ROWS = [0, 15]
LAYERS = (0, 35)
STEPS = 40


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


def test_c4_qwen3_8b_shape_graph_decode_follows_the_oracle(monkeypatch):
    from transformers import Qwen3Config, Qwen3ForCausalLM

    import dartkv_amd as dart
    from dartkv_amd.integrations import DartHFCache, GraphDecodeStep, attach_dart_fused_attention
    from dartkv_amd.integrations import huggingface as hfmod
    from dartkv_amd.integrations import qwen3 as q3mod
    from oracle import dart_oracle as O

    B, T, Hq, Hkv, D = 16, 8192, 32, 8, 128
    cfg = Qwen3Config(num_hidden_layers=36, layer_types=["full_attention"] * 36, vocab_size=151936,
                      hidden_size=4096, intermediate_size=12288, num_attention_heads=Hq, num_key_value_heads=Hkv,
                      head_dim=D, max_position_embeddings=40960, tie_word_embeddings=False)
    cache_kw = dict(bits=2, page_size=128, key_group_size=128, value_group_size=64, promote_ratio=0.25,
                    sink_tokens=32, hold_partial_pages=True, metadata_dtype=torch.float16)
    torch.manual_seed(20260823)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(DEV):
            model = Qwen3ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(prev)
    model = attach_dart_fused_attention(model).eval()
    scaling = model.model.layers[0].self_attn.scaling
    cache = DartHFCache(dart.DartKVCacheConfig(**cache_kw))
    rows = torch.tensor(ROWS, device=DEV)

    # dense K/V handed to the cache by the update path (prefill, eager seal steps), rows 0 and 15
    appended = {li: [] for li in LAYERS}
    real_update = hfmod.DartHFCache.update

    def recording_update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        if self is cache and layer_idx in appended:
            appended[layer_idx].append((key_states.index_select(0, rows).cpu(),
                                        value_states.index_select(0, rows).cpu()))
        return real_update(self, key_states, value_states, layer_idx, cache_kwargs)

    monkeypatch.setattr(hfmod.DartHFCache, "update", recording_update)

    # each decode call's query and output for the checked layers, copied by the (captured) step itself
    real_fused = q3mod.fused_dart_attention
    layer_of: dict = {}
    qbuf = {li: torch.empty(B, Hq, 1, D, dtype=torch.bfloat16, device=DEV) for li in LAYERS}
    obuf = {li: torch.empty(B, Hq, 1, D, dtype=torch.bfloat16, device=DEV) for li in LAYERS}
    calls = {li: 0 for li in LAYERS}

    def copying_fused(query, layer, *, scale=None, fallback=True, **kw):
        out = real_fused(query, layer, scale=scale, fallback=fallback, **kw)
        li = layer_of.get(id(layer))
        if li is not None:
            qbuf[li].copy_(query)
            obuf[li].copy_(out)
            if not torch.cuda.is_current_stream_capturing():
                calls[li] += 1
        return out

    monkeypatch.setattr(q3mod, "fused_dart_attention", copying_fused)

    ids = torch.randint(0, cfg.vocab_size, (B, T), generator=torch.Generator().manual_seed(5)).to(DEV)
    print("C4 test: prefill", B, "x", T, flush=True)
    with torch.inference_mode():
        out = model(ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
        next_ids = out.logits[:, -1:].argmax(-1)
        assert bool(torch.isfinite(out.logits).all())
        del out
        for li in LAYERS:
            layer_of[id(cache.layers[li].cache)] = li
            assert len(appended[li]) == 1 and appended[li][0][0].shape == (2, Hkv, T, D)
        position = torch.full((1, 1), T, dtype=torch.long, device=DEV)
        runner = GraphDecodeStep(model, cache, next_ids, position, use_graph=True)
        tokens = {li: [] for li in LAYERS}  # (k, v) [2, Hkv, 1, D] of each step, rows 0 and 15
        errs = []
        for step in range(STEPS):
            seen = {li: len(appended[li]) for li in LAYERS}
            replays = runner.replays
            runner.step()
            torch.cuda.synchronize()
            assert bool(torch.isfinite(runner.logits).all()), step
            for li in LAYERS:
                lc = cache.layers[li].cache
                if len(appended[li]) > seen[li]:  # the update path took this step's token
                    k1, v1 = appended[li][-1]
                    assert k1.shape[2] == 1
                else:  # dkv_decode_prep wrote it at the end of the held tail
                    pos = int(lc.device_tail.item())
                    k1 = lc._tail_key.index_select(0, rows)[:, :, pos - 1:pos].cpu()
                    v1 = lc._tail_value.index_select(0, rows)[:, :, pos - 1:pos].cpu()
                tokens[li].append((k1, v1))
                # this step's call, again eagerly on the same cache state: the same bits
                o32 = torch.empty(B, Hq, D, dtype=torch.float32, device=DEV)
                again = dart.decode_attention(qbuf[li], lc, scale=scaling, out_f32=o32)
                assert torch.equal(again, obuf[li]), (step, li)
                k, v = lc.get()
                assert k.shape[2] == T + step + 1
                kf = k.index_select(0, rows).float().repeat_interleave(Hq // Hkv, dim=1)
                vf = v.index_select(0, rows).float().repeat_interleave(Hq // Hkv, dim=1)
                qf = qbuf[li].index_select(0, rows).float()
                p = torch.softmax(torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * scaling, dim=-1)
                ref = torch.matmul(p, vf)[:, :, 0]
                errs.append(_rel_err(o32.index_select(0, rows).unsqueeze(2), ref.unsqueeze(2)))
                del k, v, kf, vf
            if runner.replays == replays:
                print("step", step, "eager or capture; max rel err so far", max(errs), flush=True)
        print("C4 test: captures", runner.captures, "eager steps", runner.eager_steps, "replays", runner.replays,
              "max rel err", max(errs), flush=True)
        assert runner.replays >= STEPS - 6 and runner.eager_steps >= 2
        assert max(errs) <= 2e-3, max(errs)
        assert all(n >= 2 for n in calls.values()), calls  # the eager steps' calls (replays copy too)

        # the packed pages against the oracle fed the same K/V
        for li in LAYERS:
            oc = O.OracleCache(O.OracleConfig(**cache_kw))
            k0, v0 = appended[li][0]
            oc.append(k0, v0)
            for k1, v1 in tokens[li]:
                oc.append(k1, v1)
            lc = cache.layers[li].cache
            segs, osegs = lc.iter_segments(), oc.segments()
            assert len(segs) == len(osegs), li
            sealed = sum(1 for s, _ in osegs if not isinstance(s, torch.Tensor))
            assert sealed == 64, sealed  # 63 pages from the prefill, one sealed by the decode steps
            for i, ((ks, vs), (oks, ovs)) in enumerate(zip(segs, osegs)):
                for side, a, b in (("key", ks, oks), ("value", vs, ovs)):
                    fa, fb = _fields(a), _fields(b)
                    assert len(fa) == len(fb), (li, i, side)
                    for x, y in zip(fa, fb):
                        assert bits_equal(x.index_select(0, rows).cpu(), y), (li, i, side)
            o32 = torch.empty(B, Hq, D, dtype=torch.float32, device=DEV)
            dart.decode_attention(qbuf[li], lc, scale=scaling, out_f32=o32)
            ref32 = O.streamed_attention(qbuf[li].index_select(0, rows).cpu(), oc, scale=scaling,
                                         return_fp32=True)[1]
            err = _rel_err(o32.index_select(0, rows).unsqueeze(2), ref32.reshape(2, Hq, 1, D))
            print("layer", li, "oracle rel err", err, flush=True)
            assert err <= 2e-3, (li, err)
    del model, cache, runner
    torch.cuda.empty_cache()
    assert math.isfinite(max(errs))

"""Benchmark: packed-KV single-token decode attention on a Qwen3-8B-shaped cache.

Workload (config C5, the headline decode configuration): batch 64, 32768-token context per
sequence, 8 KV heads, 32 query heads, head_dim 128, bf16 K/V with 8 outlier
channels per KV head, page 128, key group 128, value group 64, 2-bit codes
with 25 % key-channel promotion, 32 sink tokens, held tail; 36 layers of
packed cache resident in HBM, each layer a separate cache.

One step = one decode token for all 64 sequences through all 36 layers:
36 calls of the decode attention (MFMA page kernel with the dense sink/tail
chunks in its launch, split merge); ``--bits 4b`` runs the 4-bit uniform
variant.  ``value`` is
the algorithmic bytes those calls must read and write (packed pages, dense
sink and tail, query, output) per second of the whole step.  ``roofline`` is
the page kernel alone: its pages' bytes over its mean duration, timed with
HIP events recorded around its launch.

    python bench.py [--gpus 1] [--steps 10] [--warmup 3]

Prints one JSON line.  Only one GPU is supported (``--gpus`` > 1 exits).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def config_for(bits_mode: str) -> dict:
    cfg = dict(page_size=128, key_group_size=128, value_group_size=64, sink_tokens=32, hold_partial_pages=True,
               metadata_dtype=None)
    if bits_mode == "2b25":
        cfg.update(bits=2, promote_ratio=0.25)
    elif bits_mode == "4b":
        cfg.update(bits=4, promote_ratio=0.0)
    else:
        raise ValueError(bits_mode)
    return cfg


def page_bytes(head_dim: int, cfg: dict, meta_bytes: int = 2) -> int:
    """Bytes of one packed page of one (batch, kv head): key and value codes plus metadata."""
    page = cfg["page_size"]
    kg, vg = cfg["key_group_size"], cfg["value_group_size"]
    if cfg.get("promote_ratio", 0.0) > 0:
        K = min(head_dim, int(head_dim * cfg["promote_ratio"] + 1e-6))
        G = (page + kg - 1) // kg
        nb = (kg + 3) // 4
        kbytes = head_dim * G * nb + K * G * nb + 4 * K + 2 * head_dim * G * meta_bytes
    else:
        per = 8 // cfg["bits"]
        G = (page + kg - 1) // kg
        kbytes = head_dim * ((G * kg + per - 1) // per) + 2 * head_dim * G * meta_bytes
    per = 8 // cfg["bits"]
    gv = (head_dim + vg - 1) // vg
    vbytes = page * ((gv * vg + per - 1) // per) + 2 * page * gv * meta_bytes
    return kbytes + vbytes


def algorithmic_bytes(batch: int, kv_heads: int, q_heads: int, context: int, head_dim: int, cfg: dict,
                      elem: int = 2, meta_bytes: int = 2) -> int:
    """Bytes one decode launch must move: packed pages + dense sink/tail + query + output."""
    page = cfg["page_size"]
    sink = min(cfg["sink_tokens"], context)
    pages = (context - sink) // page
    tail = context - sink - pages * page
    per_bh = pages * page_bytes(head_dim, cfg, meta_bytes) + (sink + tail) * head_dim * elem * 2
    return batch * kv_heads * per_bh + 2 * batch * q_heads * head_dim * elem


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` recorded in profiles/ (PMC FETCH_SIZE + WRITE_SIZE, calibrated), or None."""
    path = os.path.join(REPO, "profiles", f"{kernel}_{workload}_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip())
    return None


def build_caches(args, torch, dart, synthetic):
    cfg = config_for(args.bits)
    cfg["metadata_dtype"] = torch.float16
    dev = torch.device("cuda:0")
    log(f"building {args.layers} layer caches: B={args.batch} T={args.context} Hkv={args.kv_heads} D={args.head_dim}")
    t0 = time.time()
    keys, values, _ = synthetic.outlier_kv(args.batch, args.kv_heads, args.context, args.head_dim,
                                           query_heads=args.q_heads, dtype=torch.bfloat16, device=dev)
    caches = []
    for layer in range(args.layers):
        cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg))
        cache.append(keys, values)
        caches.append(cache)
        if layer == 0:
            torch.cuda.synchronize()
            log(f"  layer 0 quantized in {time.time() - t0:.2f}s")
    torch.cuda.synchronize()
    del keys, values
    torch.cuda.empty_cache()
    gen = torch.Generator(device=dev).manual_seed(1)
    queries = [torch.randn(args.batch, args.q_heads, 1, args.head_dim, generator=gen, device=dev).to(torch.bfloat16)
               for _ in range(args.layers)]
    log(f"caches ready in {time.time() - t0:.1f}s; storage {sum(c.storage_bytes for c in caches) / 1e9:.2f} GB")
    return cfg, caches, queries


def cpu_baseline(args, cfg, budget_s: float = 20.0) -> dict:
    """Oracle (CPU PyTorch restatement of the reference) on a bounded sample of the same workload."""
    import torch

    from dartkv_amd import synthetic
    from oracle import dart_oracle as O

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    ocfg = dict(cfg)
    ocfg["metadata_dtype"] = torch.float16
    k, v, q = synthetic.outlier_kv(1, args.kv_heads, args.context, args.head_dim, query_heads=args.q_heads,
                                   dtype=torch.bfloat16)
    oc = O.OracleCache(O.OracleConfig(**ocfg))
    oc.append(k, v)
    bytes_one = algorithmic_bytes(1, args.kv_heads, args.q_heads, args.context, args.head_dim, cfg)
    O.streamed_attention(q, oc)  # warm-up
    reps, t0 = 0, time.perf_counter()
    while True:
        O.streamed_attention(q, oc)
        reps += 1
        if time.perf_counter() - t0 > budget_s or reps >= 50:
            break
    dt = (time.perf_counter() - t0) / reps
    return {"value": round(bytes_one / dt / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": (f"oracle streamed_attention, 1 sequence x 1 layer of the same workload "
                       f"({args.context} tokens, {bytes_one} algorithmic bytes), {reps} reps, {dt * 1e3:.1f} ms each"),
            "tok_s": round(1.0 / (dt * args.layers), 4)}


def _best_time(fn, budget_s: float, max_reps: int = 20):
    """(seconds per call, reps) of fn after one warm-up call, repeated until budget_s has passed."""
    fn()
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        if time.perf_counter() - t0 > budget_s or reps >= max_reps:
            return (time.perf_counter() - t0) / reps, reps


def cpu_baseline_c2(budget_s: float = 4.0) -> dict:
    """C2 in full on the host: the oracle's streamed attention over the config-2 cache (one decode call)."""
    import torch

    from dartkv_amd import synthetic
    from oracle import dart_oracle as O

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    k, v, q = synthetic.outlier_kv(1, 8, 1024, 128, query_heads=32, dtype=torch.bfloat16)
    cfg = config_for("2b25")
    cfg["metadata_dtype"] = torch.float16
    oc = O.OracleCache(O.OracleConfig(**cfg))
    oc.append(k, v)
    dt, reps = _best_time(lambda: O.streamed_attention(q, oc), budget_s)
    nbytes = algorithmic_bytes(1, 8, 32, 1024, 128, cfg)
    return {"value": round(dt * 1e6, 1), "unit": "us per decode call", "cores": threads, "kind": "port",
            "gbs": round(nbytes / dt / 1e9, 4),
            "sample": f"C2 in full (B1, T1024, 8/32 heads, 2-bit + 25 %): oracle streamed_attention, {reps} reps"}


def cpu_baseline_c3(budget_s: float = 6.0) -> dict:
    """C3 at batch 1 on the host: the oracle's append of [1, 8, 16384, 128] bf16 K/V into a 2-bit + 25 % cache."""
    import torch

    from dartkv_amd import synthetic
    from oracle import dart_oracle as O

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    T = 16384
    k, v, _ = synthetic.outlier_kv(1, 8, T, 128, query_heads=32, dtype=torch.bfloat16)
    cfg = config_for("2b25")
    cfg["metadata_dtype"] = torch.float16
    written = []

    def append():
        oc = O.OracleCache(O.OracleConfig(**cfg))
        oc.append(k, v)
        written.append(oc)

    dt, reps = _best_time(append, budget_s, max_reps=5)
    read = 2 * 8 * T * 128 * 2
    stored = sum(s.numel() * s.element_size() if isinstance(s, torch.Tensor) else s.nbytes
                 for pair in written[-1].segments() for s in pair)
    return {"value": round((read + stored) / dt / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "ms": round(dt * 1e3, 1),
            "sample": (f"C3 at batch 1: oracle append of [1, 8, {T}, 128] bf16 K/V into a 2-bit + 25 % cache "
                       f"({read} bytes read, {stored} written), {reps} reps")}


def cpu_baseline_c4_reduced(layers: int = 2, prompt: int = 256, steps: int = 8, seed: int = 20260823) -> dict:
    """C4 reduced, on the host: a Qwen3-8B-shaped model cut to ``layers`` layers (full width, full vocab,
    random bf16 weights), batch 1, a ``prompt``-token random prompt and ``steps`` greedy steps.  Attention
    follows the reference's dart engine on a CPU tensor: prefill attends to its raw keys and values and then
    packs them (post-quantization return), each decode step appends its token to the oracle cache and runs
    the oracle's streamed attention over the packed pages."""
    import torch
    from transformers import Qwen3Config, Qwen3ForCausalLM
    from transformers.models.qwen3 import modeling_qwen3 as M

    from oracle import dart_oracle as O

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    cfg = Qwen3Config(num_hidden_layers=layers, layer_types=["full_attention"] * layers, **QWEN3_8B)
    # weights: a 1 Mi-element random N(0, 0.02) block tiled over every matrix (an i.i.d. fill of 1.6 G
    # parameters takes about a minute on the host), norms 1
    with torch.device("meta"):
        model = Qwen3ForCausalLM(cfg)
    model = model.to(torch.bfloat16).to_empty(device="cpu").eval()
    model.model.rotary_emb = M.Qwen3RotaryEmbedding(config=cfg)
    block = (torch.randn(1 << 20, generator=torch.Generator().manual_seed(seed)) * 0.02).to(torch.bfloat16)
    with torch.no_grad():
        for name, p in model.named_parameters():
            flat = p.view(-1)
            if "norm" in name:
                flat.fill_(1.0)
                continue
            whole = flat.numel() // block.numel() * block.numel()
            if whole:
                flat[:whole].view(-1, block.numel()).copy_(block.expand(whole // block.numel(), -1))
            if flat.numel() > whole:
                flat[whole:].copy_(block[:flat.numel() - whole])
    ccfg = config_for("2b25")
    ccfg["metadata_dtype"] = torch.float16
    caches = [O.OracleCache(O.OracleConfig(**ccfg)) for _ in range(layers)]

    def attention(attn, hidden_states, position_embeddings, attention_mask=None, **kwargs):
        shape = (*hidden_states.shape[:-1], -1, attn.head_dim)
        q = attn.q_norm(attn.q_proj(hidden_states).view(shape)).transpose(1, 2)
        k = attn.k_norm(attn.k_proj(hidden_states).view(shape)).transpose(1, 2)
        v = attn.v_proj(hidden_states).view(shape).transpose(1, 2)
        q, k = M.apply_rotary_pos_emb(q, k, *position_embeddings)
        cache = caches[attn.layer_idx]
        if cache.seen == 0:
            g = q.shape[1] // k.shape[1]
            out = torch.nn.functional.scaled_dot_product_attention(
                q.float(), k.repeat_interleave(g, 1).float(), v.repeat_interleave(g, 1).float(), is_causal=True,
                scale=attn.scaling).to(q.dtype)
            cache.append(k, v)
        else:
            cache.append(k, v)
            out = O.streamed_attention(q, cache, scale=attn.scaling)
        out = out.transpose(1, 2).reshape(*hidden_states.shape[:-1], -1)
        return attn.o_proj(out), None

    for layer in model.model.layers:
        layer.self_attn.forward = (lambda a: (lambda *x, **kw: attention(a, *x, **kw)))(layer.self_attn)
    ids = torch.randint(0, cfg.vocab_size, (1, prompt), generator=torch.Generator().manual_seed(seed))
    with torch.inference_mode():
        logits = model(ids, use_cache=False, logits_to_keep=1).logits
        nxt = logits[:, -1:].argmax(-1)
        t0 = time.perf_counter()
        for step in range(steps):
            pos = torch.tensor([[prompt + step]])
            nxt = model(nxt, position_ids=pos, use_cache=False, logits_to_keep=1).logits[:, -1:].argmax(-1)
        dt = (time.perf_counter() - t0) / steps
    return {"value": round(1.0 / dt, 3), "unit": "tok/s (reduced)", "cores": threads, "kind": "port",
            "ms_per_step": round(dt * 1e3, 1),
            "sample": (f"C4 REDUCED: Qwen3-8B shape cut to {layers} layers (hidden 4096, 32/8 heads, vocab 151936, "
                       f"tiled random bf16 weights), batch 1, {prompt}-token prompt, {steps} greedy steps; oracle cache "
                       "(2-bit + 25 %, sink 32, page 128) and oracle streamed attention per decode step")}


def prefill_c3(torch, dart, synthetic, stream, cfg: dict) -> dict:
    """C3 prefill: one append of [8, 8, 16384, 128] bf16 K/V into a 2-bit + 25 % cache, then 256 one-token appends.

    ``uniform_sweep`` times the same append into uniform 2-, 4- and 8-bit caches (no promotion).
    GB/s counts the K/V bytes read plus the packed bytes written (pages, metadata, dense sink and tail).
    ``append_us`` is the mean time per append of 256 one-token appends (HIP events around the loop;
    two of them seal a page).
    """
    B, H, T, D = 8, 8, 16384, 128
    k, v, _ = synthetic.outlier_kv(B, H, T + 256, D, query_heads=32, dtype=torch.bfloat16, device="cuda:0")
    kp, vp = k[:, :, :T].contiguous(), v[:, :, :T].contiguous()
    ccfg = dict(cfg)
    warm = dart.DartKVCache(dart.DartKVCacheConfig(**ccfg))
    warm.append(kp[:, :, :1024], vp[:, :, :1024])
    for i in range(130):  # one-token appends through a page seal: first-use costs stay out of the timing
        warm.append(k[:, :, T + i % 256:T + i % 256 + 1], v[:, :, T + i % 256:T + i % 256 + 1])
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed_append(config: dict):
        """Best of three one-shot appends of the whole prefill into a fresh cache."""
        times = []
        for _ in range(3):
            cache = dart.DartKVCache(dart.DartKVCacheConfig(**config))
            torch.cuda.synchronize()
            e0.record(stream)
            cache.append(kp, vp)
            e1.record(stream)
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1))
        return min(times), cache

    read = 2 * B * H * T * D * 2
    # the uniform 2/4/8-bit widths of the config's sweep (one append each, no promotion)
    sweep = {}
    for bits in (2, 4, 8):
        ucfg = dict(ccfg, bits=bits, promote_ratio=0.0)
        ums, ucache = timed_append(ucfg)
        sweep[f"{bits}b"] = {"ms": round(ums, 3), "bytes_written": ucache.storage_bytes,
                             "gbs": round((read + ucache.storage_bytes) / (ums * 1e-3) / 1e9, 2)}
        del ucache
    ms, cache = timed_append(ccfg)
    written = cache.storage_bytes
    e0.record(stream)
    for i in range(256):
        cache.append(k[:, :, T + i:T + i + 1], v[:, :, T + i:T + i + 1])
    e1.record(stream)
    torch.cuda.synchronize()
    return {"workload": "C3 prefill: batch 8, 8 KV heads, 16384 tokens, head_dim 128, bf16, 2-bit + 25 %",
            "ms": round(ms, 3), "bytes_read": read, "bytes_written": written,
            "gbs": round((read + written) / (ms * 1e-3) / 1e9, 2),
            "append_us": round(e0.elapsed_time(e1) / 256 * 1e3, 2), "uniform_sweep": sweep}


def config2_latency(torch, dart, synthetic, stream, calls: int = 200) -> dict:
    """One decode call on config 2 (B1, T1024, 8/32 heads, 2-bit + 25 %), three ways:
    ``call_us`` eager calls back to back (HIP events around the loop: host and GPU time together),
    ``host_us`` the host's wall time per eager call, ``gpu_us`` the median GPU span of one call whose
    launches were all enqueued before the GPU reached them (GPU time alone)."""
    k2, v2, q2 = synthetic.outlier_kv(1, 8, 1024, 128, query_heads=32, dtype=torch.bfloat16, device="cuda:0")
    c2cfg = config_for("2b25")
    c2cfg["metadata_dtype"] = torch.float16
    c2 = dart.DartKVCache(dart.DartKVCacheConfig(**c2cfg))
    c2.append(k2, v2)
    for _ in range(5):
        dart.decode_attention(q2, c2)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    e0.record(stream)
    for _ in range(calls):
        dart.decode_attention(q2, c2)
    e1.record(stream)
    w1 = time.perf_counter()
    torch.cuda.synchronize()
    call_us = e0.elapsed_time(e1) / calls * 1e3
    host_us = (w1 - w0) / calls * 1e6
    # GPU span of one call: a spin kernel holds the stream while the host enqueues the call, so the two
    # events bracket GPU work only
    spans = []
    for _ in range(25):
        torch.cuda._sleep(2_000_000)
        e0.record(stream)
        dart.decode_attention(q2, c2)
        e1.record(stream)
        torch.cuda.synchronize()
        spans.append(e0.elapsed_time(e1))
    gpu_us = sorted(spans)[len(spans) // 2] * 1e3
    return {"call_us": round(call_us, 2), "host_us": round(host_us, 2), "gpu_us": round(gpu_us, 2)}


QWEN3_8B = dict(vocab_size=151936, hidden_size=4096, intermediate_size=12288, num_attention_heads=32,
                num_key_value_heads=8, head_dim=128, max_position_embeddings=40960, tie_word_embeddings=False)


def decode_c4(torch, dart, batch: int = 16, prompt: int = 8192, steps: int = 128, layers: int = 36,
              seed: int = 20260823, graph: bool = True) -> dict:
    """C4: Qwen3-8B-shaped greedy decode through DartHFCache + the fused Qwen3 adapter.

    Random-init bf16 weights (no checkpoint), ``batch`` x ``prompt`` random
    token ids, one prefill, then ``steps`` greedy one-token steps; every
    decode attention reads the packed pages (MFMA page kernel).  With
    ``graph`` each step (model forward, argmax, position update) is captured
    once in a HIP graph and replayed; a step that seals a page runs eagerly
    and the graph is captured again after it.  tok/s = batch * steps / decode
    wall time (captures and eager steps included).  ``hbm_bytes_per_step``
    counts the weights (all of them, LM head included) plus the average
    packed cache bytes a step reads.
    """
    from transformers import Qwen3Config, Qwen3ForCausalLM

    from dartkv_amd.integrations import DartHFCache, GraphDecodeStep, attach_dart_fused_attention

    cfg = Qwen3Config(num_hidden_layers=layers, layer_types=["full_attention"] * layers, **QWEN3_8B)
    torch.manual_seed(seed)
    t0 = time.perf_counter()
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("cuda:0"):
            model = Qwen3ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(prev)
    model = attach_dart_fused_attention(model).eval()
    weight_bytes = sum(p.numel() * p.element_size() for p in model.parameters())
    ccfg = config_for("2b25")
    ccfg["metadata_dtype"] = torch.float16
    cache = DartHFCache(dart.DartKVCacheConfig(**ccfg))
    ids = torch.randint(0, cfg.vocab_size, (batch, prompt), generator=torch.Generator().manual_seed(seed)).cuda()
    torch.cuda.synchronize()
    init_s = time.perf_counter() - t0
    log(f"C4: model ready ({weight_bytes / 1e9:.2f} GB weights, {init_s:.1f} s); prefill {batch} x {prompt}")
    with torch.inference_mode():
        t0 = time.perf_counter()
        out = model(ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
        next_ids = out.logits[:, -1:].argmax(-1)
        del out
        position = torch.full((1, 1), prompt, dtype=torch.long, device="cuda:0")
        torch.cuda.synchronize()
        prefill_s = time.perf_counter() - t0
        kv_start = cache.storage_bytes
        log(f"C4: prefill {prefill_s:.2f} s; packed cache {kv_start / 1e9:.2f} GB; {steps} decode steps"
            f"{' (HIP graph)' if graph else ''}")
        runner = GraphDecodeStep(model, cache, next_ids, position, use_graph=graph)
        tokens = []
        t0 = time.perf_counter()
        for _ in range(steps):
            tokens.append(runner.step().clone())
        torch.cuda.synchronize()
        decode_s = time.perf_counter() - t0
    kv_end = cache.storage_bytes
    seq = cache.get_seq_length()
    step_bytes = weight_bytes + (kv_start + kv_end) / 2
    ms = decode_s / steps * 1e3
    result = {
        "workload": (f"C4 Qwen3-8B-shaped decode: {layers} layers, hidden 4096, 32/8 heads, head_dim 128, "
                     f"vocab 151936, random bf16 weights; batch {batch}, {prompt} random prompt ids, {steps} greedy "
                     "steps; cache 2-bit + 25 % key promotion, sink 32, page 128, kg 128, vg 64, fp16 metadata"),
        "tok_s": round(batch * steps / decode_s, 2),
        "ms_per_step": round(ms, 3),
        "hip_graph": graph,
        "graph_captures": runner.captures,
        "eager_steps": runner.eager_steps,
        "prefill_s": round(prefill_s, 3),
        "seq_length_end": seq,
        "weight_bytes": weight_bytes,
        "kv_bytes_start": kv_start,
        "kv_bytes_end": kv_end,
        "hbm_bytes_per_step": int(step_bytes),
        "step_gbs": round(step_bytes / (ms * 1e-3) / 1e9, 1),
        "roofline_tok_s": round(batch / (step_bytes / (HBM_PEAK_GBS * 1e9)), 1),
        "compression_ratio": round(cache.compression_ratio, 3),
    }
    del model, cache, tokens, runner, ids
    torch.cuda.empty_cache()
    return result


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--layers", type=int, default=36)
    p.add_argument("--batch", type=int, default=64)
    p.add_argument("--context", type=int, default=32768)
    p.add_argument("--kv-heads", type=int, default=8)
    p.add_argument("--q-heads", type=int, default=32)
    p.add_argument("--head-dim", type=int, default=128)
    p.add_argument("--bits", choices=["2b25", "4b"], default="2b25")
    p.add_argument("--splits", type=int, default=0, help="split-K count (0 = heuristic)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-c2", action="store_true", help="skip the config-2 latency and C3 prefill probes (clean profiles)")
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                   help="after timing, copy a MIB-MiB buffer 3 times (known bytes for PMC counter calibration)")
    p.add_argument("--no-c4", action="store_true", help="skip the C4 Qwen3-8B-shaped decode leg")
    p.add_argument("--c3-only", action="store_true", help="run only the C3 prefill leg and print its JSON")
    p.add_argument("--c4-only", action="store_true", help="run only the C4 leg and print its JSON")
    p.add_argument("--c2-only", action="store_true", help="run only the config-2 latency leg and print its JSON")
    p.add_argument("--no-c5-4b", action="store_true", help="skip the C5 4-bit uniform sub-leg of the 2b25 run")
    p.add_argument("--no-multi-token", action="store_true", help="skip the multi-token / GQA-8 sub-leg of the C5 run")
    p.add_argument("--c4-steps", type=int, default=128)
    p.add_argument("--c4-prompt", type=int, default=8192)
    p.add_argument("--c4-eager", action="store_true", help="C4 without HIP graph capture of the decode step")
    args = p.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the decode path shards by "
              "(batch, kv-head) with no collective, so per-GPU throughput is the N=1 number.", file=sys.stderr)
        return 2

    import torch

    import dartkv_amd as dart
    from dartkv_amd import synthetic

    if args.c3_only:
        c3cfg = config_for(args.bits)
        c3cfg["metadata_dtype"] = torch.float16
        out = prefill_c3(torch, dart, synthetic, torch.cuda.current_stream(), c3cfg)
        calibration_copy(torch, args.calibrate_copy)
        print(json.dumps(out), flush=True)
        return 0

    if args.c4_only:
        print(json.dumps(decode_c4(torch, dart, prompt=args.c4_prompt, steps=args.c4_steps, graph=not args.c4_eager)),
              flush=True)
        return 0

    if args.c2_only:
        print(json.dumps(config2_latency(torch, dart, synthetic, torch.cuda.current_stream())), flush=True)
        return 0

    stream = torch.cuda.current_stream()
    c5 = time_c5(args, args.bits, torch, dart, synthetic, stream)
    c5_4b = None
    if args.bits == "2b25" and not args.no_c5_4b:
        c5_4b = time_c5(args, "4b", torch, dart, synthetic, stream)
        c5_4b = {k: c5_4b[k] for k in ("value", "unit", "ms_per_step", "hbm_frac", "decode_tok_s", "roofline")}

    prefill = None
    if not args.no_c2:
        prefill = prefill_c3(torch, dart, synthetic, stream, config_for("2b25") | {"metadata_dtype": torch.float16})

    calibration_copy(torch, args.calibrate_copy)

    # config-2 latency (single layer, B1, T1024): the reference's published shape
    c2 = None
    if not args.no_c2:
        c2 = config2_latency(torch, dart, synthetic, stream)

    # C4: the Qwen3-8B-shaped end-to-end decode (tok/s), after the C5 caches are freed
    c4 = None
    if not args.no_c4:
        torch.cuda.empty_cache()
        try:
            c4 = decode_c4(torch, dart, prompt=args.c4_prompt, steps=args.c4_steps, graph=not args.c4_eager)
        except (RuntimeError, ValueError, ImportError) as exc:
            c4 = {"error": f"{type(exc).__name__}: {exc}"[:400]}

    result = {
        "metric": "packed-KV decode-attn GB/s (% HBM peak); decode tok/s, Qwen3-8B-shape",
        "value": c5["value"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": c5["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V with 8 x10 outlier key channels per KV head; random bf16 query)",
        "config": c5["config"],
        "hbm_frac": c5["hbm_frac"],
        "decode_tok_s": c5["decode_tok_s"],
        "c5_4b": c5_4b,
        "multi_token": c5["multi_token"],
        "c2_latency_us": None if c2 is None else c2["call_us"],
        "c2": c2,
        "prefill_c3": prefill,
        "c4_decode": c4,
        "wall_s_timed": c5["wall_s_timed"],
        "roofline": c5["roofline"],
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        log("timing the CPU oracle baselines ...")
        result["cpu_baseline"] = cpu_baseline(args, config_for(args.bits))
        legs = {"c2": cpu_baseline_c2(), "c3_batch1": cpu_baseline_c3()}
        if not args.no_c4:
            legs["c4_reduced"] = cpu_baseline_c4_reduced()
        result["cpu_baseline"]["legs"] = legs
    print(json.dumps(result), flush=True)
    return 0


def calibration_copy(torch, mib: int) -> None:
    """Three copies of a ``mib``-MiB buffer: dispatches of known bytes for PMC counter calibration."""
    if not mib:
        return
    src = torch.empty(mib << 20, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"calibration copy: 3 x {mib} MiB read + written")


def time_c5(args, bits: str, torch, dart, synthetic, stream) -> dict:
    """The C5 decode leg for one bit layout: build the resident layer caches, time args.steps steps,
    return the whole-job rate and the page kernel's roofline figures; the caches are freed after."""
    a = argparse.Namespace(**vars(args))
    a.bits = bits
    cfg, caches, queries = build_caches(a, torch, dart, synthetic)
    nbytes = algorithmic_bytes(a.batch, a.kv_heads, a.q_heads, a.context, a.head_dim, cfg)
    splits = a.splits or None

    def step():
        for cache, q in zip(caches, queries):
            dart.decode_attention(q, cache, n_splits=splits)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # the page kernel (the dominant kernel) is timed by events the library
    # records around its launch on the decode stream
    plan = caches[0].decode_plan(torch.device("cuda:0"))
    fast_bytes = args.batch * args.kv_heads * plan.fast_count * page_bytes(args.head_dim, cfg)
    if plan.fast_count and plan.rest_dense >= 0:
        # every entry outside the page run is dense (the sink and the held tail): the page kernel's launch
        # attends to them too (one wave per 32-token chunk), so their K/V bytes and the query are that
        # launch's as well; the merge launch writes the output
        sink = min(cfg["sink_tokens"], args.context)
        tail = (args.context - sink) % cfg["page_size"]
        fast_bytes += (args.batch * args.kv_heads * (sink + tail) * args.head_dim * 2 * 2
                       + args.batch * args.q_heads * args.head_dim * 2)
    n = args.layers * args.steps
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for e0, e1 in events:  # create the handles before they go to the library
        e0.record(stream)
        e1.record(stream)
    t_begin = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_begin.record(stream)
    i = 0
    for _ in range(args.steps):
        for cache, q in zip(caches, queries):
            dart.decode_attention(q, cache, n_splits=splits, fast_events=events[i] if plan.fast_count else None)
            i += 1
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    total_ms = t_begin.elapsed_time(t_end)
    avg_kernel_ms = None
    if plan.fast_count:
        kernel_ms = [e0.elapsed_time(e1) for e0, e1 in events]
        avg_kernel_ms = sum(kernel_ms) / len(kernel_ms)
    ms_per_step = total_ms / args.steps
    gbs = nbytes * args.layers / (ms_per_step * 1e-3) / 1e9
    achieved = fast_bytes / (avg_kernel_ms * 1e-3) / 1e9 if avg_kernel_ms else None
    kernel = "decode_pages_fast" if plan.fast_promoted else "decode_pages_uniform"
    tok_s = args.batch / (ms_per_step * 1e-3)
    multi = multi_token_leg(torch, dart, caches, a) if bits == "2b25" and not args.no_multi_token else None
    del caches, queries, step, events, plan
    torch.cuda.empty_cache()
    return {
        "value": round(gbs, 2), "unit": "GB/s", "ms_per_step": round(ms_per_step, 4),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "decode_tok_s": round(tok_s, 2), "wall_s_timed": round(wall, 3),
        "config": {
            "workload": (f"C5 long-context decode: batch {a.batch}, {a.context}-token context, "
                         f"{a.kv_heads} KV / {a.q_heads} query heads, head_dim {a.head_dim}, "
                         f"{a.layers} layers resident, {'2-bit + 25% key promotion' if bits == '2b25' else '4-bit uniform'}, "
                         "page 128, kg 128, vg 64, sink 32, fp16 metadata"),
            "batch": a.batch, "context": a.context, "layers": a.layers, "bits": bits,
            "algorithmic_bytes_per_layer": nbytes, "splits": splits or "heuristic",
        },
        "roofline": None if achieved is None else {
            "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(kernel, "c5" if bits == "2b25" else f"c5_{bits}"),
            "kernel": f"{kernel} (MFMA page kernel)",
            "algorithmic_bytes_per_launch": fast_bytes,
            "avg_kernel_us": round(avg_kernel_ms * 1e3, 2),
        },
        "multi_token": multi,
    }


def multi_token_leg(torch, dart, caches, a, steps: int = 3) -> dict:
    """Several query tokens per head over the resident C5 layer caches (fused_dart_attention with Q tokens:
    each token one more query row of its KV group; the Dart page kernel takes 8 rows per KV head, so two
    tokens of a GQA-4 group share each page read), and one token of a GQA-8 query (8 query heads per KV
    head) over the same caches.  Microseconds per layer call (HIP events around `steps` passes over every
    layer after one untimed pass) and the ratio to one token."""
    gen = torch.Generator(device="cuda:0").manual_seed(11)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def per_call_us(queries) -> float:
        for cache, q in zip(caches, queries):
            dart.fused_dart_attention(q, cache)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            for cache, q in zip(caches, queries):
                dart.fused_dart_attention(q, cache)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (steps * len(caches))

    us = {}
    for tokens in (1, 2, 4, 8):
        us[tokens] = per_call_us([torch.randn(a.batch, a.q_heads, tokens, a.head_dim, generator=gen, device="cuda:0",
                                              dtype=torch.bfloat16) for _ in caches])
    gqa8 = per_call_us([torch.randn(a.batch, 8 * a.kv_heads, 1, a.head_dim, generator=gen, device="cuda:0",
                                    dtype=torch.bfloat16) for _ in caches])
    return {"workload": f"C5 caches, query tokens Q per head at GQA {a.q_heads // a.kv_heads}; one token at GQA 8",
            "us_per_layer_call": {f"Q{t}": round(v, 1) for t, v in us.items()},
            "ratio_to_Q1": {f"Q{t}": round(v / us[1], 3) for t, v in us.items()},
            "gqa8_one_token_us": round(gqa8, 1)}



if __name__ == "__main__":
    sys.exit(main())

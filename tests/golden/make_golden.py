"""Write golden vectors for the oracle from the reference implementation.

Run once, in the development container only (the reference is not present on
GPU machines):

    python tests/golden/make_golden.py

It puts ``/root/reference/src`` on ``sys.path`` read-only, runs the reference's
quantizers, cache lifecycle and streamed attention on seeded inputs, and
writes inputs and outputs as safetensors plus a JSON manifest next to this
script.  The fixtures pin the parts of the path that only the reference's own
op sequence fixes: bf16/fp16 codes, scales and zero points, the promoted
channel order (torch.topk tie order), value-page merging, Kitty-mode
lifecycles and the streamed-attention outputs.

Large inputs are regenerated from their seed by ``dartkv_amd.synthetic`` and
pinned by a SHA-256 of their bytes instead of being stored.
"""

from __future__ import annotations

import hashlib
import importlib.util
import json
import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REFERENCE_SRC = "/root/reference/src"


def _load_synthetic():
    spec = importlib.util.spec_from_file_location("dkv_synthetic", os.path.join(REPO, "dartkv_amd", "synthetic.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def sha256(t: torch.Tensor) -> str:
    t = t.contiguous()
    raw = t.view(torch.uint8) if t.dtype != torch.bool else t.to(torch.uint8)
    return hashlib.sha256(raw.numpy().tobytes()).hexdigest()


def main() -> None:
    sys.path.insert(0, REFERENCE_SRC)
    import dart  # noqa: E402  (reference package, read-only)
    from dart.cache import _segment_layout  # noqa: E402

    syn = _load_synthetic()
    tensors: dict[str, torch.Tensor] = {}
    digests: dict[str, dict] = {}
    manifest: dict = {"uniform": [], "mixed": [], "cache": [], "attention": []}

    def put(name: str, t: torch.Tensor, limit: int = 16384) -> str:
        """Store small tensors whole; pin large ones by shape, dtype and SHA-256."""
        t = t.detach().contiguous().clone()
        if t.numel() * t.element_size() <= limit:
            tensors[name] = t
            return name
        digests[name] = {"sha256": sha256(t), "shape": list(t.shape), "dtype": str(t.dtype).replace("torch.", "")}
        return "sha:" + name

    # ---- uniform quantize (quantization.py:134-204) ----
    case = 0
    gen = torch.Generator().manual_seed(1234)
    shapes = [(2, 3, 37, 20), (1, 2, 9, 128), (3, 5, 7)]
    axes_for = {4: ((4, -1), (64, -1), (5, -2), (128, -2)), 3: ((4, -1), (5, -2), (32, 0), (2, 1))}
    for dtype in (torch.bfloat16, torch.float16, torch.float32):
        for shape in shapes:
            base = torch.randn(*shape, generator=gen) * (torch.rand(shape[-1], generator=gen) * 8 + 0.01)
            base[..., 0] = 0.0  # constant-ish column
            data = base.to(dtype)
            for bits in (2, 4, 8):
                for group, axis in axes_for[data.ndim]:
                    for meta in (None, torch.float16, torch.float32, torch.bfloat16):
                        if (bits, meta) not in ((2, None), (4, torch.float16), (8, torch.float32), (2, torch.bfloat16), (2, torch.float16)):
                            continue
                        q = dart.quantize(data, bits=bits, group_size=group, metadata_dtype=meta, axis=axis)
                        tag = f"u{case}"
                        manifest["uniform"].append({
                            "tag": tag, "bits": bits, "group": group, "axis": axis,
                            "meta": None if meta is None else str(meta).replace("torch.", ""),
                            "input": put(tag + ".in", data, limit=1 << 20), "values": put(tag + ".values", q.values),
                            "scale": put(tag + ".scale", q.scale), "zero": put(tag + ".zero", q.zero_point),
                            "deq": put(tag + ".deq", q.dequantize()),
                            "padded_dim": q.padded_dim, "packed_dim": q.packed_dim,
                        })
                        case += 1

    # float64 sources: the reference quantizes them in float64 with eps 1e-6
    # (quantization.py:182-186) and metadata float32 by default.  The inputs get
    # low-order bits a float32 value cannot hold.
    for shape in shapes:
        base = torch.randn(*shape, generator=gen, dtype=torch.float64)
        base = base * (torch.rand(shape[-1], generator=gen, dtype=torch.float64) * 8 + 0.01)
        base[..., 0] = 0.0
        for bits, group, axis, meta in ((2, 4, -1, None), (4, 5, -2, torch.float64), (8, 32, 0, torch.float32),
                                        (2, 64, -1, torch.float16), (4, 4, -1, torch.bfloat16),
                                        (2, 128, -2, torch.float64)):
            q = dart.quantize(base, bits=bits, group_size=group, metadata_dtype=meta, axis=axis)
            tag = f"u{case}"
            manifest["uniform"].append({
                "tag": tag, "bits": bits, "group": group, "axis": axis,
                "meta": None if meta is None else str(meta).replace("torch.", ""),
                "input": put(tag + ".in", base, limit=1 << 20), "values": put(tag + ".values", q.values),
                "scale": put(tag + ".scale", q.scale), "zero": put(tag + ".zero", q.zero_point),
                "deq": put(tag + ".deq", q.dequantize()),
                "padded_dim": q.padded_dim, "packed_dim": q.packed_dim,
            })
            case += 1

    # ---- mixed keys (mixed.py:119-244) ----
    case = 0
    for dtype in (torch.bfloat16, torch.float16, torch.float32):
        for (B, H, T, D, group, ratio, strategy) in (
            (1, 8, 128, 128, 128, 0.25, "magnitude"),   # one config-2 page
            (2, 2, 17, 16, 8, 0.25, "magnitude"),
            (1, 2, 96, 128, 128, 0.25, "magnitude"),     # partial page, replicate padding
            (1, 3, 40, 64, 32, 0.5, "variance"),
            (1, 2, 5, 12, 5, 0.25, "magnitude"),
            (1, 2, 33, 32, 16, 0.01, "magnitude"),       # zero promoted channels
            (1, 1, 16, 8, 8, 1.0, "magnitude"),          # every channel promoted
            (1, 2, 64, 128, 64, 0.02, "magnitude"),      # k*64 <= n: partial_sort path
        ):
            keys, _, _ = syn.outlier_kv(B, H, T, D, dtype=torch.float32, seed=500 + case, outliers=min(8, D // 4))
            keys = keys.to(dtype)
            mk = dart.quantize_key_mixed(keys, group_size=group, promote_ratio=ratio, strategy=strategy,
                                         metadata_dtype=torch.float16)
            tag = f"m{case}"
            manifest["mixed"].append({
                "tag": tag, "group": group, "ratio": ratio, "strategy": strategy, "meta": "float16",
                "shape": [B, H, T, D], "seed": 500 + case, "outliers": min(8, D // 4),
                "dtype": str(dtype).replace("torch.", ""),
                "input": put(tag + ".in", keys), "low": put(tag + ".low", mk.low_values),
                "high": put(tag + ".high", mk.high_values), "idx": put(tag + ".idx", mk.channel_indices),
                "scale": put(tag + ".scale", mk.scale), "zero": put(tag + ".zero", mk.zero_point),
                "deq": put(tag + ".deq", mk.dequantize()), "padded_tokens": mk.padded_tokens,
            })
            case += 1
    # float64 keys (channel scores are float64 means, accumulated in double)
    gen64 = torch.Generator().manual_seed(4321)
    for (B, H, T, D, group, ratio, strategy, meta) in (
        (1, 8, 128, 128, 128, 0.25, "magnitude", torch.float16),
        (2, 2, 17, 16, 8, 0.25, "magnitude", torch.float64),
        (1, 2, 96, 128, 128, 0.25, "variance", torch.float32),
        (1, 3, 40, 64, 32, 0.5, "variance", torch.float64),
        (1, 2, 64, 128, 64, 0.02, "magnitude", torch.float64),
    ):
        keys, _, _ = syn.outlier_kv(B, H, T, D, dtype=torch.float32, seed=500 + case, outliers=min(8, D // 4))
        keys = keys.to(torch.float64) * (1 + 1e-9 * torch.randn(keys.shape, generator=gen64, dtype=torch.float64))
        mk = dart.quantize_key_mixed(keys, group_size=group, promote_ratio=ratio, strategy=strategy,
                                     metadata_dtype=meta)
        tag = f"m{case}"
        manifest["mixed"].append({
            "tag": tag, "group": group, "ratio": ratio, "strategy": strategy,
            "meta": str(meta).replace("torch.", ""), "shape": [B, H, T, D], "seed": 500 + case,
            "outliers": min(8, D // 4), "dtype": "float64",
            "input": put(tag + ".in", keys, limit=1 << 21), "low": put(tag + ".low", mk.low_values),
            "high": put(tag + ".high", mk.high_values), "idx": put(tag + ".idx", mk.channel_indices),
            "scale": put(tag + ".scale", mk.scale), "zero": put(tag + ".zero", mk.zero_point),
            "deq": put(tag + ".deq", mk.dequantize()), "padded_tokens": mk.padded_tokens,
        })
        case += 1

    # ---- cache lifecycles (cache.py:168-542) + streamed attention (attention.py:32-87) ----
    def seg_fields(seg):
        if isinstance(seg, torch.Tensor):
            return {"dense": seg}
        if isinstance(seg, dart.MixedQuantizedKey):
            return {"low": seg.low_values, "high": seg.high_values, "idx": seg.channel_indices,
                    "scale": seg.scale, "zero": seg.zero_point}
        return {"values": seg.values, "scale": seg.scale, "zero": seg.zero_point}

    lifecycles = [
        # name, cfg kwargs, B, Hkv, Hq, D, dtype, update lengths, store_inputs
        ("c2", dict(bits=2, page_size=128, key_group_size=128, value_group_size=64, promote_ratio=0.25,
                    sink_tokens=32, hold_partial_pages=True, metadata_dtype=torch.float16),
         1, 8, 32, 128, torch.bfloat16, [1024], False),
        ("c1", dict(bits=2, group_size=32, sink_tokens=2), 1, 8, 8, 128, torch.float32, [256], False),
        ("nonheld", dict(bits=4, page_size=8, key_group_size=4, value_group_size=6, sink_tokens=3,
                         metadata_dtype=torch.float16), 2, 2, 4, 12, torch.float16, [13, 5, 1, 9, 1, 1], True),
        ("held_mixed", dict(bits=2, page_size=8, key_group_size=8, value_group_size=8, sink_tokens=3,
                            promote_ratio=0.25, hold_partial_pages=True, metadata_dtype=torch.float16),
         1, 2, 4, 16, torch.bfloat16, [21, 1, 1, 9, 1], True),
        ("kitty_local", dict(bits=2, page_size=4, local_tokens=4, key_group_size=4, value_group_size=4,
                             sink_tokens=2, promote_ratio=0.25, metadata_dtype=torch.float32),
         1, 2, 4, 8, torch.float32, [11, 1, 1, 1, 1, 1], True),
        ("kitty_value_local", dict(bits=2, page_size=4, local_tokens=1, value_local_tokens=2, key_group_size=4,
                                   value_group_size=4, promote_ratio=0.25, metadata_dtype=torch.float16),
         1, 2, 2, 8, torch.float16, [8, 1, 1, 1, 1, 3, 1], True),
        ("uniform_mix_bits", dict(bits=4, key_bits=2, value_bits=8, page_size=16, key_group_size=8,
                                  value_group_size=32, sink_tokens=1, hold_partial_pages=True,
                                  metadata_dtype=torch.bfloat16), 2, 2, 8, 64, torch.bfloat16, [40, 1, 20], True),
        # float64 caches: float64 sink and tail, pages quantized in float64
        ("f64_mixed", dict(bits=2, page_size=8, key_group_size=8, value_group_size=8, sink_tokens=3,
                           promote_ratio=0.25, hold_partial_pages=True, metadata_dtype=torch.float64),
         1, 2, 4, 16, torch.float64, [21, 1, 1, 9, 1], True),
        ("f64_uniform", dict(bits=4, page_size=8, key_group_size=4, value_group_size=6, sink_tokens=3,
                             metadata_dtype=torch.float32), 2, 2, 4, 12, torch.float64, [13, 5, 1, 9, 1, 1], True),
        ("f64_meta16", dict(bits=2, page_size=16, key_group_size=16, value_group_size=8, sink_tokens=2,
                            promote_ratio=0.25, metadata_dtype=torch.float16), 1, 2, 8, 32, torch.float64,
         [40, 1, 7], True),
    ]
    gen_lc = torch.Generator().manual_seed(8642)
    for name, cfg_kwargs, B, Hkv, Hq, D, dtype, updates, store_inputs in lifecycles:
        total = sum(updates)
        keys, values, query = syn.outlier_kv(B, Hkv, total, D, query_heads=Hq, dtype=dtype,
                                             outliers=(8 if D >= 64 else 2) if name != "c1" else 0)
        if dtype == torch.float64:
            keys, values, query = (t * (1 + 1e-9 * torch.randn(t.shape, generator=gen_lc, dtype=torch.float64))
                                   for t in (keys, values, query))
        cache = dart.DartKVCache(dart.DartKVCacheConfig(**cfg_kwargs))
        start = 0
        for n in updates:
            cache.update(keys[..., start:start + n, :], values[..., start:start + n, :])
            start += n
        entry = {"name": name, "config": {k: (str(v).replace("torch.", "") if isinstance(v, torch.dtype) else v)
                                          for k, v in cfg_kwargs.items()},
                 "B": B, "Hkv": Hkv, "Hq": Hq, "D": D, "dtype": str(dtype).replace("torch.", ""),
                 "updates": updates, "keys_sha256": sha256(keys), "values_sha256": sha256(values),
                 "query_sha256": sha256(query), "segments": []}
        if store_inputs:
            entry["keys"] = put(f"{name}.keys", keys, limit=1 << 20)
            entry["values"] = put(f"{name}.values", values, limit=1 << 20)
            entry["query"] = put(f"{name}.query", query, limit=1 << 20)
        meta = cache.page_metadata()
        table = cache.page_table()
        entry["ranges"] = table.sequence_ranges().tolist()
        entry["key_modes"] = table.key_modes.tolist()
        entry["value_modes"] = table.value_modes.tolist()
        entry["layouts"] = [[m.key.kind, list(m.key.logical_shape), m.value.kind, list(m.value.logical_shape)] for m in meta]
        entry["storage_bytes"] = cache.storage_bytes
        for i, (kseg, vseg) in enumerate(cache.iter_segments()):
            rec = {"key": {}, "value": {}}
            for side, seg in (("key", kseg), ("value", vseg)):
                for field, t in seg_fields(seg).items():
                    rec[side][field] = put(f"{name}.s{i}.{side}.{field}", t)
            entry["segments"].append(rec)
        out = dart.streamed_dart_attention(query, cache)
        entry["attn_out"] = put(f"{name}.attn_out", out)
        # fp32 pre-cast output: attention.py:86 holds it before `.to(query.dtype)`;
        # an fp32 query makes the final cast the identity.
        entry["attn_out_f32"] = put(f"{name}.attn_out_f32", dart.streamed_dart_attention(query.float(), cache))
        mk, mv = cache.get()
        entry["dense_attn"] = put(f"{name}.dense_attn", dart.dense_attention(
            query, mk.repeat_interleave(Hq // Hkv, dim=1), mv.repeat_interleave(Hq // Hkv, dim=1)))
        manifest["cache"].append(entry)
        _ = _segment_layout  # layouts above come from page_metadata()

    path = os.path.join(HERE, "golden.safetensors")
    save_file(tensors, path)
    with open(os.path.join(HERE, "golden.json"), "w") as fh:
        json.dump({"torch": torch.__version__, "reference": "JaunatisBlue/DartKV @ /root/reference/src",
                   "digests": digests, **manifest}, fh, indent=1)
    print("wrote", path, os.path.getsize(path), "bytes;", len(tensors), "tensors;", len(digests), "digests")


if __name__ == "__main__":
    main()

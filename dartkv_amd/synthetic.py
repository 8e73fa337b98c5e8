"""Seeded synthetic K/V/query tensors for the benchmark and test configurations.

The distributions follow the configurations the reference is measured on:
K ~ N(0, 1) with a few outlier channels per KV head scaled x10, V ~ N(0, 1),
one query token ~ N(0, 1).  Seed 20260823 is the reference's default
(reference examples/run_baseline.py:48, examples/profile_reference.py:69).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

DEFAULT_SEED = 20260823


def outlier_kv(
    batch: int,
    kv_heads: int,
    tokens: int,
    head_dim: int,
    *,
    query_heads: Optional[int] = None,
    dtype: torch.dtype = torch.bfloat16,
    outliers: int = 8,
    seed: int = DEFAULT_SEED,
    device: torch.device | str = "cpu",
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """K [B,Hkv,T,D] with ``outliers`` channels per KV head scaled x10, V, q [B,Hq,1,D].

    Values are drawn in fp32 from a generator on ``device`` and cast to ``dtype``.
    """
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    query_heads = query_heads or kv_heads
    keys = torch.randn(batch, kv_heads, tokens, head_dim, generator=gen, device=device)
    values = torch.randn(batch, kv_heads, tokens, head_dim, generator=gen, device=device)
    if outliers:
        cpu_gen = torch.Generator().manual_seed(seed + 1)
        for head in range(kv_heads):
            channels = torch.randperm(head_dim, generator=cpu_gen)[:outliers].to(device)
            keys[:, head, :, channels] *= 10.0
    query = torch.randn(batch, query_heads, 1, head_dim, generator=gen, device=device)
    return keys.to(dtype), values.to(dtype), query.to(dtype)


def plain_kv(
    batch: int,
    heads: int,
    tokens: int,
    head_dim: int,
    *,
    query_heads: Optional[int] = None,
    dtype: torch.dtype = torch.float32,
    seed: int = DEFAULT_SEED,
    device: torch.device | str = "cpu",
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """K, V ~ N(0,1) and one query token (the CPU smoke configuration's inputs)."""
    return outlier_kv(batch, heads, tokens, head_dim, query_heads=query_heads, dtype=dtype,
                      outliers=0, seed=seed, device=device)

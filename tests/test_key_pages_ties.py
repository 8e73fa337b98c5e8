"""The many-page key path of dkv_quantize_key_pages under score ties.

Past 256 page items a data-dependent channel selection runs as three passes (scores, one selection wave
per page, codes); up to 256 the single-pass kernel selects inside each workgroup.  GPU: for magnitude and
variance scores, on pages with boundary ties (the common case for bf16 means), heavy ties, no ties at all,
all-equal scores and constant channels, the many-page launch writes the same bytes as launching each page
alone, and the oracle's bytes on sample pages.
"""

from __future__ import annotations

import pytest
import torch

from dartkv_amd import _lib, mixed
from tests.golden_util import bits_equal

DEV = "cuda"


def _keys(kind: str, B: int, H: int, T: int) -> torch.Tensor:
    g = torch.Generator().manual_seed({"outliers": 1, "coarse": 2, "distinct": 3, "flat": 4, "mixed": 5}[kind])
    x = torch.randn(B, H, T, 128, generator=g)
    if kind == "outliers":
        x[..., torch.randperm(128, generator=g)[:8]] *= 10.0
    elif kind == "coarse":  # values on a 0.5 grid: scores tie in large groups
        x = (x * 2).round() / 2
    elif kind == "distinct":  # channel scales spread far apart: no two scores equal
        x = x.abs() * (1.07 ** torch.arange(128)) + 1.0
    elif kind == "flat":  # every score equal in one head, constant channels in another
        x[:, 0] = 0.0
        x[:, 1, :, 40:] = 3.0
    elif kind == "mixed":  # pages of every kind in one launch
        x[:, 0] = (x[:, 0] * 2).round() / 2
        x[:, 1] = x[:, 1].abs() * (1.07 ** torch.arange(128)) + 1.0
        x[:, 2, :256] = 0.0
    return x.to(torch.bfloat16)


def _pack(keys: torch.Tensor, selection: str, pages: int) -> tuple:
    B, H, _, D = keys.shape
    K = 32
    low = torch.full((pages, B, H, D, 1, 32), 0xAB, dtype=torch.uint8, device=DEV)
    high = torch.full((pages, B, H, K, 1, 32), 0xCD, dtype=torch.uint8, device=DEV)
    idx = torch.full((pages, B, H, K), -7, dtype=torch.int32, device=DEV)
    scale = torch.zeros(pages, B, H, D, 1, dtype=torch.float16, device=DEV)
    zero = torch.zeros_like(scale)
    mixed.launch_key_pages(keys, page_tokens=128, n_pages=pages, key_mode=_lib.KEY_MIXED, bits=2, group=128,
                           promoted=K, selection={"magnitude": _lib.SELECT_MAGNITUDE,
                                                  "variance": _lib.SELECT_VARIANCE}[selection],
                           given_idx=None, meta=torch.float16, low=low, high=high, idx=idx, scale=scale, zero=zero)
    return low, high, idx, scale, zero


@pytest.mark.gpu
@pytest.mark.parametrize("selection", ["magnitude", "variance"])
@pytest.mark.parametrize("kind", ["outliers", "coarse", "distinct", "flat", "mixed"])
def test_many_page_launch_equals_pages_one_by_one(kind, selection):
    pages = 20
    keys = _keys(kind, 2, 8, pages * 128).to(DEV)  # 320 page items: the three-pass path
    many = _pack(keys, selection, pages)
    for p in range(pages):  # 16 page items each: the single-pass kernel
        one = _pack(keys[:, :, p * 128:(p + 1) * 128].contiguous(), selection, 1)
        for name, m, o in zip(("low", "high", "idx", "scale", "zero"), many, one):
            assert bits_equal(m[p], o[0]), (kind, selection, p, name)


@pytest.mark.gpu
@pytest.mark.parametrize("selection", ["magnitude", "variance"])
def test_many_page_launch_matches_the_oracle(selection):
    from oracle import dart_oracle as orc
    keys = _keys("mixed", 1, 4, 80 * 128)  # 320 page items
    low, high, idx, scale, zero = _pack(keys.to(DEV), selection, 80)
    for p in (0, 1, 2, 37, 79):
        ref = orc.quantize_key_mixed(keys[:, :, p * 128:(p + 1) * 128], group_size=128, promote_ratio=0.25,
                                     strategy=selection, metadata_dtype=torch.float16)
        assert bits_equal(idx[p].cpu(), ref.channel_indices.to(torch.int32)), p
        assert bits_equal(low[p].cpu(), ref.low_values), p
        assert bits_equal(high[p].cpu(), ref.high_values), p
        assert bits_equal(scale[p].cpu(), ref.scale), p
        assert bits_equal(zero[p].cpu(), ref.zero_point), p

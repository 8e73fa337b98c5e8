"""dkv_copy_token_blocks: the dense token copies of an append (held tail, sink) in one launch.

GPU: every block lands byte for byte, bytes outside the destination rows stay as they were, and the
unit width follows the alignment (16-byte rows, and rows whose addresses only allow 2 or 4 bytes).
"""

from __future__ import annotations

import pytest
import torch

from dartkv_amd import _lib

DEV = "cuda"


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_blocks_copy_exactly_and_touch_nothing_else(dtype):
    g = torch.Generator(device="cpu").manual_seed(5)
    pairs, expect = [], []
    # (B, H, T, D, source token offset, destination token offset, destination capacity)
    shapes = [(2, 3, 5, 128, 0, 0, 8), (1, 8, 96, 128, 32, 4, 160), (3, 2, 7, 33, 1, 3, 11), (2, 2, 1, 5, 2, 0, 1),
              (4, 1, 3, 64, 0, 5, 9)]
    for B, H, T, D, s0, d0, cap in shapes:
        src_full = torch.randn(B, H, T + s0 + 2, D, generator=g).to(dtype).to(DEV)
        dst_full = torch.randn(B, H, cap + d0, D, generator=g).to(dtype).to(DEV)
        src = src_full[:, :, s0:s0 + T]
        dst = dst_full[:, :, d0:d0 + T]
        want = dst_full.clone()
        want[:, :, d0:d0 + T] = src
        pairs.append((dst, src))
        expect.append((dst_full, want))
    _lib.copy_token_blocks(pairs, torch.device(DEV))
    torch.cuda.synchronize()
    for got, want in expect:
        assert torch.equal(got, want)


@pytest.mark.gpu
def test_more_pairs_than_one_launch_and_empty_blocks():
    g = torch.Generator(device="cpu").manual_seed(6)
    pairs, want = [], []
    for i in range(11):
        T = 0 if i == 4 else i + 1
        src = torch.randn(2, 2, T, 16, generator=g).to(torch.bfloat16).to(DEV)
        dst = torch.zeros(2, 2, T, 16, dtype=torch.bfloat16, device=DEV)
        pairs.append((dst, src))
        want.append(src)
    _lib.copy_token_blocks(pairs, torch.device(DEV))
    torch.cuda.synchronize()
    for (dst, _), src in zip(pairs, want):
        assert torch.equal(dst, src)


def test_rejects_mismatched_pairs():
    a = torch.zeros(1, 1, 2, 4)
    with pytest.raises(ValueError, match="one shape and dtype"):
        _lib.copy_token_blocks([(a, torch.zeros(1, 1, 3, 4))], torch.device("cpu"))
    with pytest.raises(ValueError, match="contiguous"):
        _lib.copy_token_blocks([(a, torch.zeros(1, 1, 4, 2).transpose(2, 3))], torch.device("cpu"))

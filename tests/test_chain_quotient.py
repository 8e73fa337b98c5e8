"""The quantizers' quotient step for bf16 and fp16 sources (quantize.hip, chain_quotients4): one product
with RN(1 / s) gives the same codes as the reference's IEEE division, for every 16-bit pair in range
(exhaustive host check, tests/quotient/chain_quotient.c), and on the device for group scales of every
bf16 mantissa."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
CLANG = shutil.which("clang", path="/opt/rocm/llvm/bin") or shutil.which("clang")


@pytest.mark.skipif(CLANG is None, reason="needs clang (for _Float16 on the host)")
def test_product_quotient_gives_the_division_codes(tmp_path):
    exe = tmp_path / "chain_quotient"
    subprocess.run([CLANG, "-O2", "-ffp-contract=off", "-pthread", os.path.join(HERE, "quotient", "chain_quotient.c"),
                    "-o", str(exe), "-lm"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout
    lines = out.stdout.split()
    assert lines.count("ok") == 2, out.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_rows_over_every_scale_mantissa_match_the_oracle(bits):
    """The device side of the same step: one 64-element group per row with min 0 and max every bf16 value
    in [2^-4, 2^8) (12 binades), so the group scales take every bf16 mantissa over several binades; codes,
    scales and zero points equal the oracle's."""
    import dartkv_amd as dart
    from oracle import dart_oracle as orc
    from tests.golden_util import bits_equal
    g = torch.Generator().manual_seed(bits)
    top = (torch.arange(0x3D80, 0x4380, dtype=torch.int32) << 16).view(torch.float32)
    x = (torch.rand(top.numel(), 64, generator=g) * top[:, None]).to(torch.bfloat16)
    x[:, 0] = 0.0
    x[:, 1] = top.to(torch.bfloat16)
    got = dart.quantize(x.to("cuda"), bits=bits, group_size=64, metadata_dtype=torch.bfloat16)
    ref = orc.quantize(x, bits=bits, group_size=64, metadata_dtype=torch.bfloat16)
    assert bits_equal(got.values.cpu(), ref.values)
    assert bits_equal(got.scale.cpu(), ref.scale)
    assert bits_equal(got.zero_point.cpu(), ref.zero_point)

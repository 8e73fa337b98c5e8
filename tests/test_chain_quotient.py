"""The quantizers' quotient step for bf16 and fp16 sources (quantize.hip, chain_quotients4): one product
with RN(1 / s) gives the same codes as the reference's IEEE division, for every 16-bit pair in range
(exhaustive host check, tests/quotient/chain_quotient.c)."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

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

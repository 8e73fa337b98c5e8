"""The quantize kernels divide with a reciprocal and one fma correction (div_rn in
dartkv_amd/csrc/quantize.hip) where the reference divides (reference
src/dart/quantization.py: ``(x - zero) / scale`` and ``range / qmax``).  These host
checks run the same float arithmetic in C over whole input domains:

* the group scale's range / qmax equals the IEEE quotient for every positive finite
  fp32 range and qmax 3, 15 and 255;
* the per-element diff / scale, for every pair of 16-bit values the kernels can see
  (a scale is at least eps / 255 = 3.9e-7 > 2^-22 for bf16 and fp16 sources), equals
  the IEEE quotient for fp16, and for bf16 everywhere except quotients below 2^-90
  (subnormal dividends), whose codes are 0 either way.  fp32 sources rest on
  Markstein's theorem (the checks above found no normal-range counterexample).
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "divide", "div_check.c")


@pytest.fixture(scope="module")
def div_check(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc is not available")
    exe = str(tmp_path_factory.mktemp("divide") / "div_check")
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", SRC, "-o", exe, "-lm"], check=True)
    return exe


def _run(exe, *args):
    env = dict(os.environ, OMP_NUM_THREADS=str(min(8, os.cpu_count() or 1)))
    out = subprocess.run([exe, *args], check=True, capture_output=True, text=True, env=env, timeout=600)
    return out.stdout.split()


@pytest.mark.parametrize("qmax", [3, 15, 255])
def test_range_over_qmax_is_the_ieee_quotient_for_every_fp32(div_check, qmax):
    assert _run(div_check, "qmax", str(qmax)) == ["0"]


def test_fp16_element_quotients_are_the_ieee_quotient(div_check):
    assert _run(div_check, "pairs", "f16")[0] == "0"


def test_bf16_element_quotients_differ_only_far_below_one_half(div_check):
    bad, worst = _run(div_check, "pairs", "bf16")
    assert int(bad) > 0  # subnormal dividends: the reciprocal form is not exact there
    assert float.fromhex(worst) < 2.0 ** -90

"""The channel selection restated in dartkv_amd/csrc/dkv_select.h equals libstdc++'s (CPU).

torch.topk(sorted=True) on CPU orders tied scores the way libstdc++'s
nth_element / sort / partial_sort leave them (reference src/dart/mixed.py:155-161
selects promoted channels with it), so the HIP selection restates those
algorithms.  A host build of the same header is run against std:: on random
scores with many ties, for both item forms the GPU uses, and a host model of the
wave-parallel form (dkv_select_wave.h) likewise.  The GPU kernels are
checked end to end by the golden tie-order vectors (test_gpu_parity.py).
"""

from __future__ import annotations

import os
import subprocess

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _build(tmp_path):
    exe = tmp_path / "select_harness"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", os.path.join(REPO, "dartkv_amd", "csrc"),
                    os.path.join(REPO, "tests", "select", "select_harness.cpp"), "-o", str(exe)], check=True)
    return str(exe)


def test_selection_matches_libstdcxx(tmp_path):
    out = subprocess.run([_build(tmp_path), "20000"], capture_output=True, text=True)
    print(out.stdout.strip())
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches 0" in out.stdout


def test_selection_matches_torch_topk_on_ties(tmp_path):
    """Both item forms give torch.topk(sorted=True)'s indices, tie order included."""
    import torch
    g = torch.Generator().manual_seed(5)
    cases = []
    for _ in range(300):
        n = int(torch.randint(1, 129, (1,), generator=g))
        k = int(torch.randint(1, n + 1, (1,), generator=g))
        levels = int(torch.randint(1, 12, (1,), generator=g))
        s = torch.randint(0, levels, (n,), generator=g).float() * 0.25
        if n > 4 and int(torch.randint(0, 6, (1,), generator=g)) == 0:
            s[int(torch.randint(0, n, (1,), generator=g))] = float("nan")
        cases.append((n, k, s))
    text = "".join(f"{n} {k} " + " ".join(repr(float(v)) for v in s.tolist()) + "\n" for n, k, s in cases)
    out = subprocess.run([_build(tmp_path), "stdin"], input=text, capture_output=True, text=True, check=True)
    lines = out.stdout.strip().split("\n")
    assert len(lines) == 2 * len(cases)
    for c, (n, k, s) in enumerate(cases):
        want = torch.topk(s, k, sorted=True).indices.tolist()
        assert [int(x) for x in lines[2 * c].split()] == want, (n, k)
        assert [int(x) for x in lines[2 * c + 1].split()] == want, (n, k)


def test_wave_selection_matches_libstdcxx(tmp_path):
    """The wave-parallel form (dartkv_amd/csrc/dkv_select_wave.h), its 64 lanes run in a loop on the host,
    gives the first k items of std::nth_element + std::sort for random tied scores, NaN and presorted runs
    included; where libstdc++ would take partial_sort or heap select it hands back (counted, not compared)."""
    exe = tmp_path / "select_wave"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", os.path.join(REPO, "dartkv_amd", "csrc"),
                    os.path.join(REPO, "tests", "select", "select_wave.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe), "30000"], capture_output=True, text=True)
    print(out.stdout.strip())
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches 0" in out.stdout
    fallbacks = int(out.stdout.split("fallbacks")[1])
    assert fallbacks < 30000 // 20  # the parallel form covers nearly every case (k * 64 > n)

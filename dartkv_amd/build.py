"""Build libdartkv_hip.so (HIP kernels + C ABI) for gfx950, in-tree.

    python -m dartkv_amd.build

Sources are compiled together by one hipcc invocation.  Flags:
* ``-ffp-contract=off``: the quantizer and the dequantization chain must
  round after every multiply and add, like the reference's separate torch ops;
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed-fp32 VALU ops.
"""

from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libdartkv_hip.so")
SOURCES = ["capi.hip", "quantize.hip", "decode.hip", "decode_fast.hip", "decode_uniform.hip", "prep.hip"]
ARCH = os.environ.get("DKV_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    raise RuntimeError("hipcc not found")


def command(output: str = LIB) -> list[str]:
    return [
        hipcc(), "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-shared",
        "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        "-I", os.path.join(os.path.dirname(PKG), "include"),
        *[os.path.join(CSRC, s) for s in SOURCES],
        "-o", output,
    ]


def build(verbose: bool = False) -> str:
    tmp = LIB + ".tmp"
    cmd = command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with exit code {proc.returncode}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))

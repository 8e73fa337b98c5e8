"""Build libdartkv_hip.so (HIP kernels + C ABI) for gfx950, in-tree.

    python -m dartkv_amd.build

Each source is compiled to an object by its own hipcc process (in parallel),
then the objects are linked into the shared library.  Flags:
* ``-ffp-contract=off``: the quantizer and the dequantization chain must
  round after every multiply and add, like the reference's separate torch ops;
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed-fp32 VALU ops.
"""

from __future__ import annotations

import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libdartkv_hip.so")
SOURCES = ["capi.hip", "quantize.hip", "decode.hip", "decode_fast.hip", "decode_uniform.hip", "prep.hip", "copy.hip"]
ARCH = os.environ.get("DKV_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    raise RuntimeError("hipcc not found")


def compile_flags() -> list[str]:
    return [
        "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC",
        "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        "-I", os.path.join(os.path.dirname(PKG), "include"),
    ]


def command(output: str = LIB) -> list[str]:
    """One hipcc line that compiles and links every source (the serial form of build())."""
    return [hipcc(), *compile_flags(), "-shared", *[os.path.join(CSRC, s) for s in SOURCES], "-o", output]


# Sources whose kernels must keep every value in registers: a spill to scratch
# (private memory in HBM) would add memory traffic to the page kernels' loops.
NO_SCRATCH = {"decode_fast.hip", "decode_uniform.hip"}


def _run(cmd: list[str], verbose: bool) -> str:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with exit code {proc.returncode}: {' '.join(cmd[-3:])}")
    return proc.stderr


def scratch_kernels(remarks: str) -> list[str]:
    """Kernels with a non-zero ScratchSize in hipcc's -Rpass-analysis=kernel-resource-usage remarks."""
    out, name = [], None
    for line in remarks.splitlines():
        if "Function Name:" in line:
            name = line.split("Function Name:", 1)[1].split("[")[0].strip()
        elif "ScratchSize [bytes/lane]:" in line and name is not None:
            if int(line.split("ScratchSize [bytes/lane]:", 1)[1].split("[")[0]) > 0:
                out.append(name)
    return out


def build(verbose: bool = False, jobs: int = 0) -> str:
    jobs = jobs or min(len(SOURCES), max(1, min(8, len(os.sched_getaffinity(0)))))
    with tempfile.TemporaryDirectory(prefix="dkv_build_") as tmpdir:
        objs = [os.path.join(tmpdir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
        cmds = [[hipcc(), *compile_flags(), *(["-Rpass-analysis=kernel-resource-usage"] if s in NO_SCRATCH else []),
                 "-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(SOURCES, objs)]
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            for src, fut in zip(SOURCES, [pool.submit(_run, c, verbose) for c in cmds]):
                spilled = scratch_kernels(fut.result()) if src in NO_SCRATCH else []
                if spilled:
                    raise RuntimeError(f"{src}: kernels use scratch memory: {spilled[:3]}")
        tmp = LIB + ".tmp"
        _run([hipcc(), f"--offload-arch={ARCH}", "-fPIC", "-shared", *objs, "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))

"""Loader for the golden vectors written by tests/golden/make_golden.py."""

from __future__ import annotations

import hashlib
import json
import os

import torch
from safetensors.torch import load_file

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN_DIR = os.path.join(HERE, "golden")

DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32,
          "float64": torch.float64, None: None}


def sha256(t: torch.Tensor) -> str:
    t = t.detach().cpu().contiguous()
    raw = t.view(torch.uint8) if t.dtype != torch.bool else t.to(torch.uint8)
    return hashlib.sha256(raw.numpy().tobytes()).hexdigest()


def bits_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Exact equality including float bit patterns (NaN-safe, -0 distinct)."""
    a = a.detach().cpu().contiguous()
    b = b.detach().cpu().contiguous()
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    if a.numel() == 0:
        return True
    return torch.equal(a.view(torch.uint8), b.view(torch.uint8))


class Golden:
    def __init__(self) -> None:
        with open(os.path.join(GOLDEN_DIR, "golden.json")) as fh:
            self.manifest = json.load(fh)
        self.tensors = load_file(os.path.join(GOLDEN_DIR, "golden.safetensors"))
        self.digests = self.manifest["digests"]

    def get(self, ref: str):
        """Tensor for a stored name; None for a digest-only entry."""
        if ref.startswith("sha:"):
            return None
        return self.tensors[ref]

    def matches(self, ref: str, actual: torch.Tensor) -> bool:
        """Bit-exact comparison against a stored tensor or a stored digest."""
        if ref.startswith("sha:"):
            d = self.digests[ref[4:]]
            actual = actual.detach().cpu().contiguous()
            return (list(actual.shape) == d["shape"] and str(actual.dtype).replace("torch.", "") == d["dtype"]
                    and sha256(actual) == d["sha256"])
        return bits_equal(self.tensors[ref], actual)

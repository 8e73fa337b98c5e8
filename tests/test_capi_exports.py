"""The C-ABI library builds, loads without a GPU and exports every declared symbol (CPU)."""

from __future__ import annotations

import os
import re
import subprocess

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "dartkv.h")
LIB = os.path.join(REPO, "dartkv_amd", "libdartkv_hip.so")


def declared_functions() -> set:
    text = open(HEADER).read()
    return set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]*?\b(dkv_\w+)\s*\(", text, flags=re.M))


def test_header_declares_the_entry_points():
    names = declared_functions()
    assert {"dkv_quantize_rows", "dkv_quantize_row_blocks", "dkv_quantize_key_pages", "dkv_dequantize_rows", "dkv_dequantize_mixed",
            "dkv_decode_attention", "dkv_decode_workspace_bytes", "dkv_last_error", "dkv_abi_version"} <= names


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "build the library first: python -m dartkv_amd.build"
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (dkv_\w+)", out))
    missing = declared_functions() - exported
    assert not missing, missing


def test_library_loads_and_reports_errors_without_gpu():
    from dartkv_amd import _lib
    lib = _lib.load()
    assert lib.dkv_abi_version() == _lib.ABI_VERSION
    # argument validation runs on the host before any launch
    rc = lib.dkv_quantize_rows(None, 0, 1, 4, 4, 1, 3, 4, None, None, None, 0, None)
    assert rc == _lib.DKV_ERR_INVALID
    assert b"bits" in lib.dkv_last_error()
    rc = lib.dkv_quantize_row_blocks(None, 0, 2, 64, -1, 4, 4, 2, 4, None, None, None, 0, None)
    assert rc == _lib.DKV_ERR_INVALID
    assert b"non-negative" in lib.dkv_last_error()
    assert lib.dkv_decode_workspace_bytes(2, 4, 8, 3) == 2 * 4 * 3 * 10 * 4
    assert lib.dkv_copy_token_blocks(None, 9, None) == _lib.DKV_ERR_INVALID
    assert b"n_blocks" in lib.dkv_last_error()
    assert lib.dkv_copy_token_blocks(None, 0, None) == _lib.DKV_OK  # nothing to copy, nothing launched
    blk = (_lib.CopyBlock * 1)()
    blk[0].B, blk[0].H, blk[0].T, blk[0].row_bytes = 1, 1, 4, 256
    assert lib.dkv_copy_token_blocks(blk, 1, None) == _lib.DKV_ERR_INVALID
    assert b"NULL" in lib.dkv_last_error()


def test_ctypes_structs_match_the_header(tmp_path):
    """Field offsets and sizes of the ctypes mirrors equal the C compiler's."""
    import ctypes
    from dartkv_amd import _lib
    structs = {"dkv_segment": _lib.Segment, "dkv_decode_args": _lib.DecodeArgs,
               "dkv_key_pages_args": _lib.KeyPagesArgs, "dkv_value_rows_args": _lib.ValueRowsArgs,
               "dkv_copy_block": _lib.CopyBlock}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "dartkv.h"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'  printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    got = {tuple(l.split()[:2]): int(l.split()[2]) for l in out if l.strip()}
    for cname, cls in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(cls), cname
        for field, _ in cls._fields_:
            assert got[(cname, field)] == getattr(cls, field).offset, (cname, field)


def test_build_rejects_page_kernels_that_use_scratch():
    """The build reads hipcc's kernel-resource-usage remarks for the page-kernel sources and fails when a
    kernel spills to scratch memory (private memory in HBM), which would add traffic to the page loops."""
    from dartkv_amd import build as B
    remarks = "\n".join([
        "a.hip:1:1: remark: Function Name: _Z6spillsv [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:1:1: remark:     VGPRs: 168 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:1:1: remark:     ScratchSize [bytes/lane]: 8 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:1:1: remark: Function Name: _Z5cleanv [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert B.scratch_kernels(remarks) == ["_Z6spillsv"]
    assert B.scratch_kernels("") == []
    assert {"decode_fast.hip", "decode_uniform.hip"} <= B.NO_SCRATCH <= set(B.SOURCES)

"""CPU check of the built library's gfx950 code objects: no kernel uses
private (scratch) memory.  A kernel with a private segment makes every
dispatch set up scratch and turns its spilled values into memory round
trips; the reference-API restricted head once picked up 96 bytes per lane
that way (its kernel argument struct copied to scratch because a helper
holding a reference to it was not inlined), which doubled its latency at
one row.  Reads only this build's own library."""
import os
import re
import shutil
import struct
import subprocess

import pytest

from market_sim_amd import abi

LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _tool(name):
    path = os.path.join(LLVM, name)
    return path if os.path.exists(path) else shutil.which(name)


def _fatbin_section(lib_path, tmp_path):
    out = tmp_path / "fatbin.bin"
    subprocess.run([_tool("llvm-objcopy"), f"--dump-section=.hip_fatbin={out}", lib_path,
                    str(tmp_path / "stripped.so")], check=True)
    return out.read_bytes()


def _gfx950_code_objects(blob):
    """Every gfx950 entry of the offload bundles concatenated in the section
    (one bundle per translation unit).  Bundle header: magic, entry count
    (u64), then per entry offset, size, triple length (u64 each) and the
    triple; offsets are relative to the bundle's start."""
    objects = []
    start = blob.find(MAGIC)
    while start >= 0:
        pos = start + len(MAGIC)
        (entries,) = struct.unpack_from("<Q", blob, pos)
        pos += 8
        for _ in range(entries):
            offset, size, tlen = struct.unpack_from("<QQQ", blob, pos)
            pos += 24
            triple = blob[pos:pos + tlen].decode()
            pos += tlen
            if triple.endswith("gfx950") and size > 0:
                objects.append(blob[start + offset:start + offset + size])
        start = blob.find(MAGIC, pos)
    return objects


@pytest.mark.skipif(_tool("llvm-objcopy") is None or _tool("llvm-readelf") is None,
                    reason="LLVM binutils not installed")
def test_no_kernel_uses_scratch(tmp_path):
    lib_path = abi.lib()._name
    objects = _gfx950_code_objects(_fatbin_section(lib_path, tmp_path))
    assert objects, "no gfx950 code object in the library"
    kernels = {}
    for i, co in enumerate(objects):
        elf = tmp_path / f"co{i}.elf"
        elf.write_bytes(co)
        notes = subprocess.run([_tool("llvm-readelf"), "--notes", str(elf)], check=True,
                               capture_output=True, text=True).stdout
        names = re.findall(r"^\s+\.name:\s+(\S+)$", notes, re.M)
        private = re.findall(r"\.private_segment_fixed_size:\s+(\d+)", notes)
        assert len(names) == len(private), (len(names), len(private))
        kernels.update(zip(names, map(int, private)))
    # every translation unit with kernels contributes (head, pass, dense, ...)
    assert any("head_kernel" in k for k in kernels)
    assert any("pass_kernel" in k for k in kernels)
    assert any("dense_kernel" in k for k in kernels)
    assert any("projection_kernel" in k for k in kernels)
    with_scratch = {k: v for k, v in kernels.items() if v != 0}
    assert not with_scratch, with_scratch

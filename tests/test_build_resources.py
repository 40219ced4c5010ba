"""Resource check of every kernel instance in the built library (CPU).

libvpa.so carries one clang offload bundle per HIP source in its
.hip_fatbin section; each holds the gfx950 code object. The kernel
descriptors' metadata (llvm-readelf --notes) must show no private (scratch)
segment and no register spills for any instance: a spill or a scratch array
costs a VMEM round trip inside the hot loops, and its s_waitcnt vmcnt(0)
would also drain the LDS-DMA loads the prefill keeps in flight."""

import os
import re
import shutil
import struct
import subprocess

import pytest

from vpa import _lib

LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _tool(name):
    path = os.path.join(LLVM, name)
    return path if os.path.exists(path) else shutil.which(name)


def code_objects(fatbin: bytes):
    """gfx950 code objects of every bundle in a .hip_fatbin section."""
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), fatbin)]
    for s in starts:
        pos = s + len(MAGIC)
        (n,) = struct.unpack_from("<Q", fatbin, pos)
        pos += 8
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", fatbin, pos)
            pos += 24
            triple = fatbin[pos:pos + tlen].decode()
            pos += tlen
            if "gfx950" in triple and size:
                yield fatbin[s + off:s + off + size]


def kernel_resources(tmp_path):
    objcopy, readelf = _tool("llvm-objcopy"), _tool("llvm-readelf")
    if not (objcopy and readelf):
        pytest.skip("llvm-objcopy / llvm-readelf not found")
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libvpa.so not built")
    fb = tmp_path / "fatbin.bin"
    subprocess.run([objcopy, f"--dump-section=.hip_fatbin={fb}", _lib.LIB_PATH, os.devnull],
                   check=True, capture_output=True)
    kernels = {}
    for i, co in enumerate(code_objects(fb.read_bytes())):
        path = tmp_path / f"co{i}.o"
        path.write_bytes(co)
        notes = subprocess.run([readelf, "--notes", str(path)], check=True, capture_output=True,
                               text=True).stdout
        # one metadata map per kernel: .name and its resource fields
        for block in notes.split("  - .agpr_count:")[1:]:
            name = re.search(r"\n\s+\.name:\s+(\S+)", block).group(1)
            fields = {k: int(v) for k, v in re.findall(
                r"\.(private_segment_fixed_size|vgpr_spill_count|sgpr_spill_count):\s+(\d+)",
                block)}
            kernels[name] = fields
    return kernels


def test_no_kernel_spills_or_uses_scratch(tmp_path):
    kernels = kernel_resources(tmp_path)
    assert len(kernels) > 500, f"expected every source's kernels, found {len(kernels)}"
    bad = {k: v for k, v in kernels.items() if any(v.get(f, 0) for f in (
        "private_segment_fixed_size", "vgpr_spill_count", "sgpr_spill_count"))}
    assert not bad, f"{len(bad)} kernels spill or use scratch: " + ", ".join(
        f"{k} {v}" for k, v in list(bad.items())[:5])

"""The gfx950 code object of the built library: no kernel uses scratch memory.

Scratch (private segment) accesses are vector memory operations that count in
the same in-order counter as the prefetched loads, so a spill or a kernel
argument block copied to scratch (what happens when a large device function
is not inlined and its argument struct's address is taken) makes every wait
drain everything and can double a kernel's time with no change in its
results. The metadata of every kernel in the embedded code object must
therefore report a zero private segment and no VGPR spills.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

LLVM = Path("/opt/rocm/llvm/bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def _tool(name):
    path = LLVM / name
    if path.exists():
        return str(path)
    found = shutil.which(name)
    if not found:
        pytest.skip(f"{name} not available")
    return found


def _kernel_metadata(library: Path, work: Path) -> dict:
    fatbin, code = work / "fatbin.bin", work / "gfx950.co"
    subprocess.run([_tool("llvm-objcopy"), f"--dump-section=.hip_fatbin={fatbin}", str(library),
                    str(work / "copy.so")], check=True, capture_output=True)
    subprocess.run([_tool("clang-offload-bundler"), "--unbundle", "--type=o", f"--input={fatbin}",
                    f"--targets={TARGET}", f"--output={code}"], check=True, capture_output=True)
    notes = subprocess.run([_tool("llvm-readelf"), "--notes", str(code)], check=True,
                           capture_output=True, text=True).stdout
    kernels = {}
    for block in notes.split(".name:")[1:]:
        name = block.split()[0]
        fields = dict(re.findall(r"\.(private_segment_fixed_size|vgpr_spill_count|sgpr_count):\s+(\d+)", block))
        if "private_segment_fixed_size" in fields:
            kernels[name] = {k: int(v) for k, v in fields.items()}
    return kernels


def test_no_kernel_uses_scratch(built_library, tmp_path):
    kernels = _kernel_metadata(Path(built_library), tmp_path)
    names = " ".join(kernels)
    for expected in ("map_install_stream_kernel", "map_install_support_kernel", "map_install_gen_kernel",
                     "map_install_any_kernel", "copy_rows_kernel", "delta_state128_kernel"):
        assert expected in names, expected
    offenders = {n: m for n, m in kernels.items()
                 if m["private_segment_fixed_size"] != 0 or m.get("vgpr_spill_count", 0) != 0}
    assert not offenders, offenders

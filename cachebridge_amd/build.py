"""Build ``libcachebridge_hip.so`` in-tree with hipcc for gfx950.

    python -m cachebridge_amd.build
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
SOURCES = [PACKAGE / "csrc" / "cb_handoff.hip"]
OUTPUT = PACKAGE / "libcachebridge_hip.so"
ARCH = os.environ.get("CACHEBRIDGE_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Keep the compiler from emitting packed fp32 VALU ops on this target.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found")


def build_library(verbose: bool = False) -> Path:
    """Compile every HIP source into the package's shared library."""
    tmp = OUTPUT.with_suffix(".so.tmp")
    cmd = [hipcc(), *FLAGS, *map(str, SOURCES), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if verbose or result.returncode:
        sys.stderr.write(result.stdout + result.stderr)
    if result.returncode:
        raise RuntimeError(f"hipcc failed ({result.returncode}): {' '.join(cmd)}")
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))

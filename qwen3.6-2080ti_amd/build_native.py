"""Build the gfx950 hot-path library ``build/libqwen36_hip.so`` with hipcc.

Replaces the reference's ``setup.py`` ``CUDAExtension`` build (``setup.py:12-41``):
plain ``hipcc --offload-arch=gfx950`` compiles of ``csrc/*.hip`` and
``csrc/*.cpp`` into position-independent objects, linked into one shared
library with a C ABI (``include/qwen36_hip.h``).  No torch headers, no pybind.

Usage: ``python build_native.py`` (from any directory).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC = PACKAGE_DIR / "csrc"
BUILD = PACKAGE_DIR / "build"
LIBRARY = BUILD / "libqwen36_hip.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-unused-result",
    # Packed FP32 VALU forms are kept out of every device object.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found")


def _compile(hipcc: str, source: Path) -> Path:
    obj = BUILD / (source.stem + ".o")
    cmd = [hipcc, *COMMON_FLAGS, "-c", str(source), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{stderr}")
    if stderr.strip():
        print(stderr, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    hipcc = _hipcc()
    BUILD.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objects = list(pool.map(lambda src: _compile(hipcc, src), sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(sources)} sources")
    return LIBRARY


if __name__ == "__main__":
    build()

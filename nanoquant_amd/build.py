"""Build recipe for the gfx950 HIP library ``nanoquant_amd/_lib/libnqamd.so``.

Every ``csrc/*.hip`` is compiled with hipcc for gfx950 only and linked into one
shared library that exports the C ABI declared in ``include/nqamd.h``.

Usage: ``python -m nanoquant_amd.build`` (or ``build_library()`` from Python).
"""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE_DIR / "csrc"
LIB_DIR = PACKAGE_DIR / "_lib"
LIBRARY_PATH = LIB_DIR / "libnqamd.so"
INCLUDE_DIR = PACKAGE_DIR.parent / "include"

OFFLOAD_ARCH = "gfx950"
# Packed fp32 VALU ops stay disabled in every device compile.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE_DIR}",
]


def hipcc() -> str:
    candidates = [os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"]
    for candidate in candidates:
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the HIP library cannot be built")


def _compile(source: Path, obj: Path) -> None:
    cmd = [hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stderr}")


def build_library(*, jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile all sources and link the shared library; returns its path."""

    sources = sorted(SOURCE_DIR.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {SOURCE_DIR}")
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    objects = [obj_dir / (src.stem + ".o") for src in sources]
    workers = jobs or min(len(sources), 8)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(_compile, sources, objects))
    tmp = LIBRARY_PATH.with_name(LIBRARY_PATH.name + ".tmp")
    cmd = [hipcc(), f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objects),
           "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(tmp, LIBRARY_PATH)
    if verbose:
        print(f"built {LIBRARY_PATH}")
    return LIBRARY_PATH


if __name__ == "__main__":
    build_library(verbose=True)

"""Build the in-tree HIP library ``longspark_amd/liblongspark_amd.so`` for gfx950.

Each ``csrc/*.hip`` / ``csrc/*.cpp`` source is compiled by ``hipcc`` into an
object under ``longspark_amd/_build/`` (in parallel), then linked into one
shared library.  The library exports only the ``extern "C"`` entry points
declared in ``include/longspark_amd.h``.

Usage: ``python -m longspark_amd.build`` or ``longspark_amd.build.build_library()``.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = PKG / "_build"
LIB = PKG / "liblongspark_amd.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]
# Device code: gfx950 only; packed-fp32 instructions are kept out of the
# generated code.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _sources():
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [HIPCC, *COMMON_FLAGS]
    if src.suffix == ".hip":
        cmd += ["-x", "hip", *DEVICE_FLAGS]
    else:
        cmd += ["-x", "c++"]
    cmd += ["-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj


def build_library(verbose: bool = True) -> Path:
    """Compile every HIP/C++ source and link ``liblongspark_amd.so``; always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    sources = _sources()
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build_library()

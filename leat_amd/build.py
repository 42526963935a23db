"""Builds libleatmi.so, the gfx950 HIP kernels behind the C ABI of include/leatmi.h, in-tree.

    python -m leat_amd.build        # or leat_amd.build.build()

Each .hip source compiles to an object in parallel, then hipcc links the shared library. Packed
f32 instructions are disabled (-packed-fp32-ops): hipcc -O3 would otherwise form them itself.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
LIB = HERE / "libleatmi.so"
OBJ = HERE / "_obj"
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(CSRC),
    "-I", str(INCLUDE),
]  # fmt: skip


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the HIP toolchain is needed to build libleatmi.so")
    return path


def _compile(src: Path) -> Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [hipcc(), *FLAGS, "-c", str(src), "-o", str(obj)]
    done = subprocess.run(cmd, capture_output=True, text=True)
    if done.returncode != 0:
        raise RuntimeError(f"compiling {src.name} failed:\n{done.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compiles every kernel source for gfx950 and links libleatmi.so; returns its path."""
    OBJ.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    done = subprocess.run(cmd, capture_output=True, text=True)
    if done.returncode != 0:
        raise RuntimeError(f"linking libleatmi.so failed:\n{done.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True)

"""Build libenilnets_amd.so from the HIP sources in this directory.

    python -m enilnets_amd.csrc.build          # or: python enilnets_amd/csrc/build.py

Every ``*.hip`` file here is compiled for gfx950 only, in parallel, and the
objects are linked into ``enilnets_amd/libenilnets_amd.so`` (in-tree, so the
library travels with the source tree).  No CUDA, no second target.
"""

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
PACKAGE = HERE.parent
REPO = PACKAGE.parent
INCLUDE = REPO / "include"
OUT = PACKAGE / "libenilnets_amd.so"
BUILD_DIR = HERE / "_build"

ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # Packed fp32 arithmetic is kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{HERE}",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = shutil.which("hipcc") or os.path.join(rocm, "bin", "hipcc")
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; a ROCm toolchain is required to build")
    return path


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    warnings = [l for l in proc.stderr.splitlines()
                if "warning" in l and "packed-fp32-ops" not in l and "target-feature" not in l]
    if warnings:
        sys.stderr.write("\n".join(warnings) + "\n")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(HERE.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {HERE}")
    workers = min(len(sources), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(sources)} sources")
    return OUT


if __name__ == "__main__":
    build()

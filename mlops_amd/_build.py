"""Compile the HIP sources of ``mlops_amd/csrc`` into ``libmlops_mi355x.so``.

The library is built in-tree for gfx950 only, with hipcc, one object per
source (in parallel) and a shared link. Packed-fp32 instructions are disabled
(``-packed-fp32-ops``): the compiler otherwise forms them from ordinary float
code and some of their forms are unreliable on this hardware.
"""

from __future__ import annotations

import concurrent.futures
import os
import subprocess
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
SOURCES = PACKAGE / "csrc"
INCLUDE = PACKAGE.parent / "include"
LIBRARY = PACKAGE / "libmlops_mi355x.so"
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: the block-scale fold reads every result with VALU
    # FMAs, which would otherwise copy each one out of the AGPRs first.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-result",
]


def _hipcc() -> str:
    root = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(root) / "bin" / "hipcc")


def _compile(source: Path, obj: Path) -> None:
    cmd = [_hipcc(), *FLAGS, f"-I{INCLUDE}", "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name}:\n{result.stderr}")


def build(verbose: bool = False) -> Path:
    """Compile every ``csrc/*.hip`` and link the shared library; returns its path."""
    objdir = PACKAGE / "_build"
    objdir.mkdir(exist_ok=True)
    sources = sorted(SOURCES.glob("*.hip"))
    objects = [objdir / (s.stem + ".o") for s in sources]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        list(pool.map(_compile, sources, objects))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)

"""Builds the gfx950 HIP rasterizer library in-tree.

Every ``csrc/*.hip`` file is compiled with ``hipcc --offload-arch=gfx950`` to an
object and linked into ``gaussian_splats/_lib/libgs_raster.so``, the C-ABI
library declared by ``include/gs_raster.h``.  Run ``python build.py`` or call
:func:`build`.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_ROOT.parent
CSRC = PACKAGE_ROOT / "csrc"
INCLUDE = REPO_ROOT / "include"
BUILD_DIR = PACKAGE_ROOT / "_build"
LIB_DIR = PACKAGE_ROOT / "gaussian_splats_hip" / "_lib"
LIB_PATH = LIB_DIR / "libgs_raster.so"

ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # Packed FP32 instructions are disabled for all device code.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]

# The projection computes tile rectangles as floor((u -/+ r) / tile); contracting
# u - extent * sqrt(cov) into an FMA would change which tile a boundary
# Gaussian lands in relative to the CPU restatement.
PER_FILE_FLAGS = {
    "project_fwd.hip": ["-ffp-contract=off"],
}


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the HIP rasterizer cannot be built")
    return path


def _compile(source: Path, obj: Path) -> None:
    cmd = [_hipcc(), *COMMON_FLAGS, *PER_FILE_FLAGS.get(source.name, []), "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stdout}\n{result.stderr}")


def build(verbose: bool = False) -> Path:
    """Compiles every HIP source and links the shared library; returns its path."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objects = [BUILD_DIR / (s.stem + ".o") for s in sources]
    workers = min(len(sources), max(1, (os.cpu_count() or 2) // 2))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        futures = [pool.submit(_compile, s, o) for s, o in zip(sources, objects)]
        for f in futures:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stdout}\n{result.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

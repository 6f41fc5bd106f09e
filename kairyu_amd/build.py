"""Compile the gfx950 HIP kernels into ``kairyu_amd/_lib/libkairyu_quant.so``.

Each ``csrc/*.hip`` file is compiled by ``hipcc --offload-arch=gfx950`` into an
object under ``_build/`` (in parallel), then all objects are linked into one
shared library exporting the C ABI declared in ``include/kairyu_quant.h``.
Nothing is JIT-compiled at import time; the built ``.so`` travels with the
source tree.
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
LIB_DIR = PACKAGE_DIR / "_lib"
BUILD_DIR = PACKAGE_DIR.parent / "_build"
LIB_NAME = "libkairyu_quant.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# Per-source additions.  kq_peaks.hip: MFMA results in VGPRs, so the
# register-only MFMA loop carries its accumulators without AGPR copies (the
# default form moves them between AGPRs and VGPRs every iteration there).
EXTRA_FLAGS = {"kq_peaks.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    candidates = [os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"]
    for candidate in candidates:
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the ROCm toolchain is required to build kairyu_amd")


def _compile(source: Path, compiler: str) -> Path:
    obj = BUILD_DIR / (source.stem + ".o")
    cmd = [compiler, *HIPCC_FLAGS, *EXTRA_FLAGS.get(source.name, []), "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every kernel source and link the shared library; returns its path."""

    compiler = hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = jobs or min(len(sources), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(lambda s: _compile(s, compiler), sources))
    target = LIB_DIR / LIB_NAME
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    cmd = [compiler, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(tmp, target)
    if verbose:
        print(f"built {target}", file=sys.stderr)
    return target


if __name__ == "__main__":
    build(verbose=True)

"""Build libdionw_hip.so (the C-ABI library) for gfx950 with hipcc.

Each source compiles to an object in ``_build/`` next to this file; the
objects link into ``dionw_amd/libdionw_hip.so``. Run ``python -m
dionw_amd.csrc.build`` or call ``build()``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
PACKAGE = HERE.parent
LIBRARY = PACKAGE / "libdionw_hip.so"
SOURCES = ("errors.cpp", "momentum.hip", "select.hip", "normuon.hip", "adamw_ema.hip", "gemm.hip")
ARCH = "gfx950"
FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    f"-I{PACKAGE.parent / 'include'}",
    # Packed fp32 instructions stay off (they have given wrong results on
    # this hardware pool); hipcc's host pass warns that it does not know the
    # feature, which is harmless.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
)


def _hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found: the dionw HIP library cannot be built")
    return found


def _compile(hipcc: str, source: str, build_dir: Path) -> Path:
    src = HERE / source
    obj = build_dir / (source + ".o")
    lang = ["-x", "hip"] if source.endswith(".hip") else []
    cmd = [hipcc, *FLAGS, *lang, "-c", str(src), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source}:\n{result.stderr}")
    noise = [
        line
        for line in result.stderr.splitlines()
        if line.strip() and "packed-fp32-ops" not in line
    ]
    if noise:
        print("\n".join(noise))
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every source and link the shared library; returns its path."""
    hipcc = _hipcc()
    build_dir = HERE / "_build"
    build_dir.mkdir(exist_ok=True)
    jobs = min(len(SOURCES), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(lambda s: _compile(hipcc, s, build_dir), SOURCES))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build()

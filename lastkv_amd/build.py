"""Compile the gfx950 HIP sources of this package into ``lastkv_amd/liblastkv_amd.so``.

Every ``csrc/*.hip`` file is compiled with hipcc for gfx950 only, then linked into one shared
library exporting the C ABI declared in ``include/lastkv_amd.h``.  Run as
``python -m lastkv_amd.build``.
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

PKG_DIR = pathlib.Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "liblastkv_amd.so"
LIB_PATH = PKG_DIR / LIB_NAME
OBJ_DIR = PKG_DIR / "_build"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 arithmetic stays disabled: it has produced silent miscomputations on this pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO_DIR / 'include'}",
]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build lastkv_amd")
    return exe


def _compile(src: pathlib.Path, verbose: bool) -> pathlib.Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "not a recognized feature for this target"
    log = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{log}")
    if verbose and log.strip():
        print(log, file=sys.stderr)
    return obj


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every HIP source and link ``liblastkv_amd.so``; returns its path."""

    OBJ_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose=True)
    print(path)

"""Builds libmarian_hip.so (gfx950) from csrc/ with hipcc, in-tree.

Flags that are part of the arithmetic contract:
  -ffp-contract=off                         no fused multiply-add contraction
  -fhip-fp32-correctly-rounded-divide-sqrt  IEEE fp32 division and square root
  -fno-gpu-flush-denormals-to-zero          keep fp32 denormals
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed fp32 ALU ops
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
BUILD_DIR = PKG / "_build"
LIB = PKG / "libmarian_hip.so"
SOURCES = ["gemm.hip", "attention.hip", "block.hip", "rows.hip", "ssru.hip", "lngemm.hip", "engine.hip", "ops.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def source_hash() -> str:
    """SHA-256 over every source the library is built from (csrc/ and the
    public headers, in name order); compiled into the library as its build id."""
    import hashlib

    h = hashlib.sha256()
    files = sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.h")) + list(INCLUDE.glob("*.h")))
    for f in files:
        h.update(f.name.encode())
        h.update(b"\0")
        h.update(f.read_bytes())
    return h.hexdigest()


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the marian-hip library needs ROCm to build")
    return path


def _compile(src: str, build_id: str) -> Path:
    obj = BUILD_DIR / (Path(src).stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-DMARIAN_HIP_BUILD_ID=\"{build_id}\"", "-c",
           str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr[-6000:]}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compiles every source and links the shared library; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    jobs = min(len(SOURCES), max(1, (os.cpu_count() or 2) // 2))
    build_id = source_hash()
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda src: _compile(src, build_id), SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-6000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)

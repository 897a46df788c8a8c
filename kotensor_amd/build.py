"""Builds libkotensor_hip.so in-tree with hipcc for gfx950.

Run ``python -m kotensor_amd.build`` (or ``__graft_entry__.build()``). Every
``csrc/*.hip`` file is compiled to an object under ``kotensor_amd/_build/`` and
linked into ``kotensor_amd/libkotensor_hip.so``.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_build"
LIBRARY = PKG / "libkotensor_hip.so"
ARCH = "gfx950"

# Flags every translation unit shares. Packed fp32 instructions are disabled, fp32
# denormals are kept (quantize must see subnormal scales exactly as IEEE does), and
# '/' stays correctly rounded (HIP's default).
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # the first 16 dwords of a kernel's arguments arrive in scalar registers with the
    # wave (the code keeps a fallback that loads them where the firmware does not), so
    # the first dependent loads do not wait for an argument fetch
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unknown-pragmas",
]
# Per-file extras: quantize rounds exactly like the reference, so nothing may fuse.
EXTRA = {
    "kt_quantize.hip": ["-ffp-contract=off"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def _compile(src: Path) -> Path:
    obj = OUT_DIR / (src.stem + ".o")
    cmd = [hipcc(), *COMMON, *EXTRA.get(src.name, []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compiles every HIP source and links the shared library; returns its path."""
    OUT_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

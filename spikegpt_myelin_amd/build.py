"""Build libwkv_hip.so for gfx950 with hipcc (in-tree; no JIT cache).

Usage: ``python -m spikegpt_myelin_amd.build`` (or ``build()`` from Python).
Every ``csrc/*.hip`` translation unit is compiled to an object in parallel and
linked into ``spikegpt_myelin_amd/libwkv_hip.so``.  hipcc cross-compiles, so
this runs on a machine without a GPU.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libwkv_hip.so"
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from emitting packed (two-wide) fp32
# VALU instructions; plain fp32 arithmetic is used everywhere.
# -ffp-contract=off: every fused multiply-add is an explicit fmaf() in the
# source, so each element type's instantiation rounds identically.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the WKV library needs ROCm's hipcc to build")
    return path


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    if verbose and res.stderr.strip():
        # The host pass does not know the packed-fp32 feature flag; harmless.
        lines = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln]
        if any(ln.strip() for ln in lines):
            print("\n".join(lines), file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = min(len(sources), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    # --no-undefined: a declaration that matches no definition fails here,
    # not when the library is loaded.
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined",
           *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build())

"""Builds libfellm_rocm_kernels.so (HIP kernels for gfx950 + the plugin C ABI).

Run ``python -m fellm_amd.build``.  Objects go to ``fellm_amd/_build/``; the
shared library lands in-tree at ``fellm_amd/libfellm_rocm_kernels.so`` so it
travels with the source tree to the GPU host.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB_NAME = "libfellm_rocm_kernels.so"
LIB_PATH = PKG / LIB_NAME
ARCH = os.environ.get("FELLM_ROCM_ARCH", "gfx950")

SOURCES = ["norm.hip", "elementwise.hip", "embedding.hip", "rope.hip", "router.hip", "gemv.hip", "attention.hip", "moe.hip", "graph.cpp", "plugin.cpp"]

# -ffp-contract=off keeps the reference's operation order (no silent FMA);
# the packed-fp32 feature is disabled for every HIP translation unit.
COMMON_FLAGS = [
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-ffp-contract=off",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
    "-Wall",
    "-Wno-unused-function",
    # A requested unroll that fails leaves register arrays in scratch memory.
    "-Werror=pass-failed",
]
DEVICE_FLAGS = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def _compile(src: str, build_dir: Path = BUILD, extra=()) -> Path:
    obj = build_dir / (Path(src).stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, *extra, "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def _stale(src: str, build_dir: Path) -> bool:
    obj = build_dir / (Path(src).stem + ".o")
    if not obj.exists():
        return True
    # Every header the sources may include: csrc/*.hpp and include/*.h.
    deps = [CSRC / src, *CSRC.glob("*.hpp"), *(ROOT / "include").glob("*.h")]
    return any(d.stat().st_mtime > obj.stat().st_mtime for d in deps if d.exists())


def build(verbose: bool = False, out: Path = LIB_PATH, build_dir: Path = BUILD, defines=(),
          incremental: bool = False) -> Path:
    """Compile every source and link ``out``; ``defines`` are extra -D flags.
    ``incremental`` recompiles only sources newer than their objects (headers
    included); the default rebuilds everything."""
    build_dir.mkdir(parents=True, exist_ok=True)
    extra = [f"-D{d}" for d in defines]
    todo = [s for s in SOURCES if not incremental or _stale(s, build_dir)]
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), 8)) as ex:
        list(ex.map(lambda src: _compile(src, build_dir, extra), todo))
    objs = [build_dir / (Path(src).stem + ".o") for src in SOURCES]
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), *DEVICE_FLAGS, "-shared", "-fPIC", f"-Wl,--version-script={CSRC / 'exports.map'}",
           "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True, incremental="--incremental" in sys.argv)
    sys.exit(0)

"""Builds the gfx950 kernel library ``vortex_torch/_lib/libvortex_hip.so``.

Every ``csrc/*.hip`` file is compiled with hipcc for gfx950 only (object files
under ``_build/``, compiled in parallel) and linked into one shared library
that exports the C ABI declared in ``include/vortex_hip.h``.

Usage: ``python build_native.py [-v]`` or ``build_native.build()``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
CSRC = PKG_ROOT / "csrc"
BUILD_DIR = PKG_ROOT / "_build"
LIB_DIR = PKG_ROOT / "vortex_torch" / "_lib"
LIB_PATH = LIB_DIR / "libvortex_hip.so"

ARCH = "gfx950"

# Packed-FP32 VALU forms are disabled: ordinary float code is left scalar.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Leading pointer and integer kernel arguments (up to eight) are preloaded
    # into SGPRs by the dispatch, so a kernel's first loads need no
    # kernel-argument round trip (arguments after a by-value struct are not).
    "-mllvm", "-amdgpu-kernarg-preload-count=8",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = (res.stdout or "") + (res.stderr or "")
    # The host pass does not know the packed-fp32 feature and says so.
    lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln]
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n" + "\n".join(lines))
    if verbose and lines:
        print("\n".join(lines), flush=True)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compiles every kernel source and links the shared library; returns its path."""
    hipcc = _hipcc()
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    include = f"-I{PKG_ROOT.parent / 'include'}"

    def compile_one(src: Path) -> Path:
        obj = BUILD_DIR / (src.stem + ".o")
        _run([hipcc, *HIP_FLAGS, include, "-c", str(src), "-o", str(obj)], verbose)
        return obj

    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, sources))

    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)

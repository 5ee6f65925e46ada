"""Build libsnnk.so (HIP, gfx950) in-tree.

Every ``csrc/*.hip`` source is compiled to an object with ``hipcc`` in
parallel and the objects are linked into ``snnk/libsnnk.so``.  The build is
explicit (no JIT, no torch extension cache) so the shared library sits next
to the Python package and ships with the source tree.

Usage:  python -m snnk.build            (from triton-pass-analysis_amd/)
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

PKG_DIR = pathlib.Path(__file__).resolve().parent
SRC_ROOT = PKG_DIR.parent
CSRC = SRC_ROOT / "csrc"
BUILD_DIR = SRC_ROOT / "_build"
INCLUDE = SRC_ROOT.parent / "include"
LIB_PATH = PKG_DIR / "libsnnk.so"

ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed-FP32 VALU forms are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # No a*b+c contraction: the neuron updates round every product and sum
    # to fp32 in the reference's order (explicit fmaf calls stay fused).
    "-ffp-contract=off",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found; libsnnk needs ROCm's hipcc")
    return exe


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def sources() -> list[pathlib.Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = True) -> pathlib.Path:
    """Compile every HIP source and link libsnnk.so.  Always rebuilds."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = max(1, min(len(srcs), os.cpu_count() or 1, 8))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC",
           *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    # a kernel whose launch stub the host pass failed to emit leaves an
    # undefined symbol that only shows when the library is loaded
    res = subprocess.run(["nm", "-D", "--undefined-only", str(tmp)], capture_output=True,
                         text=True)
    missing = [ln.split()[-1] for ln in res.stdout.splitlines() if "__device_stub__" in ln]
    if missing:
        raise RuntimeError(f"libsnnk has undefined kernel stubs: {missing[:3]}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[snnk.build] {len(srcs)} sources -> {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build()
    sys.exit(0)

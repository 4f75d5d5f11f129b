"""Build libnmb.so (the gfx950 kernels behind include/nmb.h) in-tree with hipcc.

Usage: ``python -m nano_megatron_amd.build`` or ``nano_megatron_amd.build.build()``.
The library lands next to this file so it travels with the source tree.
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

PKG_DIR = pathlib.Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libnmb.so"
ROOT = PKG_DIR.parent

ARCH = os.environ.get("NMB_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 VALU ops are disabled for every kernel in this library
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; ROCm is required to build libnmb.so")
    return path


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [_hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line
        for line in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in line  # host pass does not know the device feature
    )
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{out}")
    if out.strip():
        print(out, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> pathlib.Path:
    """Compile every csrc/*.hip for gfx950 and link libnmb.so; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, (os.cpu_count() or 2)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()

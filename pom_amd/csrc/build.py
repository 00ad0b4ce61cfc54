"""Build libpom_amd.so (HIP kernels + C ABI) for gfx950 with hipcc.

Usage: python pom_amd/csrc/build.py [--jobs N]
The library is written next to the package (pom_amd/libpom_amd.so).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
SOURCES = ["kernels_bf16.hip", "kernels_f16.hip", "kernels_f32.hip", "transpose.hip", "gemm.hip", "capi.cpp",
           "layer.cpp"]
OUT = os.path.join(PKG, "libpom_amd.so")
BUILD_DIR = os.path.join(PKG, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("POM_AMD_ARCH", "gfx950")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # packed fp32 ops are disabled: some forms have given wrong results on these boxes
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    f"-I{os.path.join(ROOT, 'include')}",
]


def _deps(path: str, seen: set) -> set:
    """The file and every local header it includes, recursively."""
    if path in seen or not os.path.exists(path):
        return seen
    seen.add(path)
    with open(path) as f:
        for line in f:
            m = re.match(r'\s*#\s*include\s+"([^"]+)"', line)
            if m:
                _deps(os.path.normpath(os.path.join(os.path.dirname(path), m.group(1))), seen)
    return seen


def _stale(src: str, obj: str) -> bool:
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(d) > t for d in _deps(os.path.join(HERE, src), set()))


def _compile(src: str, incremental: bool = False) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    if incremental and not _stale(src, obj):
        return obj
    lang = ["-x", "hip"]
    cmd = [HIPCC, *FLAGS, *lang, "-c", os.path.join(HERE, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed on {src}")
    return obj


def build(jobs: int = 4, verbose: bool = True, incremental: bool = False) -> str:
    """Compile every source (or, with incremental=True, only stale objects) and link."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, incremental), SOURCES))
    tmp = OUT + ".tmp"
    # rocBLAS / hipBLASLt by SONAME: in a process that imported torch first these
    # resolve to torch's loaded copies (pom_blas_library reports which)
    rocm_lib = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
           f"-L{rocm_lib}", "-lrocblas", "-lhipblaslt"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("link failed")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--incremental", action="store_true", help="recompile only stale objects")
    a = ap.parse_args()
    build(a.jobs, incremental=a.incremental)

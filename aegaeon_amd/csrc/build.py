"""Build libaegkv.so (the C-ABI KV data path) for gfx950 with hipcc.

Each .hip translation unit is compiled to an object under ``_build/`` next to
the package, in parallel, then linked into ``aegaeon_amd/libaegkv.so``.
Usage: ``python -m aegaeon_amd.csrc.build`` or ``build_library()``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sysconfig
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
ROOT = PKG.parent
BUILD_DIR = ROOT / "_build"
LIB_PATH = PKG / "libaegkv.so"

SOURCES = [
    "runtime.hip", "blocks.hip", "append.hip", "attention.hip", "inputs.hip",
    "prefill.hip", "signals.hip", "block_manager.cpp",
]
ARCH = "gfx950"

# Packed FP32 instructions are disabled for every HIP translation unit.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the KV data path needs ROCm's hipcc")
    return exe


def _compile(src: str) -> Path:
    obj = BUILD_DIR / (Path(src).stem + ".o")
    if src.endswith(".cpp"):
        # host-only bookkeeping: plain C++, no device code
        cmd = ["g++", "-O2", "-fPIC", "-std=c++17", "-Wall", "-c", str(CSRC / src), "-o", str(obj)]
    else:
        cmd = [_hipcc(), *COMMON_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed for {src}:\n{res.stdout}\n{res.stderr}")
    return obj


def build_listpack() -> Path:
    """Compile the CPython extension that packs the request lists
    (``aegaeon_amd/_listpack``, plain C against this interpreter's headers)."""
    out = CSRC.parent / ("_listpack" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_name(out.name + ".tmp")
    cmd = ["gcc", "-O2", "-shared", "-fPIC", "-Wall", f"-I{sysconfig.get_paths()['include']}",
           str(CSRC / "listpack.c"), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed for listpack.c:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    return out


def build_library(verbose: bool = False) -> Path:
    """Compile every source and link ``libaegkv.so`` (and the list-packing
    extension); returns the library's path."""
    BUILD_DIR.mkdir(exist_ok=True)
    jobs = min(len(SOURCES), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        pack = ex.submit(build_listpack)
        objs = list(ex.map(_compile, SOURCES))
        pack.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build_library(verbose=True)
    sys.exit(0)

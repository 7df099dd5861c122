"""Build ``libw4a16.so`` (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python -m w4a16._build            # from the package directory's parent

The library's sources under ``csrc/`` are compiled for gfx950 only, then linked
into ``w4a16/libw4a16.so`` next to this file, where :mod:`w4a16._lib` loads it.
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(ROOT_DIR, "csrc")
BUILD_DIR = os.path.join(CSRC, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libw4a16.so")
SOURCES = ["gemv.hip", "gemm_mfma.hip", "gemm_occ2.hip", "gemm_stream.hip", "gemm_skinny.hip",
           "simt.hip", "quant.hip", "capi.cpp"]
HEADERS = ["w4a16_device.h", "w4a16_launch.h", "decode_table.inc"]
PUBLIC_HEADER = os.path.join(os.path.dirname(ROOT_DIR), "include", "w4a16.h")
ARCH = "gfx950"


def source_hash() -> str:
    """sha256 over the names and contents of every file the library is built
    from (the csrc sources and headers, and the public header) and over the
    compiler flags.  Compiled into
    the library (w4a16_build_id) and compared by the loader, so a library
    built from other sources is refused rather than silently run."""
    h = hashlib.sha256()
    files = [(n, os.path.join(CSRC, n)) for n in sorted(SOURCES + HEADERS)]
    files.append(("include/w4a16.h", PUBLIC_HEADER))
    for name, path in files:
        with open(path, "rb") as f:
            data = f.read()
        h.update(name.encode() + b"\0" + len(data).to_bytes(8, "little") + data)
    h.update(repr((COMMON_FLAGS, sorted(SOURCE_FLAGS.items()))).encode())
    return h.hexdigest()

# -packed-fp32-ops keeps the compiler from emitting packed fp32 VALU ops.
# No fast-math: the quantiser relies on IEEE division and signed zeros.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# Per source: the kernels' leading kernel arguments preloaded into
# SGPRs by the dispatch (their first loads then wait for no kernel-argument
# load; firmware without the feature runs the compiler's load prologue
# instead).
_PRELOAD = ["-mllvm", "-amdgpu-kernarg-preload-count=16"]
SOURCE_FLAGS = {
    "gemv.hip": _PRELOAD,
    "gemm_skinny.hip": _PRELOAD,
    "gemm_stream.hip": _PRELOAD,
    "gemm_occ2.hip": _PRELOAD,   # and the split-K reduction kernel
}


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found: the ROCm toolchain is needed to build libw4a16.so")
    return exe


def _compile(src: str, verbose: bool, defines: list[str]) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *SOURCE_FLAGS.get(src, []), *defines, "-x", "hip", "-c",
           os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stdout}\n{res.stderr}")
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in (res.stderr or "").splitlines() if noise not in ln and ln.strip()]
    if msgs and verbose:
        print("\n".join(msgs), file=sys.stderr)
    return obj


def _link(objs: list[str], path: str, verbose: bool) -> None:
    tmp = path + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, path)


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every source and link libw4a16.so; returns the library path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1, 8)
    defines = [f'-DW4A16_SOURCE_HASH="{source_hash()}"']
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose, defines), SOURCES))
    _link(objs, LIB_PATH, verbose)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

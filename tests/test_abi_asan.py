"""Host-side AddressSanitizer run of the C ABI (CPU, no GPU).

The library's host code -- ``csrc/capi.cpp``: argument checks, the planner,
status strings, workspace sizing -- is compiled once more with
``-fsanitize=address`` (host side only; the kernels are the ordinary objects)
and linked with ``tests/asan/abi_driver.cpp``, which calls every entry point of
``include/w4a16.h`` along the paths that return before any device work.  Any
heap / stack overflow, use after free or similar in those paths aborts the
driver with an ASan report; wrong status codes fail it with a message.
"""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
DRIVER = os.path.join(ROOT, "tests", "asan", "abi_driver.cpp")
INCLUDE = os.path.join(ROOT, "include")


def _clang() -> str | None:
    for c in ("/opt/rocm/llvm/bin/clang++", shutil.which("amdclang++") or ""):
        if c and os.path.exists(c):
            return c
    return None


def _run(cmd: list[str], **kw) -> subprocess.CompletedProcess:
    return subprocess.run(cmd, capture_output=True, text=True, **kw)


@pytest.mark.timeout(900)
def test_c_abi_host_paths_under_asan(tmp_path):
    from w4a16 import _build

    clang = _clang()
    try:
        hipcc = _build.hipcc()
    except RuntimeError:
        hipcc = None
    if not clang or not hipcc:
        pytest.skip("ROCm clang++ / hipcc not available")
    # the kernels: the ordinary objects (built here if build() has not run)
    os.makedirs(_build.BUILD_DIR, exist_ok=True)
    defines = [f'-DW4A16_SOURCE_HASH="{_build.source_hash()}"']
    objs = []
    for src in _build.SOURCES:
        if src == "capi.cpp":
            continue
        obj = os.path.join(_build.BUILD_DIR, os.path.splitext(src)[0] + ".o")
        if not os.path.exists(obj) or os.path.getmtime(obj) < os.path.getmtime(
                os.path.join(_build.CSRC, src)):
            obj = _build._compile(src, False, defines)
        objs.append(obj)
    # the host code with AddressSanitizer (host side only)
    asan = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]
    capi = str(tmp_path / "capi_asan.o")
    r = _run([hipcc, *_build.COMMON_FLAGS, *defines, *asan, "-x", "hip", "-c",
              os.path.join(_build.CSRC, "capi.cpp"), "-o", capi])
    assert r.returncode == 0, r.stderr
    lib = str(tmp_path / "libw4a16_asan.so")
    r = _run([hipcc, f"--offload-arch={_build.ARCH}", "-shared", "-fPIC", *asan, "-o", lib, capi,
              *objs])
    assert r.returncode == 0, r.stderr
    exe = str(tmp_path / "abi_driver")
    r = _run([clang, "-std=c++17", "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer",
              f"-I{INCLUDE}", DRIVER, f"-L{tmp_path}", "-lw4a16_asan", f"-Wl,-rpath,{tmp_path}",
              "-o", exe])
    assert r.returncode == 0, r.stderr
    env = dict(os.environ)
    # the HIP runtime's own allocations are not this library's to report
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1:abort_on_error=0"
    r = _run([exe], env=env, timeout=600)
    assert r.returncode == 0 and "abi_driver ok" in r.stdout, r.stdout + r.stderr
    assert "AddressSanitizer" not in r.stderr, r.stderr

"""ctypes binding of ``libw4a16.so`` (declarations: ``include/w4a16.h``).

The library is built in-tree by :mod:`w4a16._build`.  Loading never falls back to
anything: a missing library, one lacking a declared symbol, one of another ABI
version, or one built from other sources than those beside it (the sha256 the
build compiles in, ``w4a16_build_id``, against the sources' own) raises
``ImportError`` with the build command, so no caller can silently run without
the HIP kernels or on kernels older than the sources.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libw4a16.so")
ABI_VERSION = 2

# enum w4a16_kernel
KERNEL_AUTO, KERNEL_GEMV, KERNEL_MFMA, KERNEL_SIMT, KERNEL_SKINNY = 0, 1, 2, 3, 4
KERNEL_NAMES = {KERNEL_GEMV: "gemv", KERNEL_MFMA: "mfma", KERNEL_SIMT: "simt",
                KERNEL_SKINNY: "skinny"}
# plan tile_cfg numbers each family has (others are refused: retired tilings)
MFMA_CONFIGS = (1, 2, 6, 7, 11, 12, 13, 14)
MFMA_SPLIT_CONFIGS = (7, 11, 12, 13, 14)
GEMV_CONFIGS = (1, 2, 4, 5)          # 8 / 16 waves, + LDS-staged activations (M <= 2)
GEMV_MFMA_CONFIGS = (6, 7)           # 16 / 8 waves, staged, MFMA dot products (M <= 2, 64 / 128 columns)
SKINNY_CONFIGS = (0, 2, 3)           # 16 / 32 / 64-column blocks
# w4a16_plan.flags: W4A16_PLAN_ANY_ZEROS (zeros other than integers in [-1024, 1024])
PLAN_ANY_ZEROS = 1
# W4A16_NOALLOC_SCRATCH_BYTES: the static scratch of w4a16_gemm_f16_noalloc
NOALLOC_SCRATCH_BYTES = 16 << 20

# enum w4a16_status
STATUS = {
    0: "W4A16_OK",
    -1: "W4A16_ERR_NULL_POINTER",
    -2: "W4A16_ERR_BAD_SHAPE",
    -3: "W4A16_ERR_BAD_GROUP",
    -4: "W4A16_ERR_WORKSPACE",
    -5: "W4A16_ERR_BAD_PLAN",
    -6: "W4A16_ERR_NO_DEVICE",
}


class Plan(ctypes.Structure):
    """Mirror of ``struct w4a16_plan``."""

    _fields_ = [
        ("kernel", ctypes.c_int32),
        ("split_k", ctypes.c_int32),
        ("tile_cfg", ctypes.c_int32),
        ("tile_m", ctypes.c_int32),
        ("tile_n", ctypes.c_int32),
        ("grid_x", ctypes.c_int64),
        ("grid_y", ctypes.c_int64),
        ("workspace_bytes", ctypes.c_int64),
        ("flags", ctypes.c_int32),
    ]

    def as_dict(self) -> dict:
        d = {name: getattr(self, name) for name, _ in self._fields_}
        d["kernel_name"] = KERNEL_NAMES.get(self.kernel, "?")
        return d


_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_sz = ctypes.c_size_t
_int = ctypes.c_int

# name -> (restype, argtypes); exactly the functions include/w4a16.h declares
SIGNATURES = {
    "w4a16_abi_version": (_int, []),
    "w4a16_build_id": (ctypes.c_char_p, []),
    "w4a16_status_string": (ctypes.c_char_p, [_int]),
    "w4a16_gemm_plan": (_int, [_i64, _i64, _i64, _i64, _i32, _i32, ctypes.POINTER(Plan)]),
    "w4a16_gemm_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "w4a16_zeros_check_f16": (_int, [_vp, _i64, _vp, _vp]),
    "w4a16_gemm_f16": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _sz, _vp]),
    "w4a16_linear_f16": (
        _int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _sz, _vp]),
    "w4a16_gemm_f16_planned": (
        _int,
        [ctypes.POINTER(Plan), _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _sz, _vp],
    ),
    "w4a16_gemm_f16_strided": (
        _int,
        [ctypes.POINTER(Plan), _vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
         _vp, _sz, _vp],
    ),
    "w4a16_gemm_f16_noalloc": (
        _int,
        [ctypes.POINTER(Plan), _vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
         _vp],
    ),
    "w4a16_quantize_pack_f16": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "w4a16_quantize_pack_f32": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "w4a16_pack_int4": (_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "w4a16_unpack_int4": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "w4a16_dequantize_f16": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
}

_LIB = None
_LOCK = threading.Lock()


def _sources_hash() -> str | None:
    """sha256 of the sources beside the package (None when they are absent,
    e.g. a library installed without its sources)."""
    from . import _build

    if not os.path.isdir(_build.CSRC):
        return None
    return _build.source_hash()


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise ImportError if it is unusable."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; build it with `python -m w4a16._build` "
                "(or __graft_entry__.build()) -- there is no non-HIP fallback")
        try:
            lib = ctypes.CDLL(LIB_PATH)
        except OSError as e:
            raise ImportError(f"cannot load {LIB_PATH}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as e:
                raise ImportError(f"{LIB_PATH} lacks {name} (built from older sources); "
                                  "rebuild it") from e
            fn.restype = res
            fn.argtypes = args
        ver = lib.w4a16_abi_version()
        if ver != ABI_VERSION:
            raise ImportError(f"{LIB_PATH} has ABI {ver}, expected {ABI_VERSION}; rebuild it")
        want = _sources_hash()
        got = lib.w4a16_build_id().decode()
        if want is not None and got != want:
            raise ImportError(
                f"{LIB_PATH} was built from other sources (build id {got[:12]}, sources "
                f"{want[:12]}); rebuild it with `python -m w4a16._build`")
        _LIB = lib
        return lib


def status_text(code: int) -> str:
    lib = load()
    return lib.w4a16_status_string(code).decode()


def check(code: int, what: str) -> None:
    """Raise RuntimeError for a non-zero status (like the reference's TORCH_CHECK)."""
    if code != 0:
        name = STATUS.get(code, "hipError" if code > 0 else "?")
        raise RuntimeError(f"{what} failed: {name} ({code}): {status_text(code)}")


def plan(M: int, N: int, K: int, group_size: int, kernel: int = 0, split_k: int = 0) -> Plan:
    """The launch the library will make for this shape (see w4a16_gemm_plan)."""
    p = Plan()
    check(load().w4a16_gemm_plan(M, N, K, group_size, kernel, split_k, ctypes.byref(p)),
          "w4a16_gemm_plan")
    return p

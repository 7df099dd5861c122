"""CPU tests of the C ABI library and of the Python host logic (no GPU compute).

* libw4a16.so loads and exports every function include/w4a16.h declares;
* the ABI rejects invalid arguments with its negative status codes before it
  touches a device (null pointers, bad shapes / group sizes, missing workspace);
* the planner picks the kernel family by shape;
* the Python wrappers raise the reference's exception types for bad input
  (AssertionError / ValueError, reference quant.py:114-119, triton_kernel.py:153-187,
  linear.py:38-41) before any device work.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
HEADER = os.path.join(ROOT, "include", "w4a16.h")


def _declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(w4a16_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_api():
    names = _declared_functions()
    for required in ("w4a16_gemm_f16", "w4a16_quantize_pack_f16", "w4a16_pack_int4",
                     "w4a16_unpack_int4", "w4a16_dequantize_f16", "w4a16_linear_f16",
                     "w4a16_gemm_plan", "w4a16_abi_version", "w4a16_status_string"):
        assert required in names


def test_library_exports_every_declared_symbol(lib):
    from w4a16 import _lib

    for name in _declared_functions():
        assert hasattr(lib, name), f"libw4a16.so does not export {name}"
        assert name in _lib.SIGNATURES, f"ctypes binding lacks {name}"
    assert set(_lib.SIGNATURES) == set(_declared_functions())


def test_abi_version_and_status_strings(lib):
    assert lib.w4a16_abi_version() == 2
    for code in (0, -1, -2, -3, -4, -5, -6):
        s = lib.w4a16_status_string(code)
        assert s and isinstance(s, bytes)
    assert lib.w4a16_status_string(-99) == b"unknown status"


NULL = None


@pytest.mark.parametrize("M,N,K,G,expect", [
    (-1, 16, 64, 32, -2),     # negative M
    (1, 16, 60, 32, -2),      # K % 8 != 0
    (1, 16, 64, 0, -3),       # G <= 0
    (1, 16, 64, 48, -3),      # K % G != 0
    (1, 2**31, 64, 32, -2),   # N > INT32_MAX
])
def test_gemm_rejects_bad_shapes(lib, M, N, K, G, expect):
    dummy = ctypes.c_void_p(256)
    code = lib.w4a16_gemm_f16(dummy, dummy, dummy, dummy, dummy, M, N, K, G, NULL, 0, NULL)
    assert code == expect


def test_gemm_rejects_null_pointers(lib):
    dummy = ctypes.c_void_p(256)
    assert lib.w4a16_gemm_f16(NULL, dummy, dummy, dummy, dummy, 1, 16, 64, 32, NULL, 0, NULL) == -1
    assert lib.w4a16_gemm_f16(dummy, NULL, dummy, dummy, dummy, 1, 16, 64, 32, NULL, 0, NULL) == -1
    assert lib.w4a16_gemm_f16(dummy, dummy, dummy, dummy, NULL, 1, 16, 64, 32, NULL, 0, NULL) == -1
    # empty problems are valid and launch nothing
    assert lib.w4a16_gemm_f16(NULL, NULL, NULL, NULL, NULL, 0, 16, 64, 32, NULL, 0, NULL) == 0
    assert lib.w4a16_gemm_f16(NULL, NULL, NULL, NULL, NULL, 4, 0, 64, 32, NULL, 0, NULL) == 0


def test_split_k_gemv_requires_workspace(lib):
    from w4a16 import _lib

    # a forced 4-way split-K GEMV needs 4 * M * N fp32 partials
    p = _lib.plan(1, 1024, 4096, 128, _lib.KERNEL_GEMV, 4)
    assert p.kernel == _lib.KERNEL_GEMV and p.split_k == 4 and p.workspace_bytes == 4 * 1024 * 4
    a = ctypes.c_void_p(1 << 12)   # aligned fake pointers: never dereferenced
    code = lib.w4a16_gemm_f16_planned(ctypes.byref(p), a, a, a, a, NULL, a, 1, 1024, 4096, 128,
                                      NULL, 0, NULL)
    assert code == -4
    code = lib.w4a16_gemm_f16_planned(ctypes.byref(p), a, a, a, a, NULL, a, 1, 1024, 4096, 128,
                                      a, 16, NULL)
    assert code == -4
    # a wave configuration the kernel does not have
    p.tile_cfg = 6
    code = lib.w4a16_gemm_f16_planned(ctypes.byref(p), a, a, a, a, NULL, a, 1, 1024, 4096, 128,
                                      a, 1 << 30, NULL)
    assert code == -5
    # 16 waves and the LDS-staged activation configurations are for M <= 2 only
    p4 = _lib.plan(4, 1024, 4096, 128, _lib.KERNEL_GEMV, 4)
    for cfg in (2, 3, 4, 5):
        p4.tile_cfg = cfg
        code = lib.w4a16_gemm_f16_planned(ctypes.byref(p4), a, a, a, a, NULL, a, 4, 1024, 4096,
                                          128, a, 1 << 30, NULL)
        assert code == -5
    p.tile_cfg = 1
    # a column width the kernel does not have
    p.tile_n = 48
    code = lib.w4a16_gemm_f16_planned(ctypes.byref(p), a, a, a, a, NULL, a, 1, 1024, 4096, 128,
                                      a, 1 << 30, NULL)
    assert code == -5


def test_plan_flags_and_zeros_check_arguments(lib):
    """Plans start with no flags; a flag bit other than W4A16_PLAN_ANY_ZEROS is
    refused before any launch; the zeros check validates its arguments and
    launches nothing for an empty tensor."""
    from w4a16 import _lib

    p = _lib.plan(1, 1024, 4096, 128)
    assert p.flags == 0
    a = ctypes.c_void_p(1 << 12)   # aligned fake pointers: never dereferenced
    for bad in (2, 4, 1 | 8, -1):
        p.flags = bad
        assert lib.w4a16_gemm_f16_planned(ctypes.byref(p), a, a, a, a, NULL, a, 1, 1024, 4096,
                                          128, NULL, 0, NULL) == -5
        assert lib.w4a16_gemm_f16_strided(ctypes.byref(p), a, 4096, a, a, a, NULL, a, 1024, 1,
                                          1024, 4096, 128, NULL, 0, NULL) == -5
        assert lib.w4a16_gemm_f16_noalloc(ctypes.byref(p), a, 4096, a, a, a, NULL, a, 1024, 1,
                                          1024, 4096, 128, NULL) == -5
    assert lib.w4a16_zeros_check_f16(a, -1, a, NULL) == -2
    assert lib.w4a16_zeros_check_f16(NULL, 8, a, NULL) == -1
    assert lib.w4a16_zeros_check_f16(a, 8, NULL, NULL) == -1
    assert lib.w4a16_zeros_check_f16(NULL, 0, NULL, NULL) == 0


def test_retired_configurations_refused(lib):
    """Tile / wave configurations retired from the library (measured slower on
    every shape) are refused by number before anything is launched (fake,
    never dereferenced pointers: no call here may reach a launch; a live GEMV
    configuration with a split and no workspace stops at the workspace
    check)."""
    from w4a16 import _lib

    a = ctypes.c_void_p(1 << 12)
    M, N, K, G = 128, 1024, 4096, 128
    for cfg in range(16):
        if cfg in _lib.MFMA_CONFIGS:
            continue       # valid: would launch
        p = _lib.plan(M, N, K, G, _lib.KERNEL_MFMA, 1)
        p.tile_cfg = cfg
        code = lib.w4a16_gemm_f16_planned(ctypes.byref(p), a, a, a, a, NULL, a, M, N, K, G,
                                          NULL, 0, NULL)
        assert code == -5, cfg
    for cfg in range(8):
        p = _lib.plan(1, N, K, G, _lib.KERNEL_GEMV, 4)
        p.tile_cfg = cfg
        code = lib.w4a16_gemm_f16_planned(ctypes.byref(p), a, a, a, a, NULL, a, 1, N, K, G,
                                          NULL, 0, NULL)
        assert code == (-4 if cfg in _lib.GEMV_CONFIGS else -5), cfg
    for cols in (16, 32, 64, 128, 256):      # MFMA dot products: 64 / 128 columns only
        for cfg in _lib.GEMV_MFMA_CONFIGS:
            p = _lib.plan(1, N, K, G, _lib.KERNEL_GEMV, 4)
            p.tile_cfg, p.tile_n = cfg, cols
            code = lib.w4a16_gemm_f16_planned(ctypes.byref(p), a, a, a, a, NULL, a, 1, N, K, G,
                                              NULL, 0, NULL)
            assert code == (-4 if cols in (64, 128) else -5), (cfg, cols)
    for cfg in range(6):
        p = _lib.plan(16, N, K, G, _lib.KERNEL_SKINNY, 0)
        p.tile_cfg = cfg
        if cfg in _lib.SKINNY_CONFIGS:
            continue       # valid: would launch
        code = lib.w4a16_gemm_f16_planned(ctypes.byref(p), a, a, a, a, NULL, a, 16, N, K, G,
                                          NULL, 0, NULL)
        assert code == -5, cfg


def test_skinny_row_groups_are_checked(lib):
    """A skinny plan's tile_m is the rows of y per workgroup: all of them (M
    rounded up to 16) or one 16- or 8-row group; 32-column blocks hold at most
    32 rows, 64-column blocks 16.  Anything else is refused before a launch."""
    from w4a16 import _lib

    N, K, G = 1024, 4096, 128
    a = ctypes.c_void_p(1 << 12)
    # (the accepted forms -- e.g. M = 40 with 48 or 16 rows on 16-column
    # blocks, 16 rows on 32- or 64-column blocks -- run in the GPU tests)
    for M, cfg, rows in ((40, 0, 32), (40, 2, 48), (24, 3, 32), (8, 0, 0), (8, 0, 4),
                         (64, 3, 64), (64, 2, 64), (17, 0, 17), (16, 0, 48), (40, 0, 24)):
        p = _lib.plan(M, N, K, G, _lib.KERNEL_SKINNY, 0)
        p.tile_cfg, p.tile_m = cfg, rows
        code = lib.w4a16_gemm_f16_planned(ctypes.byref(p), a, a, a, a, NULL, a, M, N, K, G,
                                          NULL, 0, NULL)
        assert code == -5, (M, cfg, rows, code)


def test_skinny_plans_check_their_load_alignment(lib):
    """32- and 64-column skinny blocks load 2 / 4 adjacent columns per lane in
    one load: 8 / 16-byte weights and 4 / 8-byte scales and zeros.  Pointers
    aligned for 16-column blocks only are refused for those plans."""
    from w4a16 import _lib

    M, N, K, G = 16, 1024, 4096, 128
    good = ctypes.c_void_p(1 << 12)
    for cfg, qw_off, sz_off in ((2, 4, 2), (3, 8, 4), (3, 4, 2)):
        p = _lib.plan(M, N, K, G, _lib.KERNEL_SKINNY, 0)
        p.tile_cfg = cfg
        qw = ctypes.c_void_p((1 << 12) + qw_off)
        sz = ctypes.c_void_p((1 << 12) + sz_off)
        assert lib.w4a16_gemm_f16_planned(ctypes.byref(p), good, qw, good, good, NULL, good, M, N,
                                          K, G, NULL, 0, NULL) == -5, cfg
        assert lib.w4a16_gemm_f16_planned(ctypes.byref(p), good, good, sz, good, NULL, good, M, N,
                                          K, G, NULL, 0, NULL) == -5, cfg
        assert lib.w4a16_gemm_f16_planned(ctypes.byref(p), good, good, good, sz, NULL, good, M, N,
                                          K, G, NULL, 0, NULL) == -5, cfg


def test_planned_rejects_mismatched_plan(lib):
    from w4a16 import _lib

    p = _lib.plan(1, 4096, 4096, 128, _lib.KERNEL_GEMV, 1)
    a = ctypes.c_void_p(1 << 12)
    # GEMV plan used for M = 64 (GEMV takes M <= 8)
    code = lib.w4a16_gemm_f16_planned(ctypes.byref(p), a, a, a, a, NULL, a, 64, 4096, 4096, 128,
                                      NULL, 0, NULL)
    assert code == -5
    # misaligned activation pointer for a vector kernel
    code = lib.w4a16_gemm_f16_planned(ctypes.byref(p), ctypes.c_void_p((1 << 12) + 2), a, a, a,
                                      NULL, a, 1, 4096, 4096, 128, NULL, 0, NULL)
    assert code == -5


def test_strided_entry_validates_row_strides(lib):
    """w4a16_gemm_f16_strided: ldx >= K and ldy >= N (else BAD_SHAPE, before any
    launch); a vector plan refuses strides its loads / stores cannot take."""
    from w4a16 import _lib

    a = ctypes.c_void_p(1 << 12)
    M, N, K, G = 64, 4096, 4096, 128
    p = _lib.plan(M, N, K, G, _lib.KERNEL_MFMA, 1)
    for ldx, ldy in ((K - 8, N), (K, N - 4), (1 << 31, N), (K, 1 << 31)):
        for plan in (ctypes.byref(p), NULL):
            code = lib.w4a16_gemm_f16_strided(plan, a, ldx, a, a, a, NULL, a, ldy, M, N, K, G,
                                              NULL, 0, NULL)
            assert code == -2, (ldx, ldy)
    # rows of x not 16-byte aligned (ldx % 8 != 0), rows of y not 8-byte
    # aligned for the MFMA kernels' 4-column stores (ldy % 4 != 0)
    for ldx, ldy in ((K + 4, N), (K, N + 2)):
        code = lib.w4a16_gemm_f16_strided(ctypes.byref(p), a, ldx, a, a, a, NULL, a, ldy, M, N,
                                          K, G, NULL, 0, NULL)
        assert code == -5, (ldx, ldy)
    # the skinny kernel stores single elements: any ldy
    ps = _lib.plan(M, N, K, G, _lib.KERNEL_SKINNY, 0)
    code = lib.w4a16_gemm_f16_strided(ctypes.byref(ps), a, K + 4, a, a, a, NULL, a, N + 1, M, N,
                                      K, G, NULL, 0, NULL)
    assert code == -5    # (ldx still must keep rows 16-byte aligned)
    # a strided x beyond one buffer resource (2 GiB) is refused by a vector plan
    code = lib.w4a16_gemm_f16_strided(ctypes.byref(p), a, 1 << 25, a, a, a, NULL, a, N, M, N, K,
                                      G, NULL, 0, NULL)
    assert code == -5
    # empty shapes return before looking at pointers
    assert lib.w4a16_gemm_f16_strided(NULL, NULL, K, NULL, NULL, NULL, NULL, NULL, N, 0, N, K, G,
                                      NULL, 0, NULL) == 0


def test_group_reciprocal_division_is_exact():
    """The kernels find the quantisation group of row k as
    (umulhi(k, magic) + k) >> shift, with shift = ceil(log2 G) and
    magic = floor(2^32 (2^shift - G) / G) + 1 (group_div in csrc/w4a16_launch.h).
    Checked against integer division for every G up to 4096 and for large G,
    at multiples of G +- 1 near 0 and near 2^31 and at random k < 2^31."""
    import numpy as np

    rng = np.random.default_rng(0)
    rand = rng.integers(0, 2**31, size=2000, dtype=np.uint64)
    for G in list(range(1, 4097)) + [8192, 14336, 28672, 1 << 20, 3 << 20, (1 << 31) - 1]:
        shift = (G - 1).bit_length()
        magic = ((1 << 32) * ((1 << shift) - G)) // G + 1
        assert 1 <= magic < 2**32
        mult = np.arange(0, 64, dtype=np.uint64) * np.uint64(G)
        top = np.uint64(((2**31 - 1) // G) * G) - np.arange(0, 64, dtype=np.uint64) * np.uint64(G)
        k = np.concatenate([mult, mult + 1, mult - 1, top, top + 1, top - 1, rand,
                            np.array([0, 1, 2**31 - 1], dtype=np.uint64)])
        k = k[k < 2**31]
        q = (((k * np.uint64(magic)) >> np.uint64(32)) + k) >> np.uint64(shift)
        assert np.array_equal(q, k // np.uint64(G)), G


def test_quant_entry_points_reject_bad_args(lib):
    a = ctypes.c_void_p(1 << 12)
    assert lib.w4a16_quantize_pack_f16(a, a, a, a, 100, 16, 64, a, NULL) == -2
    assert lib.w4a16_quantize_pack_f16(a, a, a, a, 96, 16, 64, a, NULL) == -3
    assert lib.w4a16_quantize_pack_f16(a, a, a, a, 128, 16, 64, NULL, NULL) == -1
    assert lib.w4a16_quantize_pack_f32(NULL, a, a, a, 128, 16, 64, a, NULL) == -1
    assert lib.w4a16_pack_int4(a, a, 12, 4, a, NULL) == -2
    assert lib.w4a16_pack_int4(NULL, a, 16, 4, a, NULL) == -1
    assert lib.w4a16_unpack_int4(a, NULL, 16, 4, NULL) == -1
    assert lib.w4a16_dequantize_f16(a, a, a, NULL, 128, 4, 64, NULL) == -1
    assert lib.w4a16_dequantize_f16(a, a, a, a, 128, 4, 0, NULL) == -3
    # empty inputs launch nothing
    assert lib.w4a16_quantize_pack_f16(NULL, NULL, NULL, NULL, 0, 16, 64, NULL, NULL) == 0
    assert lib.w4a16_unpack_int4(NULL, NULL, 16, 0, NULL) == 0


@pytest.mark.parametrize("M,N,K,G,kernel", [
    (1, 4096, 4096, 128, "gemv"),
    (3, 28672, 4096, 128, "skinny"),  # wide N, K <= 4096: 64-column skinny blocks from M = 3
    (3, 28672, 8192, 128, "skinny"),  # ... and at longer K (the skinny loop)
    (3, 28672, 4096, 32, "skinny"),   # ... at any G with K <= 4096
    (3, 28672, 8192, 32, "gemv"),     # ... but G = 32 with K > 4096 keeps the GEMV
    (3, 2048, 16384, 128, "gemv"),    # few column blocks, long K: the GEMV split along K
    (5, 2048, 16384, 128, "skinny"),  # ... at M <= 4 for half the CUs' worth of blocks
    (6, 1024, 8192, 128, "gemv"),     # ... up to M = 8 for a quarter
    (1, 2560, 2048, 128, "skinny"),   # M <= 2, K <= 2048: the skinny kernel ...
    (1, 6144, 2048, 128, "gemv"),     # ... outside the 32-column band
    (2, 6144, 1024, 128, "skinny"),   # ... (which it takes up to K = 1024)
    (4, 28672, 4096, 128, "skinny"),
    (2, 6144, 4096, 128, "skinny"),   # M <= 2, 4096 < N <= 8192: the skinny kernel's 32-column blocks
    (2, 6144, 4096, 32, "skinny"),    # ... at any G up to K = 4096
    (2, 6144, 8192, 64, "gemv"),
    (2, 6144, 2048, 128, "gemv"),     # ... not for K <= 2048
    (3, 4096, 14336, 128, "skinny"),  # 3 <= M <= 8 up to N = 16384: MFMA skinny
    (8, 4096, 4096, 128, "skinny"),
    (5, 28672, 4096, 128, "skinny"),
    (5, 28672, 4096, 64, "skinny"),   # 64-column blocks with G % 64 == 0 ...
    (8, 28672, 8192, 64, "skinny"),
    (8, 28672, 8192, 32, "mfma"),     # ... or K <= 4096; else the streamed small-M tiles
    (16, 11008, 4096, 32, "skinny"),
    (8, 4096, 28672, 128, "skinny"),  # long rows on 16-column blocks: skinny up to M = 8 ...
    (12, 4096, 28672, 128, "mfma"),   # ... the streamed tiles from M = 9 at K >= 24576
    (16, 4096, 20480, 64, "mfma"),    # ... from M = 16 beyond K = 16384
    (16, 4096, 14336, 64, "skinny"),
    (16, 4096, 11008, 32, "mfma"),    # ... and beyond K = 8192 with G = 32
    (17, 4096, 11008, 64, "mfma"),    # ... or from M = 17 with G = 64
    (12, 8192, 28672, 128, "skinny"),  # 32-column blocks at long K up to M = 16
    (32, 8192, 28672, 128, "mfma"),    # ... not beyond
    (9, 4096, 4096, 128, "skinny"),
    (64, 4096, 11008, 64, "mfma"),
    (24, 4096, 4096, 128, "skinny"),  # 8 MiB of weights: skinny up to M = 32
    (65, 4096, 4096, 128, "mfma"),
    (4096, 14336, 4096, 128, "mfma"),
    (16, 4096, 4096, 32, "skinny"),
    (32, 6144, 4096, 128, "skinny"),  # 32-column blocks beat the streamed tiles to N = 8192
    (16, 14336, 4096, 128, "skinny"),  # ... and to N = 16384 for M <= 16
    (32, 14336, 4096, 128, "skinny"),  # 16-row groups on 64-column blocks, two rounds
    (48, 14336, 4096, 128, "mfma"),    # ... not three
    (16, 28672, 4096, 128, "skinny"),
    (24, 28672, 4096, 128, "mfma"),
    (4, 8192, 28672, 128, "skinny"),   # long K: whole K per workgroup
    (16, 4098, 4096, 32, "skinny"),   # any N
    (1, 4098, 4096, 128, "skinny"),   # N % 4 != 0: the 16-column kernel takes any N
    (1, 4098, 4096, 16, "simt"),      # ... but needs G % 32 == 0
    (64, 4096, 4096, 16, "simt"),     # G % 32 != 0 beyond the GEMV's M range
    (1, 8, 8, 4, "simt"),             # G = 4: words straddle groups
])
def test_planner_kernel_choice(M, N, K, G, kernel):
    from w4a16 import _lib

    p = _lib.plan(M, N, K, G)
    assert _lib.KERNEL_NAMES[p.kernel] == kernel
    assert p.grid_x >= 1 and p.grid_y >= 1
    if kernel == "skinny":
        # M > 16 with K <= 4096 and few enough blocks: one 16-row group per
        # workgroup (test_planner_skinny_row_groups); 13 <= M <= 16 two 8-row
        # groups, except M = 16 with 1024 < K <= 4096 (the whole 16-row tile,
        # its activations staged); else 32-column blocks (cfg 2) where
        # 16-column ones outnumber the CUs (256 on MI355X, also the library's
        # value without a device), M <= 32 and N even; else 16-column blocks
        g = (M + 15) // 16
        rg = (M > 16 and K <= 4096 and
              (N % 2 == 0 and (N + 31) // 32 * g <= 256 or
               N % 4 == 0 and (N + 63) // 64 * g <= (512 if G % 64 == 0 or K > 1024 else 256)))
        rg8 = (13 <= M <= 16 and N % 2 == 0 and (N + 31) // 32 * 2 <= 256 and
               (K <= 4096 or G % 128 == 0 and K <= 16384) and
               not (M == 16 and 1024 < K <= 4096))
        quad = M <= 16 and N % 4 == 0 and (G % 64 == 0 or K <= 4096) and (N + 63) // 64 > 128
        wide = (N + 15) // 16 > 256 and N % 2 == 0 and M <= 32
        if rg or rg8:
            want = (2, 32) if (N + 31) // 32 * g <= 256 or rg8 else (3, 64)
        else:
            want = (3, 64) if quad else (2, 32) if wide else (0, 16)
        assert (p.tile_cfg, p.tile_n) == want, (M, N)
        assert p.tile_m == (16 if rg else 8 if rg8 else g * 16), (M, N)


def _rules(M, N, K, G):
    """The GEMV rules' plan for a decode shape (the measured table decides the
    automatic plan inside its grid; a forced GEMV plan takes the rules)."""
    from w4a16 import _lib

    return _lib.plan(M, N, K, G, _lib.KERNEL_GEMV, 0)


def test_planner_decode_64_column_band():
    """M <= 2 where 32-column blocks would outnumber the CUs (256 without a
    device) but 64-column ones would not (8192 < N < 16384), K > 2048:
    64-column blocks, unsplit -- the skinny kernel's for K <= 4096 with
    G % 128 == 0, else the GEMV with staged activations and MFMA dot products
    (cfg 7); K = 2048 takes the skinny kernel's 64-column blocks.  (Inside the
    measured table's grid the table decides; the GEMV rules are checked
    through forced GEMV plans there.)"""
    from w4a16 import _lib

    for M, N, K, G, kern, cfg in ((1, 11008, 4096, 128, "skinny", 3), (2, 14336, 4096, 128, "skinny", 3),
                                  (1, 11008, 4096, 32, "gemv", 7), (1, 10240, 8192, 64, "gemv", 7),
                                  (2, 11008, 8192, 64, "gemv", 7)):
        p = _lib.plan(M, N, K, G) if kern == "skinny" else _rules(M, N, K, G)
        assert (_lib.KERNEL_NAMES[p.kernel], p.tile_cfg, p.tile_n, p.split_k) == (kern, cfg, 64, 1), (M, N, K, G)
    p = _lib.plan(1, 11008, 2048, 64)          # K <= 2048: the skinny kernel's blocks
    assert (_lib.KERNEL_NAMES[p.kernel], p.tile_n) == ("skinny", 64)
    # at the band's edges: N = 8192 (256 32-column blocks) and N = 16384 (256
    # 64-column blocks) keep their plans
    assert _rules(1, 8192, 8192, 64).tile_n == 32
    assert (_rules(1, 16384, 4096, 64).tile_n, _rules(1, 16384, 4096, 64).tile_cfg) == (64, 7)


def test_planner_gemv_split_rule():
    """The automatic decode plan splits K four ways only for long K (>= 8192) with
    fewer 16-column blocks than CUs (measured faster there, slower at K = 4096
    and neutral at one block per CU); a forced split gives every split at least
    one packed row and sizes the fp32 partials."""
    from w4a16 import _lib

    lib = _lib.load()
    for N in (512, 1024, 4096, 6144, 28672):
        p = _lib.plan(1, N, 4096, 128, _lib.KERNEL_GEMV, 0)
        assert _lib.KERNEL_NAMES[p.kernel] == "gemv"
        assert p.split_k == 1 and p.workspace_bytes == 0
        assert p.tile_n in (16, 32, 64, 128, 256)
        assert p.tile_cfg in (1, 2, 4, 5, 7)
        assert lib.w4a16_gemm_workspace_bytes(1, N, 4096, 128) == 0
    assert _rules(1, 28672, 4096, 64).tile_n == 128
    for M, N, K in ((1, 1024, 14336), (2, 512, 8192), (2, 1024, 28672)):
        p = _lib.plan(M, N, K, 128)
        assert _lib.KERNEL_NAMES[p.kernel] == "gemv" and p.split_k == 4
        assert p.workspace_bytes == 4 * M * N * 4
        assert lib.w4a16_gemm_workspace_bytes(M, N, K, 128) == p.workspace_bytes
    # long rows on 32 .. 223 64-column blocks: MFMA dot products, K split to
    # reach 7/8 of the CUs (power of two, at most 8) -- the rules (inside the
    # measured table's grid the table may pick another measured plan)
    for M, N, K, split in ((1, 8192, 28672, 2), (1, 4096, 28672, 4), (1, 2048, 28672, 8),
                           (2, 2048, 28672, 8), (2, 4096, 14336, 4), (2, 8192, 28672, 2)):
        p = _rules(M, N, K, 128)
        assert (p.tile_n, p.tile_cfg, p.split_k) == (64, 7, split), (M, N, K)
        assert p.workspace_bytes == split * M * N * 4
        assert lib.w4a16_gemm_workspace_bytes(M, N, K, 128) == p.workspace_bytes
    for M, N, K in ((1, 4096, 14336), (1, 8192, 8192), (1, 1024, 28672), (3, 8192, 28672)):
        p = _rules(M, N, K, 64)                      # shorter rows, too few blocks, M > 2
        assert p.tile_cfg != 7 or p.split_k == 1, (M, N, K)
    assert _rules(1, 28672, 14336, 64).split_k == 1      # enough column blocks
    assert _rules(1, 4096, 14336, 64).split_k == 1       # one block per CU
    for split in (2, 3, 7, 600):
        p = _lib.plan(2, 1024, 4096, 128, _lib.KERNEL_GEMV, split)
        rows = -(-512 // p.split_k)
        assert 1 < p.split_k <= 512
        assert (p.split_k - 1) * rows < 512        # every split owns at least one row
        assert p.workspace_bytes == p.split_k * 2 * 1024 * 4
    p1 = _lib.plan(1, 1024, 4096, 128, _lib.KERNEL_GEMV, 1)
    assert p1.split_k == 1 and p1.workspace_bytes == 0


def test_planner_gemv_blocks_and_waves():
    """Decode block, wave and activation-staging rules (measured on MI355X): on
    16/32-column blocks the activations are read directly with 16 waves at
    M = 1 for any K (but 8 on 16-column blocks with 2048 < K <= 4096) and at
    M = 2 up to 8192 rows per split, else 8; 32-column
    blocks where 16-column ones would leave every CU between one and two blocks
    (K < 8192 only); activations staged in LDS for M <= 2 on 64-column blocks
    and on 128-column blocks where those give 7/8 of the CUs one each (cfg 7:
    8 waves, dot products on the matrix cores) and on 256-column blocks (cfg
    4), one chunk, no split."""
    from w4a16 import _lib

    p = _rules(1, 4096, 4096, 64)            # C2: 256 blocks of 16 (256 CUs), 8 waves
    assert (p.tile_n, p.tile_cfg) == (16, 1)
    p = _rules(2, 4096, 4096, 64)            # ... 16 at M = 2
    assert (p.tile_n, p.tile_cfg) == (16, 2)
    p = _lib.plan(1, 4096, 2048, 128, _lib.KERNEL_GEMV, 0)   # ... and at K = 2048
    assert (p.tile_n, p.tile_cfg) == (16, 2)
    assert _lib.KERNEL_NAMES[_lib.plan(1, 4096, 2048, 64).kernel] == "skinny"   # (planned there)
    p = _lib.plan(1, 6144, 4096, 128, _lib.KERNEL_GEMV, 0)   # 384 blocks of 16 -> 192 of 32
    assert (p.tile_n, p.tile_cfg) == (32, 2)
    p = _lib.plan(2, 6144, 4096, 128, _lib.KERNEL_GEMV, 0)
    assert (p.tile_n, p.tile_cfg) == (32, 2)
    p = _rules(1, 6144, 14336, 64)            # ... at any K, unsplit, 16 waves
    assert (_lib.KERNEL_NAMES[p.kernel], p.tile_n, p.tile_cfg, p.split_k) == ("gemv", 32, 2, 1)
    p = _rules(1, 6144, 28672, 64)            # ... even past the long-row split's K
    assert (p.tile_n, p.tile_cfg, p.split_k) == (32, 2, 1)
    p = _rules(1, 8192, 28672, 64)           # not at N = 8192 (256 blocks of 32)
    assert (p.tile_n, p.tile_cfg, p.split_k) == (64, 7, 2)
    # 128-column blocks, unsplit, where 64-column ones would take more than one
    # round (N > 16384) and 128-column ones not; N = 16384 keeps one round of 64
    for N, K in ((16896, 4096), (20480, 8192), (20480, 28672), (32768, 4096)):
        p = _rules(1, N, K, 64)
        assert (p.tile_n, p.tile_cfg, p.split_k) == (128, 7, 1), (N, K)
    assert _rules(1, 16384, 4096, 64).tile_n == 64
    p = _rules(2, 4096, 10240, 64)           # long rows at M = 2: 8 waves
    assert p.tile_cfg == 1
    p = _rules(2, 4096, 14336, 64)           # ... longer: MFMA dots, split K
    assert (p.tile_n, p.tile_cfg, p.split_k) == (64, 7, 4)
    p = _rules(1, 4096, 14336, 64)           # ... 16 at M = 1, direct
    assert p.tile_cfg == 2
    p = _rules(1, 16384, 4096, 64)           # 64-column blocks: 8 waves, staged, MFMA dots
    assert (p.tile_n, p.tile_cfg) == (64, 7)
    p = _rules(1, 28672, 4096, 64)           # 224 blocks of 128: 8 waves, MFMA dots
    assert (p.tile_n, p.tile_cfg, p.split_k) == (128, 7, 1)
    p = _rules(2, 28672, 8192, 64)
    assert (p.tile_n, p.tile_cfg, p.split_k) == (128, 7, 1)
    p = _rules(1, 65536, 4096, 64)           # 256-column blocks: dot2, staged
    assert (p.tile_n, p.tile_cfg) == (256, 4)
    p = _lib.plan(3, 28672, 8192, 128, _lib.KERNEL_GEMV, 0)   # M > 2 keeps 64-column blocks
    assert (p.tile_n, p.tile_cfg) == (64, 1)
    p = _rules(1, 4096, 8192, 64)            # shorter rows: direct reads
    assert p.tile_cfg == 2
    p = _rules(1, 8192, 28672, 64)           # C5 down-proj: MFMA dots, split 2
    assert (p.tile_n, p.tile_cfg, p.split_k) == (64, 7, 2)
    p = _lib.plan(1, 8192, 28672, 128, _lib.KERNEL_GEMV, 1)   # unsplit: 16 waves, direct
    assert (p.tile_n, p.tile_cfg) == (32, 2)
    p = _lib.plan(2, 8192, 28672, 128, _lib.KERNEL_GEMV, 1)   # ... 8 waves at M = 2
    assert (p.tile_n, p.tile_cfg) == (32, 1)
    p = _rules(2, 1024, 8192, 64)            # split 4: 2048 rows per split
    assert p.split_k == 4 and p.tile_cfg == 2


def _decode_table():
    """Entries of csrc/decode_table.inc: (G class, M, K, N, kernel, cfg, cols, rows, split)."""
    path = os.path.join(ROOT, "w4a16-dequant-fused-matmul-kernel_amd", "csrc", "decode_table.inc")
    rows = []
    for line in open(path):
        m = re.match(r"\{(\d+)" + r", (\d+)" * 10 + r"\},", line)
        if m:
            rows.append(tuple(int(v) for v in m.groups()[:9]))
    return rows


def test_planner_decode_table():
    """M <= 2 inside a group-size class's measured grid (class 128: G % 128 ==
    0; 64: G % 64 == 0; 32: the other G % 32 == 0): the automatic plan is the
    grid's fastest plan (csrc/decode_table.inc) at every grid point and the
    nearest grid point's in (log2 K, log2 N) between them, for any G of the
    class; shapes outside the grid follow the rules."""
    import math

    from w4a16 import _lib

    table = _decode_table()
    classes = sorted({r[0] for r in table})
    assert 128 in classes and set(classes) <= {32, 64, 128}
    members = {128: (128, 256), 64: (64, 192), 32: (32, 96)}
    for gc in classes:
        sub = [r[1:] for r in table if r[0] == gc]
        assert len(sub) >= 300 and {r[0] for r in sub} == {1, 2}, gc
        ks, ns = sorted({r[1] for r in sub}), sorted({r[2] for r in sub})
        assert len(sub) == 2 * len(ks) * len(ns), "a full grid per M"
        kmin, kmax, nmin, nmax = ks[0], ks[-1], ns[0], ns[-1]

        def expect(M, K, N):
            return min((r for r in sub if r[0] == M),
                       key=lambda r: math.log2(K / r[1]) ** 2 + math.log2(N / r[2]) ** 2)

        def check(M, K, N, G):
            p = _lib.plan(M, N, K, G)
            if K * N // 2 >= 1 << 31:
                # weights past the vector kernels' 2 GiB limit: SIMT, whatever
                # the table holds there (its 0-us entries serve fitting shapes)
                assert p.kernel == _lib.KERNEL_SIMT, (G, M, K, N, p.as_dict())
                return
            e = expect(M, K, N)
            kern, cfg, cols, rows, split = e[3:8]
            assert p.kernel == kern and p.tile_cfg == cfg, (G, M, K, N, e, p.as_dict())
            if kern == _lib.KERNEL_GEMV:
                assert (p.tile_n, p.split_k) == (cols, split), (G, M, K, N, e, p.as_dict())
                assert p.workspace_bytes == (split * M * N * 4 if split > 1 else 0)
                assert p.grid_x == -(-N // cols) * split
            else:
                assert (p.tile_n, p.tile_m, p.split_k) == (cols, rows, 1), (G, M, K, N, e)

        for r in sub:
            if all(r[1] % G == 0 for G in members[gc]):
                for G in members[gc]:
                    check(r[0], r[1], r[2], G)
            else:
                check(r[0], r[1], r[2], gc)
        rng = np.random.default_rng(5)
        for _ in range(300):
            M = int(rng.integers(1, 3))
            G = members[gc][int(rng.integers(0, 2))]
            K = int(rng.integers(-(-kmin // G), kmax // G + 1)) * G
            N = int(rng.integers(nmin // 4, nmax // 4 + 1)) * 4
            if kmin <= K <= kmax:
                check(M, K, N, G)
    # outside the grid's domain the rules decide alike for every group size:
    # N or K outside the grid
    sub = [r[1:] for r in table if r[0] == 128]
    kmin, kmax = min(r[1] for r in sub), max(r[1] for r in sub)
    nmin, nmax = min(r[2] for r in sub), max(r[2] for r in sub)
    for M, N, K in ((1, nmin // 2, kmax), (2, nmin, 2 * kmax), (1, 2 * nmax, kmin), (2, nmin, kmin // 2)):
        a, b = _lib.plan(M, N, K, 128).as_dict(), _lib.plan(M, N, K, 64).as_dict()
        assert a == b, (M, N, K, a, b)


def test_planner_small_groups_small_m_long_rows_gemv():
    """G % 64 != 0, M = 3..4, K >= 11008, 3072 <= N <= 4096: the GEMV on
    64-column blocks split four ways (measured faster than the skinny kernel
    there); not with larger groups, at K = 8192, M = 5 or N = 5120."""
    from w4a16 import _lib

    for M, K in ((3, 11008), (4, 14336), (3, 28672), (4, 20480)):
        p = _lib.plan(M, 4096, K, 32).as_dict()
        assert (p["kernel_name"], p["tile_cfg"], p["tile_n"], p["split_k"]) == ("gemv", 1, 64, 4), (M, K)
        assert p["workspace_bytes"] == 4 * M * 4096 * 4
    for M, N, K, G in ((3, 4096, 11008, 64), (4, 4096, 14336, 128), (3, 4096, 8192, 32),
                       (5, 4096, 14336, 32), (3, 5120, 13824, 32)):
        p = _lib.plan(M, N, K, G).as_dict()
        assert not (p["kernel_name"] == "gemv" and p["tile_n"] == 64 and p["split_k"] == 4), (M, N, K, G, p)


def test_planner_lm_head_small_batch_split():
    """32-row streamed tiles past one round of two per CU (512 without a
    device): split two ways where that packs the tiles into fewer rounds."""
    from w4a16 import _lib

    for M, K, N in ((16, 4096, 151936), (32, 3584, 152064)):
        p = _lib.plan(M, N, K, 128).as_dict()
        assert (p["tile_cfg"], p["split_k"], p["grid_x"]) == (12, 2, 1188), (M, K, N)
    p = _lib.plan(16, 128256, 8192, 128).as_dict()             # 501 tiles: one round
    assert (p["tile_cfg"], p["split_k"]) == (12, 1)
    assert _lib.plan(64, 151936, 4096, 128).split_k == 1     # 64-row tiles stay unsplit


def test_planner_small_batch_wide_weights_stream():
    """4 <= M <= 64 on large enough, wide weights takes the streamed prefill
    kernel with 32-row (M <= 32, cfg 12) or 64-row tiles (cfg 13), split along K
    (>= 8 k-steps per split) for one workgroup per CU where up to 64 64-row
    tiles fill 3/4 of the CUs that way, else for close to two per CU; narrow N, small
    weights, or N <= 8192 (16384 for M <= 16) with M <= 32 stay on the skinny
    kernel (or the GEMV for M <= 3)."""
    from w4a16 import _lib

    for M, N, K, cfg, s in ((32, 28672, 4096, 12, 4), (24, 28672, 8192, 12, 4),
                            (17, 28672, 8192, 12, 4), (64, 28672, 8192, 13, 4),
                            (48, 14336, 4096, 13, 4), (64, 4096, 16384, 13, 16),
                            (32, 22016, 4096, 12, 6), (32, 10240, 8192, 12, 11),
                            # 64-row tiles whose one-per-CU split would leave < 10
                            # k-steps take 32-row tiles one per CU
                            (64, 5120, 5120, 12, 5), (64, 4096, 11008, 13, 15),
                            # 64-column skinny blocks past two per CU at M > 8
                            (16, 57344, 8192, 12, 2), (12, 57344, 8192, 12, 2)):
        p = _lib.plan(M, N, K, 128)
        rows = 32 if cfg == 12 else 64
        assert _lib.KERNEL_NAMES[p.kernel] == "mfma" and p.tile_cfg == cfg, (M, N, K)
        assert (p.tile_m, p.tile_n) == (rows, 256)
        assert p.split_k == s and p.workspace_bytes >= s * M * N * 4, (M, N, K, p.split_k)
        assert p.grid_x == s * ((N + 255) // 256) * ((M + rows - 1) // rows)
    for M, N, K in ((16, 4096, 4096), (16, 4096, 14336), (24, 4096, 4096), (16, 6144, 4096),
                    (8, 57344, 8192), (16, 28672, 4096),
                    (9, 8192, 8192), (16, 28672, 4160)):      # K % 256 != 0: no streamed kernel
        assert _lib.KERNEL_NAMES[_lib.plan(M, N, K, 64).kernel] == "skinny", (M, N, K)
    # up to N = 8192 (N = 16384 for M <= 16) the skinny kernel's 32-column
    # blocks beat the streamed tiles, long K included up to M = 16, K <= 8192
    # beyond
    for M, N, K in ((16, 8192, 28672), (4, 8192, 28672), (17, 8192, 8192), (20, 8192, 6144)):
        p = _lib.plan(M, N, K, 128)
        assert _lib.KERNEL_NAMES[p.kernel] == "skinny" and (p.tile_cfg, p.tile_n) == (2, 32), (M, N, K)
        assert p.grid_x == N // 32
    for M, N, K in ((17, 8192, 14336), (24, 8192, 28672)):
        assert _lib.KERNEL_NAMES[_lib.plan(M, N, K, 128).kernel] == "mfma", (M, N, K)
    # M <= 16 with more than 128 64-column blocks: 64-column skinny blocks,
    # with G % 64 == 0 or K <= 4096
    for M, N, K, G in ((16, 28672, 4096, 128), (8, 28672, 8192, 128), (4, 14336, 4096, 128),
                       (8, 28672, 8192, 64), (8, 14336, 4096, 32)):
        p = _lib.plan(M, N, K, G)
        assert _lib.KERNEL_NAMES[p.kernel] == "skinny" and (p.tile_cfg, p.tile_n) == (3, 64), (M, N, K, G)
    # ... the 32-column blocks' rule was measured with G = 128; smaller groups
    # keep the streamed tiles there, as does G = 32 with K > 4096 on 64-column
    # blocks
    for M, N, K, G in ((16, 8192, 28672, 32), (16, 8192, 28672, 64), (8, 28672, 8192, 32)):
        p = _lib.plan(M, N, K, G)
        assert _lib.KERNEL_NAMES[p.kernel] == "mfma" and p.tile_cfg == 12, (M, N, K, G)


def test_planner_skinny_row_groups():
    """17 <= M <= 64: skinny blocks with one 16-row group per workgroup
    (tile_m 16, ceil(M / 16) workgroups per column block) where the workgroups
    stay near the CU count: 32-column blocks while they fit one round, else
    64-column blocks up to two rounds for K <= 4096 (one round at G = 32 with
    K <= 1024);
    with longer K only two row groups on one round, 32-column blocks up to
    K = 16384 (K = 8192 below G = 128) and 64-column ones from M = 24 up to
    K = 8192 with G % 128 == 0."""
    from w4a16 import _lib

    for M, N, K, G, cfg in ((32, 4096, 4096, 128, 2), (17, 4096, 4096, 128, 2),
                            (24, 6144, 4096, 128, 3), (40, 4096, 4096, 128, 3),
                            (64, 4096, 4096, 128, 3), (64, 8192, 4096, 128, 3),
                            (32, 14336, 4096, 128, 3), (32, 4096, 14336, 128, 2),
                            (17, 4096, 14336, 128, 2), (24, 8192, 8192, 128, 3),
                            (32, 4096, 16384, 128, 2), (32, 4096, 4096, 64, 2),
                            (32, 4096, 4096, 32, 2), (48, 4096, 4096, 32, 3),
                            (64, 8192, 4096, 64, 3), (32, 4096, 8192, 64, 2),
                            (24, 4096, 8192, 32, 2), (48, 6144, 4096, 32, 3),
                            (64, 6144, 4096, 32, 3), (32, 14336, 4096, 32, 3)):
        p = _lib.plan(M, N, K, G)
        assert _lib.KERNEL_NAMES[p.kernel] == "skinny", (M, N, K, G)
        cols = 64 if cfg == 3 else 32
        assert (p.tile_cfg, p.tile_m, p.tile_n) == (cfg, 16, cols), (M, N, K, G)
        assert p.grid_x == (N + cols - 1) // cols * ((M + 15) // 16) and p.split_k == 1
    # 13 <= M <= 16: two 8-row groups on 32-column blocks that fit the CUs, up
    # to K = 4096 at any G and K = 16384 with G % 128 == 0 ...
    for M, N, K, G in ((15, 4096, 4096, 128), (13, 4096, 14336, 128), (16, 4096, 14336, 128),
                       (16, 4096, 1024, 64), (14, 4096, 4096, 32)):
        p = _lib.plan(M, N, K, G)
        assert _lib.KERNEL_NAMES[p.kernel] == "skinny", (M, N, K, G)
        assert (p.tile_cfg, p.tile_m, p.tile_n, p.grid_x) == (2, 8, 32, N // 32 * 2), (M, N, K, G)
    # ... except M = 16 with 1024 < K <= 4096: the whole 16-row tile (its
    # activations staged in LDS), 16-column blocks at N = 4096
    for G in (128, 64, 32):
        p = _lib.plan(16, 4096, 4096, G)
        assert (p.tile_cfg, p.tile_m, p.tile_n, p.grid_x) == (0, 16, 16, 256), G
    # not: wide N, three or more row groups with K > 4096, M = 17 on 64-column
    # blocks with K > 4096, long rows (32-column blocks beyond K = 16384,
    # 64-column ones beyond 8192), smaller groups with longer K or (G = 32)
    # 64-column blocks beyond one round, M <= 12, M <= 16 on more blocks
    for M, N, K, G in ((32, 28672, 4096, 128), (48, 14336, 4096, 128), (48, 8192, 8192, 128),
                       (64, 4096, 14336, 128), (17, 8192, 8192, 128), (32, 8192, 28672, 128),
                       (32, 4096, 28672, 128), (24, 4096, 20480, 128), (32, 6144, 14336, 128),
                       (16, 4096, 28672, 128), (32, 4096, 14336, 64), (32, 6144, 8192, 64),
                       (16, 4096, 14336, 64), (48, 14336, 4096, 32),
                       (12, 4096, 4096, 128), (16, 6144, 4096, 128)):
        p = _lib.plan(M, N, K, G)
        assert not (_lib.KERNEL_NAMES[p.kernel] == "skinny" and p.tile_m < (M + 15) // 16 * 16), (M, N, K, G)
    # a forced skinny plan takes the same row groups
    p = _lib.plan(32, 4096, 4096, 128, _lib.KERNEL_SKINNY, 0)
    assert (p.tile_cfg, p.tile_m) == (2, 16)


def test_empty_shapes_plan_simt_for_every_family():
    """M, N or K = 0 plans the SIMT kernel whatever family is forced (nothing is
    launched for M = 0 / N = 0; K = 0 writes zeros with it).  Forcing the
    MFMA family on an empty shape once divided by its zero tile count
    (SIGFPE in the planner, found by the host-side AddressSanitizer run)."""
    from w4a16 import _lib

    for M, N, K in ((0, 0, 0), (0, 64, 64), (4, 0, 64), (4, 64, 0), (300, 0, 4096)):
        for kernel in (0, _lib.KERNEL_GEMV, _lib.KERNEL_MFMA, _lib.KERNEL_SIMT,
                       _lib.KERNEL_SKINNY):
            for split in (0, 1, 4):
                p = _lib.plan(M, N, K, 32, kernel, split)
                assert p.kernel == _lib.KERNEL_SIMT and p.split_k == 1, (M, N, K, kernel, split)
                assert p.workspace_bytes == 0
    with pytest.raises(RuntimeError):
        _lib.plan(4, 64, 64, 32, 9, 0)       # no such family


def test_planner_prefill_split_k():
    from w4a16 import _lib

    # 128 x 256 tiles that fit one per CU (256 without a device): two k-slices
    # per workgroup (cfg 14), split for about one workgroup per CU.  C5
    # down-projection at M = 256: 64 tiles -> 4 splits; the up-projection's 224
    # tiles -> none; M = 128 (112 tiles) -> 2
    p = _lib.plan(256, 8192, 28672, 128)
    assert _lib.KERNEL_NAMES[p.kernel] == "mfma" and p.tile_cfg == 14
    assert p.split_k == 4 and p.grid_x == 256
    assert p.workspace_bytes >= p.split_k * 256 * 8192 * 4
    q = _lib.plan(256, 28672, 8192, 128)
    assert (q.tile_cfg, q.split_k, q.workspace_bytes) == (14, 1, 0)
    assert (_lib.plan(128, 28672, 8192, 128).tile_cfg, _lib.plan(128, 28672, 8192, 128).split_k) == (14, 2)
    assert _lib.plan(512, 14336, 4096, 128).tile_cfg == 14      # C4 M = 512: 224 tiles
    # long rows (K >= 16384) on fewer tiles than CUs: cfg 11 split along K --
    # from 86 tiles the most of 8 / 4 / 2 splits within three workgroups per
    # CU, from K = 24576 with more than 64 tiles about two per CU; 64 tiles
    # and shorter rows below 86 tiles keep cfg 14
    for M, N, K, cfg, split in ((384, 8192, 28672, 11, 8), (512, 8192, 28672, 11, 4),
                                (768, 8192, 28672, 11, 4), (768, 8192, 16384, 11, 4),
                                (768, 10240, 20480, 11, 2), (384, 6144, 28672, 11, 7),
                                (512, 5120, 28672, 11, 6), (256, 8192, 28672, 14, 4),
                                (512, 5120, 16384, 14, 3)):
        p = _lib.plan(M, N, K, 128)
        assert (p.tile_cfg, p.split_k) == (cfg, split), (M, N, K, p.tile_cfg, p.split_k)
    # ... K = N = 4096 at M = 128: 64-row tiles, 6 splits of >= 10 k-steps
    p = _lib.plan(128, 4096, 4096, 128)
    assert (p.tile_cfg, p.split_k) == (13, 6)
    # G = 32 (a scale / zero load per half-step): the same cfg 14 rules, except
    # long rows from 60 tiles and 80..128 tiles past K = 4096, which take cfg 11
    # split for about two workgroups per CU
    p = _lib.plan(256, 8192, 28672, 32)
    assert (p.tile_cfg, p.split_k, p.grid_x) == (11, 8, 512)
    assert (_lib.plan(256, 8192, 28672, 128).tile_cfg, _lib.plan(256, 8192, 28672, 128).split_k) == (14, 4)
    assert (_lib.plan(256, 28672, 8192, 32).tile_cfg, _lib.plan(256, 28672, 8192, 32).split_k) == (14, 1)
    p = _lib.plan(512, 5120, 5120, 32)                          # 80 tiles
    assert (p.tile_cfg, p.split_k) == (11, 5)
    assert _lib.plan(512, 5120, 5120, 128).tile_cfg == 14
    # splits never take the streamed tiles past two workgroups per CU (512
    # without a device): 296 tiles stay unsplit, 148 64-row tiles split 3 ways
    p = _lib.plan(256, 37888, 3584, 128)
    assert (p.tile_cfg, p.split_k, p.grid_x) == (11, 1, 296)
    p = _lib.plan(64, 37888, 3584, 128)
    assert (p.tile_cfg, p.split_k, p.grid_x) == (13, 3, 444)
    # a forced split that two k-slices (8-step units) cannot honour: cfg 11
    p = _lib.plan(512, 1028, 2048, 64, _lib.KERNEL_MFMA, 3)
    assert (p.tile_cfg, p.split_k) == (11, 3)
    p = _lib.plan(512, 1028, 2048, 64, _lib.KERNEL_MFMA, 2)
    assert (p.tile_cfg, p.split_k) == (14, 2)
    # 64 < M <= 256 on small layers: 64-row tiles (cfg 13) where cfg 14's
    # slices would hold <= 4 k-steps, split for ~a workgroup per CU with >= 10
    # k-steps per split ...
    for M, N, K, split in ((96, 4096, 4096, 6), (192, 4096, 4096, 4), (256, 4096, 4096, 4),
                           (128, 4096, 2048, 4)):
        p = _lib.plan(M, N, K, 128)
        assert (p.tile_cfg, p.tile_m, p.split_k) == (13, 64, split), (M, N, K)
        assert p.grid_x == split * (N // 256) * ((M + 63) // 64)
    # ... or unsplit with K <= 2048 where the tiles give half the CUs one each
    for M in (128, 192, 256):
        p = _lib.plan(M, 16384, 2048, 128)
        assert (p.tile_cfg, p.split_k, p.workspace_bytes) == (13, 1, 0), M
    # ... and at M <= 128 with 86..128 64-row tiles (K > 2048), split for
    # about two workgroups per CU
    for M, N, K, split in ((128, 12288, 4096, 4), (128, 15360, 5120, 4), (96, 14336, 4096, 4)):
        p = _lib.plan(M, N, K, 128)
        assert (p.tile_cfg, p.tile_m, p.split_k) == (13, 64, split), (M, N, K)
        assert p.grid_x == split * (N // 256) * 2
    # ... not with longer slices, more or fewer tiles (M > 256: the rule below)
    for M, N, K in ((128, 8192, 8192), (128, 27648, 5120), (128, 10240, 8192)):
        assert _lib.plan(M, N, K, 128).tile_cfg == 14, (M, N, K)
    # 64-row tiles split for about two workgroups per CU (>= 10 k-steps each)
    # where the last 128-row tile is at most half used (128 < M <= 192, at most
    # 160 64-row tiles) and for few tiles of long rows (M <= 128, K >= 8192, at
    # most 40 tiles); any G
    for M, N, K, split in ((192, 5120, 5120, 7), (160, 10240, 8192, 4), (192, 4096, 11008, 9),
                           (192, 6144, 4096, 6), (96, 4096, 11008, 15), (128, 4096, 14336, 14),
                           (128, 5120, 13824, 11)):
        for G in (128, 64, 32):
            p = _lib.plan(M, N, K, G)
            assert (p.tile_cfg, p.tile_m, p.split_k) == (13, 64, split), (M, N, K, G)
            assert p.grid_x == split * (N // 256) * ((M + 63) // 64)
            assert p.workspace_bytes == split * M * N * 4
    # ... not where the splits would hold fewer than 10 k-steps (K = N = 4096:
    # the one-per-CU rule above), nor on more tiles
    assert (_lib.plan(192, 4096, 4096, 128).tile_cfg, _lib.plan(192, 4096, 4096, 128).split_k) == (13, 4)
    assert _lib.plan(192, 15360, 5120, 128).tile_cfg == 14      # 180 64-row tiles
    p = _lib.plan(192, 5120, 28672, 128)                        # long rows too
    assert (p.tile_cfg, p.split_k) == (13, 8)
    # 256 < M <= 512, K <= 12288: 64-row tiles split for about two workgroups
    # per CU where the busiest CU's work falls to 5/6 of the 128-row plan's or
    # less, or stays level on splits of at most 20 k-steps
    for M, N, K, split in ((320, 12288, 4096, 2), (288, 6144, 4096, 4), (320, 4096, 4096, 6),
                           (320, 5120, 5120, 5), (288, 8192, 8192, 3), (320, 22016, 4096, 1),
                           (320, 11008, 4096, 2), (384, 4096, 4096, 4), (448, 4096, 4096, 4),
                           (384, 5120, 5120, 4), (320, 4096, 11008, 6)):
        p = _lib.plan(M, N, K, 128)
        assert (p.tile_cfg, p.tile_m, p.split_k) == (13, 64, split), (M, N, K)
        assert p.grid_x == split * ((N + 255) // 256) * ((M + 63) // 64)
        assert p.grid_x <= 512
    # ... not on level work with longer splits, past two workgroups per CU,
    # on long rows, or past M = 512
    for M, N, K in ((320, 10240, 8192), (320, 15360, 5120), (320, 28672, 4096),
                    (384, 22016, 4096), (320, 4096, 13824),
                    (320, 14336, 4096), (384, 12288, 4096), (640, 4096, 4096)):
        assert _lib.plan(M, N, K, 128).tile_cfg in (11, 14), (M, N, K)
    # G = 32: against the 128-row cfg 11 split of 80..128 tiles as well
    p = _lib.plan(320, 8192, 8192, 32)
    assert (p.tile_cfg, p.split_k) == (13, 3)
    # smaller groups: the few-tile case up to 64 tiles, K <= 16384
    for G in (64, 32):
        p = _lib.plan(128, 8192, 8192, G)
        assert (p.tile_cfg, p.tile_m, p.split_k) == (13, 64, 8), G
    assert _lib.plan(128, 8192, 8192, 128).tile_cfg == 14
    assert _lib.plan(128, 8192, 28672, 64).tile_cfg == 14
    # more tiles than CUs: cfg 11
    p = _lib.plan(1024, 14336, 4096, 128)
    assert (p.tile_cfg, p.split_k) == (11, 1)
    assert _lib.plan(2048, 14336, 4096, 128).split_k == 1    # 896 tiles
    # large M: no split, no workspace
    p = _lib.plan(4096, 14336, 4096, 128)
    assert p.split_k == 1 and p.workspace_bytes == 0 and p.tile_cfg == 11
    # K % 256 != 0: the register-staged kernel of the same tiles
    p = _lib.plan(4096, 14336, 4160, 64)
    assert p.split_k == 1 and p.tile_cfg == 7
    # a forced split on a tile configuration without split-K support is refused
    q = _lib.plan(256, 8192, 28672, 128, _lib.KERNEL_MFMA, 4)
    q.tile_cfg = 6
    a = ctypes.c_void_p(1 << 12)
    lib = _lib.load()
    assert lib.w4a16_gemm_f16_planned(ctypes.byref(q), a, a, a, a, NULL, a, 256, 8192, 28672,
                                      128, a, 1 << 30, NULL) == -5


def test_planner_invariants_over_shape_grid():
    """Every automatic plan over a grid of 36 M x 13 N x 9 K x 3 G (decode to
    prefill, odd and LM-head widths, short and long rows) is well formed: the
    grid is the tile count times the splits, every split holds at least one
    k-block of its kernel, a split plan's workspace holds its fp32 partials
    and the workspace query covers it, an unsplit plan needs none, and each
    family stays within the M it serves."""
    import itertools
    from w4a16 import _lib

    lib = _lib.load()
    Ms = [1, 2, 3, 4, 5, 8, 13, 16, 17, 24, 32, 33, 48, 64, 65, 80, 96, 128, 129, 160, 192,
          200, 256, 257, 288, 320, 384, 448, 512, 513, 640, 768, 1024, 1500, 2048, 4096]
    Ns = [4, 12, 256, 1000, 1028, 4096, 6144, 11008, 14336, 22016, 28672, 57344, 128256]
    Ks = [256, 512, 2048, 4096, 5120, 8192, 11008, 14336, 28672]
    seen = set()
    for M, N, K, G in itertools.product(Ms, Ns, Ks, (32, 64, 128)):
        p = _lib.plan(M, N, K, G)
        name = _lib.KERNEL_NAMES[p.kernel]
        seen.add((name, p.tile_cfg))
        case = (M, N, K, G, name, p.tile_cfg, p.split_k)
        assert p.split_k >= 1 and p.grid_x >= 1 and p.grid_y >= 1, case
        if p.split_k == 1:
            assert p.workspace_bytes == 0, case
        else:
            assert p.workspace_bytes >= p.split_k * M * N * 4, case
        assert lib.w4a16_gemm_workspace_bytes(M, N, K, G) >= p.workspace_bytes, case
        if name == "mfma":
            assert p.grid_x == -(-N // p.tile_n) * -(-M // p.tile_m) * p.split_k, case
            if p.tile_cfg >= 11:
                # streamed tiles: whole 4-step (256-k) blocks per split, and
                # 8-step blocks with the two k-slices of cfg 14
                assert K % 256 == 0 and p.split_k <= K // 256, case
                assert p.tile_cfg != 14 or p.split_k <= max(1, K // 512), case
            if 256 < M <= 512 and p.tile_cfg == 13:
                assert p.grid_x <= 512, case             # at most two workgroups per CU
        elif name == "skinny":
            assert M <= 64 and p.split_k == 1, case
            assert p.grid_x == -(-N // p.tile_n) * -(-M // p.tile_m), case
        elif name == "gemv":
            assert M <= 8 and p.split_k <= K // 8, case
            assert p.grid_x == -(-N // p.tile_n) * p.split_k, case
        else:
            raise AssertionError(f"unexpected kernel for a fitting shape: {case}")
    # the grid reaches every family and the streamed prefill configurations
    for want in (("gemv", 1), ("gemv", 7), ("skinny", 0), ("skinny", 2), ("skinny", 3),
                 ("mfma", 11), ("mfma", 12), ("mfma", 13), ("mfma", 14)):
        assert want in seen, want


def test_planner_forced_kernel_must_fit():
    from w4a16 import _lib

    with pytest.raises(RuntimeError):
        _lib.plan(16, 4096, 4096, 128, _lib.KERNEL_GEMV, 0)   # GEMV takes M <= 8
    with pytest.raises(RuntimeError):
        _lib.plan(64, 4098, 4096, 128, _lib.KERNEL_MFMA, 0)   # MFMA needs N % 4 == 0


# --------------------------------------------------------------------------- #
# Python wrappers: precondition errors before any device work                  #
# --------------------------------------------------------------------------- #
def test_quantize_weight_divisibility_errors():
    """Reference test_quant.py:103-109 (raised before staging to a device)."""
    from w4a16 import quantize_weight

    with pytest.raises(ValueError):
        quantize_weight(torch.randn(100, 16, dtype=torch.float16), group_size=64)
    with pytest.raises(ValueError):
        quantize_weight(torch.randn(96, 16, dtype=torch.float16), group_size=64)
    with pytest.raises(AssertionError):
        quantize_weight(torch.randn(8, 8, 8, dtype=torch.float16), group_size=8)


def test_pack_requires_k_div_8():
    """Reference test_quant.py:50-52."""
    from w4a16 import pack_int4

    with pytest.raises(AssertionError):
        pack_int4(torch.zeros((7, 4), dtype=torch.int32))


def test_w4a16_matmul_requires_device_tensors():
    from w4a16 import w4a16_matmul

    x = torch.zeros(1, 64, dtype=torch.float16)
    qw = torch.zeros(8, 16, dtype=torch.int32)
    s = torch.zeros(2, 16, dtype=torch.float16)
    with pytest.raises(AssertionError):
        w4a16_matmul(x, qw, s, s, 32)


def test_linear_constructor_errors():
    """Reference linear.py:38-41."""
    from w4a16 import W4A16Linear

    with pytest.raises(ValueError):
        W4A16Linear(100, 16)
    with pytest.raises(ValueError):
        W4A16Linear(192, 16, group_size=128)
    m = W4A16Linear(256, 48, group_size=128, bias=True)
    sd = m.state_dict()
    assert list(sd) == ["qweight", "scales", "zeros", "bias"]
    assert sd["qweight"].shape == (32, 48) and sd["qweight"].dtype == torch.int32
    assert sd["scales"].shape == (2, 48) and sd["scales"].dtype == torch.float16
    assert sd["zeros"].shape == (2, 48) and sd["bias"].shape == (48,)
    assert "group_size=128" in repr(m)
    assert W4A16Linear(256, 48, bias=False).bias is None


def test_no_cpu_fallback_without_device(monkeypatch):
    """With no HIP device visible, compute entry points raise instead of running
    anything on the CPU."""
    from w4a16 import quantize_weight, unpack_int4

    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    with pytest.raises(RuntimeError):
        quantize_weight(torch.zeros(64, 8, dtype=torch.float16), 32)
    with pytest.raises(RuntimeError):
        unpack_int4(torch.zeros(8, 8, dtype=torch.int32))


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from w4a16 import _lib

    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "libw4a16.so"))
    with pytest.raises(ImportError):
        _lib.load()


def test_package_exports_reference_names():
    """Reference __init__.py:21-36 names, plus HAS_TRITON (False here)."""
    import w4a16

    for name in ("quantize_weight", "dequantize_weight", "pack_int4", "unpack_int4",
                 "reference_w4a16", "dequant_then_matmul", "fp16_matmul", "w4a16_matmul",
                 "W4A16Linear"):
        assert name in w4a16.__all__ and hasattr(w4a16, name)
    assert w4a16.HAS_TRITON is False and w4a16.HAS_HIP is True
    from w4a16.triton_kernel import w4a16_matmul as alias

    assert alias is w4a16.w4a16_matmul
    from w4a16 import cuda_kernel

    assert set(cuda_kernel.__all__) == {"w4a16_matmul_cuda", "load_cuda_module", "is_available"}


def test_workload_bytes_formula():
    """bench_gemm.py:61-67 bytes and :86 flops at the headline configs."""
    from w4a16 import workloads as wl

    c2 = wl.CONFIGS["C2"][0]
    assert c2.bytes() == 8_929_280
    c4 = [c for c in wl.CONFIGS["C4"] if c.M == 4096][0]
    assert c4.flops() == 2 * 4096 * 14336 * 4096
    assert c4.bytes() == 182_190_080


def test_sampled_columns_cover_every_block():
    """The GPU tests check wide outputs on sampled columns; the sample must hit
    every 16-column block (and hence every 32/64/256-column block and tile) of
    each BASELINE width, at varying lane positions within the block."""
    from _helpers import STRATUM, sample_cols

    for N in (4096, 6144, 8192, 14336, 28672, 4100, 1028):
        cols = sample_cols(N, 128)
        assert cols.min() >= 0 and cols.max() < N
        assert len(np.unique(cols)) == len(cols)
        for width in (STRATUM, 32, 64, 256):
            hit = np.zeros((N + width - 1) // width, bool)
            hit[cols // width] = True
            assert hit.all(), (N, width)
        assert len(np.unique(cols % STRATUM)) == STRATUM, N


def test_library_built_from_these_sources(lib):
    """The library carries the sha256 of the sources it was built from, and it
    equals the hash of the sources in the tree."""
    from w4a16 import _build

    assert lib.w4a16_build_id().decode() == _build.source_hash()


def test_stale_library_refused(monkeypatch):
    """A library built from other sources than those beside it is refused."""
    from w4a16 import _lib

    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setattr(_lib, "_sources_hash", lambda: "0" * 64)
    with pytest.raises(ImportError, match="other sources"):
        _lib.load()

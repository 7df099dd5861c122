"""GPU: row-strided activations and outputs (w4a16_gemm_f16_strided).

x and y as column slices of wider row-major buffers -- the case the reference's
kernel supports through its stride arguments
(w4a16-kernel/src/w4a16/triton_kernel.py:71-75, 94, 127) and its wrapper
refuses (:170-173).  For every kernel path and tile configuration the strided
call must give the same bits as the contiguous call with the same plan (the
kernels only change where rows start), with the padding columns of x holding
NaN, which would show in Y if read, and the padding columns of the output
buffer left untouched.  The contiguous results are pinned to the oracle
by the other GPU tests; here the SIMT fallback for misaligned strides and the
public entry points are also checked against the oracle directly.
"""
from __future__ import annotations

import pytest
import torch

from _helpers import DEV, assert_gemm_close, log, np_
from oracle import w4a16_oracle as O

pytestmark = pytest.mark.gpu

SENTINEL = -7.5


def _case(M, K, N, G, seed):
    from w4a16 import quantize_weight

    g = torch.Generator().manual_seed(seed)
    X = torch.randn(M, K, generator=g).to(torch.float16)
    W = torch.randn(K, N, generator=g).to(torch.float16)
    qw, s, z = quantize_weight(W.to(DEV), G)
    return X.to(DEV), qw, s, z


def _views(X, N, padx, pady, seed):
    """x as the first K columns of [M, K + padx] whose padding holds NaN (any
    read of it reaches Y, even times a zero weight), and an output view of the
    first N columns of [M, N + pady] filled with SENTINEL."""
    M, K = X.shape
    xb = torch.full((M, K + padx), float("nan"), dtype=torch.float16, device=DEV)
    xb[:, :K] = X
    yb = torch.full((M, N + pady), SENTINEL, dtype=torch.float16, device=DEV)
    return xb[:, :K], yb, yb[:, :N]


def _check_same(X, qw, s, z, G, p, padx, pady, bias=None, what=""):
    from w4a16.hip_kernel import w4a16_matmul_planned

    M, N = X.shape[0], qw.shape[1]
    ref = w4a16_matmul_planned(X, qw, s, z, G, p, bias=bias)
    xv, yb, yv = _views(X, N, padx, pady, seed=M + N + padx)
    assert not bool(torch.isnan(ref).any())
    # (torch calls a single row contiguous whatever its stride; the library
    # is then given ldx = K)
    assert M == 1 or (not xv.is_contiguous() and xv.stride(0) == X.shape[1] + padx)
    out = w4a16_matmul_planned(xv, qw, s, z, G, p, bias=bias, out=yv)
    assert out.data_ptr() == yv.data_ptr()
    assert torch.equal(yv, ref), f"strided != contiguous: {what}"
    if pady:
        assert bool((yb[:, N:] == SENTINEL).all()), f"padding columns of y written: {what}"


@pytest.mark.parametrize("M,N", [(1, 4096), (2, 1028), (3, 516), (8, 2052)])
def test_gemv_strided(M, N):
    from w4a16.hip_kernel import plan_for

    K, G = 2048, 128
    X, qw, s, z = _case(M, K, N, G, seed=M)
    cfgs = (1, 2, 4, 5, 6, 7) if M <= 2 else (1,)
    for cfg in cfgs:
        for cols in ((64, 128) if cfg >= 6 else (16, 32, 64, 128, 256)):
            for split in (1, 4):
                p = plan_for(M, N, K, G, "gemv", split)
                p.tile_cfg = cfg
                p.tile_n = cols
                log(f"gemv strided M={M} N={N} cfg={cfg} cols={cols} split={p.split_k}")
                _check_same(X, qw, s, z, G, p, padx=72, pady=12,
                            what=f"gemv cfg={cfg} cols={cols} split={split}")


@pytest.mark.parametrize("M,N", [(16, 1030), (33, 2048), (64, 516), (8, 4100)])
def test_skinny_strided(M, N):
    from w4a16.hip_kernel import plan_for

    K, G = 2048, 64
    X, qw, s, z = _case(M, K, N, G, seed=M + 1)
    for cfg in (0,) + ((2,) if M <= 32 and N % 2 == 0 else ()) + (
            (3,) if M <= 16 and N % 4 == 0 else ()):
        p = plan_for(M, N, K, G, "skinny", 0)
        p.tile_cfg = cfg
        log(f"skinny strided M={M} N={N} cfg={cfg}")
        # odd output stride: the skinny kernel stores single elements
        _check_same(X, qw, s, z, G, p, padx=8, pady=3, what=f"skinny cfg={cfg}")


@pytest.mark.parametrize("M,K,N,G", [(130, 2048, 516, 64), (40, 1024, 1028, 128)])
def test_mfma_strided_every_config(M, K, N, G):
    from w4a16 import _lib
    from w4a16.hip_kernel import plan_for

    X, qw, s, z = _case(M, K, N, G, seed=M + K)
    b = (torch.randn(N) * 2).to(torch.float16).to(DEV)
    for cfg in _lib.MFMA_CONFIGS:
        p = plan_for(M, N, K, G, "mfma", 1)
        p.tile_cfg = cfg
        log(f"mfma strided M={M} K={K} N={N} cfg={cfg}")
        _check_same(X, qw, s, z, G, p, padx=40, pady=4, bias=b if cfg % 3 == 0 else None,
                    what=f"mfma cfg={cfg}")
    for cfg in (7, 11, 12, 13, 14):
        p = plan_for(M, N, K, G, "mfma", 3)
        p.tile_cfg = cfg
        assert p.split_k > 1
        log(f"mfma strided split-K M={M} cfg={cfg} split={p.split_k}")
        _check_same(X, qw, s, z, G, p, padx=16, pady=8, bias=b, what=f"split cfg={cfg}")


def test_public_entry_points_take_row_strided_views():
    """w4a16_matmul / w4a16_linear with row-strided x and out: same plan as the
    contiguous call when the strides keep rows aligned, the SIMT kernel when
    they do not -- both against the oracle."""
    from w4a16 import w4a16_matmul
    from w4a16.hip_kernel import w4a16_linear

    for M, K, N, G, padx, pady in ((1, 4096, 4096, 128, 64, 8), (24, 2048, 1024, 64, 8, 4),
                                   (256, 2048, 2048, 128, 256, 4), (5, 512, 96, 64, 3, 1)):
        log(f"public strided M={M} K={K} N={N} padx={padx} pady={pady}")
        X, qw, s, z = _case(M, K, N, G, seed=M * 7)
        ref = O.reference_w4a16(np_(X), np_(qw), np_(s), np_(z), G)
        xv, yb, yv = _views(X, N, padx, pady, seed=M)
        out = w4a16_matmul(xv, qw, s, z, G, out=yv)
        assert_gemm_close(out, ref, f"strided M={M} padx={padx}")
        assert bool((yb[:, N:] == SENTINEL).all())
        if padx % 8 == 0 and pady % 4 == 0:
            assert torch.equal(out, w4a16_matmul(X, qw, s, z, G))
        # the fused bias is the unfused result + bias in fp16 on every path
        b = (torch.randn(N) * 2).to(torch.float16).to(DEV)
        assert torch.equal(w4a16_linear(xv, qw, s, z, b, G), out + b)


def test_other_layouts_still_assert():
    """Reference test_correctness.py:49-59: a transposed view raises AssertionError
    (only row-major views with unit inner stride are taken)."""
    from w4a16 import w4a16_matmul

    X, qw, s, z = _case(8, 128, 64, 64, seed=3)
    with pytest.raises(AssertionError):
        w4a16_matmul(torch.randn(128, 8, dtype=torch.float16, device=DEV).t(), qw, s, z, 64)
    # overlapping rows (row stride < K) are not a row-major view either
    base = torch.randn(8 * 64 + 64, dtype=torch.float16, device=DEV)
    with pytest.raises(AssertionError):
        w4a16_matmul(base.as_strided((8, 128), (64, 1)), qw, s, z, 64)
    with pytest.raises(AssertionError):
        w4a16_matmul(X, qw, s, z, 64, out=torch.empty(64, 8, dtype=torch.float16, device=DEV).t())

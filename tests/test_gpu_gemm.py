"""GPU parity: the fused W4A16 GEMM (every kernel path) vs the CPU oracle.

Acceptance: each fp16 output within one fp16 ulp of the oracle's
fp16(fp32(X) @ fp32(dequant(W))), or within rtol = atol = 1e-3 where split-K
reorders the fp32 sums.  Mirrors the reference's
test_correctness.py (w4a16-kernel/tests/test_correctness.py:35-112) with the
tighter tolerance, plus every BASELINE configuration and each kernel path
forced over ragged shapes.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import DEV, assert_gemm_close, case_tensors, log, np_, oracle_cols, sample_cols
from oracle import w4a16_oracle as O

pytestmark = pytest.mark.gpu


def _build_case(M, K, N, G, seed=0, std=1.0):
    """Reference test_correctness.py:23-32: X, W ~ N(0, 1) fp16, quantised on the GPU."""
    from w4a16 import quantize_weight

    g = torch.Generator().manual_seed(seed)
    X = torch.randn(M, K, generator=g).to(torch.float16)
    W = (torch.randn(K, N, generator=g) * std).to(torch.float16)
    qw, s, z = quantize_weight(W.to(DEV), G)
    return X.to(DEV), qw, s, z


def _ref(X, qw, s, z, G):
    return O.reference_w4a16(np_(X), np_(qw), np_(s), np_(z), G)


@pytest.mark.parametrize("K,N", [(4096, 4096), (4096, 11008), (11008, 4096)])
@pytest.mark.parametrize("group_size", [64, 128])
def test_matches_oracle_reference_grid(K, N, group_size):
    """Reference test_correctness.py:35-46 grid, M in {1, 16, 64, 256}."""
    from w4a16 import w4a16_matmul

    for M in (1, 16, 64, 256):
        log(f"grid M={M} K={K} N={N} G={group_size}")
        X, qw, s, z = _build_case(M, K, N, group_size)
        out = w4a16_matmul(X, qw, s, z, group_size)
        assert out.shape == (M, N) and out.dtype == torch.float16
        assert_gemm_close(out, _ref(X, qw, s, z, group_size), f"M={M} K={K} N={N} G={group_size}")


@pytest.mark.parametrize("cfg", ["C1", "C2"])
def test_baseline_configs_small(cfg):
    from w4a16 import w4a16_matmul
    from w4a16 import workloads as wl

    for case in wl.CONFIGS[cfg]:
        log(case.name)
        X, W, qw, s, z = case_tensors(case)
        out = w4a16_matmul(X, qw, s, z, case.G)
        assert_gemm_close(out, _ref(X, qw, s, z, case.G), case.name)


@pytest.mark.parametrize("KN", [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)])
def test_config_c3_decode_sweep(KN):
    """C3: M in {1,4,8,16,32} on one Llama-3-8B block's linears; columns sampled
    for the oracle when N is large."""
    from w4a16 import w4a16_matmul
    from w4a16 import workloads as wl

    for case in [c for c in wl.CONFIGS["C3"] if (c.K, c.N) == KN]:
        log(case.name)
        X, W, qw, s, z = case_tensors(case)
        out = w4a16_matmul(X, qw, s, z, case.G)
        if case.N <= 8192:
            assert_gemm_close(out, _ref(X, qw, s, z, case.G), case.name)
        else:
            cols = sample_cols(case.N, 512)
            assert_gemm_close(out[:, cols], oracle_cols(X, qw, s, z, case.G, cols), case.name)


@pytest.mark.parametrize("M", [512, 2048, 4096])
def test_config_c4_prefill(M):
    """C4 at full size (outlier columns); oracle on sampled columns."""
    from w4a16 import w4a16_matmul
    from w4a16 import workloads as wl

    case = [c for c in wl.CONFIGS["C4"] if c.M == M][0]
    log(case.name)
    X, W, qw, s, z = case_tensors(case)
    out = w4a16_matmul(X, qw, s, z, case.G)
    cols = sample_cols(case.N, 160)
    assert_gemm_close(out[:, cols], oracle_cols(X, qw, s, z, case.G, cols), case.name)
    assert bool(torch.isfinite(out).all())


@pytest.mark.parametrize("KN", [(8192, 28672), (28672, 8192)])
@pytest.mark.parametrize("G", [32, 64, 128])
def test_config_c5_large_layer(KN, G):
    """C5: 70B-style layers, heavy-tailed weights, M in {1, 16, 256}."""
    from w4a16 import w4a16_matmul
    from w4a16 import workloads as wl

    for case in [c for c in wl.CONFIGS["C5"] if (c.K, c.N) == KN and c.G == G]:
        log(case.name)
        X, W, qw, s, z = case_tensors(case)
        out = w4a16_matmul(X, qw, s, z, case.G)
        cols = sample_cols(case.N, 128)
        assert_gemm_close(out[:, cols], oracle_cols(X, qw, s, z, case.G, cols), case.name)


# --------------------------------------------------------------------------- #
# each kernel path forced, ragged shapes                                        #
# --------------------------------------------------------------------------- #
RAGGED = [
    (1, 64, 260, 32), (3, 96, 12, 32), (8, 4096, 4100, 128), (5, 11008, 1028, 64),
    (2, 1024, 256, 32), (7, 160, 520, 32), (2, 16640, 132, 128),
]


@pytest.mark.parametrize("M,K,N,G", RAGGED)
def test_gemv_splits(M, K, N, G):
    """Decode GEMV with every column-block width, both wave counts (8, and 16
    waves per workgroup for M <= 2), the LDS-staged activations (cfg 4, 5,
    M <= 2; K = 16640 needs several staging chunks) and k-splits 1, 2, 3, 7,
    auto."""
    from w4a16.hip_kernel import plan_for, w4a16_matmul_planned

    X, qw, s, z = _build_case(M, K, N, G, seed=M + K)
    ref = _ref(X, qw, s, z, G)
    for cfg in ((1, 2, 4, 5, 6, 7) if M <= 2 else (1,)):
        for cols in ((64, 128) if cfg >= 6 else (16, 32, 64, 128, 256)):
            for split in (1, 2, 3, 7, 0):
                if split > K // 8:
                    continue
                p = plan_for(M, N, K, G, "gemv", split)
                p.tile_n = cols
                p.tile_cfg = cfg
                if split == 0:
                    p.split_k = max(1, min(p.split_k, K // 8))
                log(f"gemv M={M} K={K} N={N} G={G} cfg={cfg} cols={cols} split={p.split_k}")
                out = w4a16_matmul_planned(X, qw, s, z, G, p)
                assert_gemm_close(out, ref, f"gemv cfg={cfg} cols={cols} split={p.split_k}")


@pytest.mark.parametrize("M,K,N,G", [
    (9, 96, 260, 32), (33, 160, 516, 32), (127, 4096, 1028, 128), (129, 4096, 516, 64),
    (200, 1024, 1540, 32), (64, 4096, 4096, 128), (1, 64, 128, 32), (16, 11008, 4096, 64),
    (600, 1024, 2048, 64), (520, 2112, 772, 96), (260, 768, 1028, 96),
])
def test_mfma_tile_configs(M, K, N, G):
    """Prefill MFMA kernels with every tile configuration over tails in M, N, K
    (configs 1 and 2, one wave per SIMD with 32x32x16 MFMAs, any K; config 7,
    two waves per SIMD with 16x16x32 MFMAs, where K % 64 == 0; config 6, two
    waves per SIMD with 32x32x16 MFMAs, where K % 128 == 0; configs 11, 12
    and 13, activations and weights streamed into LDS with 128-, 32- and
    64-row tiles, and 14, the 128-row tile with two k-slices of four waves
    per workgroup, where K % 256 == 0)."""
    from w4a16.hip_kernel import plan_for, w4a16_matmul_planned
    from w4a16 import _lib

    X, qw, s, z = _build_case(M, K, N, G, seed=M * 3 + N)
    ref = _ref(X, qw, s, z, G)
    for cfg in _lib.MFMA_CONFIGS:
        if (cfg == 7 and K % 64) or (cfg == 6 and K % 128) or (cfg >= 11 and K % 256):
            continue
        p = plan_for(M, N, K, G, "mfma", 1)
        p.tile_cfg = cfg
        log(f"mfma M={M} K={K} N={N} G={G} cfg={cfg}")
        out = w4a16_matmul_planned(X, qw, s, z, G, p)
        assert_gemm_close(out, ref, f"mfma cfg={cfg}")
        b = (torch.randn(N) * 2).to(torch.float16).to(DEV)
        assert torch.equal(w4a16_matmul_planned(X, qw, s, z, G, p, bias=b), out + b)
    assert _lib.KERNEL_NAMES[p.kernel] == "mfma"


@pytest.mark.parametrize("M,K,N,G", [
    (65, 4096, 1028, 128), (200, 2048, 516, 32), (256, 11008, 772, 64), (130, 2112, 260, 96),
])
def test_mfma_split_k(M, K, N, G):
    """Prefill split-K (cfg 7 and, where K % 256 == 0, 11-13): fp32 partials per
    k-split, summed in split order by a second kernel; every split count, fused
    bias; then a forced GEMV split-K call reuses the same cached workspace."""
    from w4a16 import w4a16_matmul
    from w4a16.hip_kernel import plan_for, w4a16_matmul_planned

    X, qw, s, z = _build_case(M, K, N, G, seed=M + N + K)
    ref = _ref(X, qw, s, z, G)
    b = (torch.randn(N) * 2).to(torch.float16).to(DEV)
    for cfg in (7, 11, 12, 13, 14) if K % 256 == 0 else (7,):
        for split in (2, 3, 5, K // 64):
            p = plan_for(M, N, K, G, "mfma", split)
            p.tile_cfg = cfg
            assert p.split_k > 1 and p.workspace_bytes > 0
            log(f"mfma split-K M={M} K={K} N={N} G={G} cfg={cfg} split={p.split_k}")
            out = w4a16_matmul_planned(X, qw, s, z, G, p)
            assert_gemm_close(out, ref, f"split-K cfg={cfg} split={p.split_k}")
            outb = w4a16_matmul_planned(X, qw, s, z, G, p, bias=b)
            assert torch.equal(outb, out + b)
    Xg, qg, sg, zg = _build_case(1, 4096, 1024, 128, seed=5)
    pg = plan_for(1, 1024, 4096, 128, "gemv", 4)
    assert pg.split_k == 4
    assert_gemm_close(w4a16_matmul_planned(Xg, qg, sg, zg, 128, pg), _ref(Xg, qg, sg, zg, 128),
                      "GEMV split-K after prefill split-K")
    assert plan_for(1, 1024, 4096, 128).split_k == 1


@pytest.mark.parametrize("M,K,N,G,split", [
    (320, 4096, 4096, 128, 6), (300, 5120, 5120, 64, 5), (450, 4096, 4096, 32, 4),
    (290, 4096, 11008, 128, 2),
])
def test_mid_m_64_row_split(M, K, N, G, split):
    """256 < M <= 512: the automatic path where the planner takes 64-row
    streamed tiles (cfg 13) split for about two workgroups per CU instead of
    the 128-row plan (ragged last 64-row tile at M = 300 / 450 / 290), against
    the oracle, with and without the fused bias."""
    from w4a16 import w4a16_matmul
    from w4a16.hip_kernel import plan_for, w4a16_linear

    p = plan_for(M, N, K, G)
    assert (p.tile_cfg, p.tile_m, p.split_k) == (13, 64, split), (p.tile_cfg, p.split_k)
    X, qw, s, z = _build_case(M, K, N, G, seed=M + 7 * G)
    ref = _ref(X, qw, s, z, G)
    log(f"mid-M auto M={M} K={K} N={N} G={G} cfg=13 split={split}")
    out = w4a16_matmul(X, qw, s, z, G)
    assert_gemm_close(out, ref, f"mid-M cfg 13 split={split}")
    b = (torch.randn(N) * 2).to(torch.float16).to(DEV)
    assert torch.equal(w4a16_linear(X, qw, s, z, b, G), out + b)


@pytest.mark.parametrize("M,K,N,G", [
    (9, 96, 260, 32), (16, 4096, 4096, 128), (17, 160, 7, 32), (32, 11008, 1028, 64),
    (33, 1024, 130, 32), (48, 4096, 516, 128), (64, 4096, 4100, 64), (1, 4096, 1000, 128),
    (5, 320, 33, 32), (24, 2048, 6150, 64), (4, 4096, 8194, 128),
    # G = 32 (scales / zeros every k-step) on 16 single-batch waves and on the
    # 4-wave loop, as the planner now picks for K <= 4096 and K <= 8192
    (48, 4096, 4100, 32), (20, 8192, 1030, 32),
])
def test_skinny_path(M, K, N, G):
    """Skinny-M MFMA kernel (16x16x32) over ragged M (1..64), any N, K % 64 != 0,
    with 16-column blocks, (N even) 32-column blocks with two columns per lane
    and (N % 4 == 0) 64-column blocks with four; each with all rows in one
    workgroup (32- / 64-column blocks: M <= 32 / 16) and with one 16- or 8-row
    group per workgroup (the last one ragged)."""
    from w4a16.hip_kernel import plan_for, w4a16_matmul_planned

    X, qw, s, z = _build_case(M, K, N, G, seed=M * 7 + N)
    ref = _ref(X, qw, s, z, G)
    b = (torch.randn(N) * 2).to(torch.float16).to(DEV)
    whole = (M + 15) // 16 * 16
    for rows in sorted({whole, 16, 8}):
        cfgs = (0,) + ((2,) if rows <= 32 and N % 2 == 0 else ()) + (
            (3,) if rows <= 16 and N % 4 == 0 else ())
        for cfg in cfgs:
            log(f"skinny M={M} K={K} N={N} G={G} cfg={cfg} rows={rows}")
            p = plan_for(M, N, K, G, "skinny")
            p.tile_cfg, p.tile_m = cfg, rows
            out = w4a16_matmul_planned(X, qw, s, z, G, p)
            assert_gemm_close(out, ref, f"skinny cfg={cfg} rows={rows}")
            outb = w4a16_matmul_planned(X, qw, s, z, G, p, bias=b)
            assert torch.equal(outb, out + b)


@pytest.mark.parametrize("M,K,N,G", [
    (16, 2080, 1030, 32), (24, 1056, 516, 32), (31, 4064, 772, 32), (40, 4096, 2052, 128),
    (17, 3104, 260, 32), (24, 8224, 516, 32), (32, 11008, 1030, 64), (17, 5120, 260, 128),
    (9, 2080, 516, 32), (12, 4096, 1030, 128), (15, 1056, 772, 32),
])
def test_skinny_staged_activations(M, K, N, G):
    """16-row tiles at M >= 9 stage each wave's activations in LDS by
    whole-line loads with one batch per wave on 8 or 16 waves (1024 < K <=
    4096; longer K, the 4-wave loop's direct loads, alongside).  Ragged K (a
    wave's batch partly or wholly past K: K = 2080 / 1056 / 3104 leave one
    step to the last busy wave, 4064 seven, 8224 one in the loop) and a
    row-strided X whose elements past K hold inf and NaN, which a whole-line
    load would read and which must count as zero, as the direct loads'
    out-of-range steps do; every block width, against the oracle."""
    from w4a16.hip_kernel import plan_for, w4a16_matmul_planned

    X, qw, s, z = _build_case(M, K, N, G, seed=K + M)
    ref = _ref(X, qw, s, z, G)
    ldx = K + 64
    Xp = torch.full((M, ldx), float("nan"), dtype=torch.float16, device=DEV)
    Xp[:, K:K + 32] = float("inf")
    Xp[:, :K] = X
    Xs = Xp[:, :K]
    assert Xs.stride(0) == ldx
    for cfg in (0,) + ((2,) if N % 2 == 0 else ()) + ((3,) if N % 4 == 0 else ()):
        p = plan_for(M, N, K, G, "skinny")
        p.tile_cfg, p.tile_m = cfg, 16
        for name, x in (("dense", X), ("strided", Xs)):
            log(f"skinny staged M={M} K={K} N={N} G={G} cfg={cfg} {name}")
            out = w4a16_matmul_planned(x, qw, s, z, G, p)
            assert_gemm_close(out, ref, f"skinny staged cfg={cfg} {name}")


@pytest.mark.parametrize("M,K,N,G", [(1, 64, 130, 32), (17, 96, 7, 32), (4, 24, 12, 12), (2, 8, 5, 4)])
def test_simt_path_any_shape(M, K, N, G):
    """SIMT kernel: odd N, G not a multiple of 8."""
    from w4a16.cuda_kernel import w4a16_matmul_cuda

    log(f"simt M={M} K={K} N={N} G={G}")
    X, qw, s, z = _build_case(M, K, N, G, seed=N)
    out = w4a16_matmul_cuda(X, qw, s, z, G)
    assert_gemm_close(out, _ref(X, qw, s, z, G), "simt")


@pytest.mark.parametrize("M", [1, 64])
@pytest.mark.parametrize("K,N", [(4096, 4096), (11008, 4096)])
@pytest.mark.parametrize("group_size", [64, 128])
def test_cuda_module_matches_reference(M, K, N, group_size):
    """Reference test_correctness.py:96-112: the native (SIMT) backend vs the oracle."""
    from w4a16.cuda_kernel import load_cuda_module, w4a16_matmul_cuda

    load_cuda_module(verbose=False)
    log(f"cuda-module M={M} K={K} N={N} G={group_size}")
    X, qw, s, z = _build_case(M, K, N, group_size)
    out = w4a16_matmul_cuda(X, qw, s, z, group_size)
    assert out.shape == (M, N) and out.dtype == torch.float16
    assert_gemm_close(out, _ref(X, qw, s, z, group_size), "simt")


# --------------------------------------------------------------------------- #
# API behaviour                                                                 #
# --------------------------------------------------------------------------- #
def test_fused_bias_epilogue():
    """W4A16Linear arithmetic (linear.py:90-91): the GEMM result rounded to fp16,
    then ``+ bias`` in fp16.  On every path: the bias-free output is within
    tolerance of the oracle, and the fused output equals fp16(Y + bias) of that
    same Y bit for bit."""
    from w4a16.hip_kernel import plan_for, w4a16_matmul_planned

    for (M, K, N, G, kern) in [(1, 4096, 4096, 128, "gemv"), (4, 1024, 516, 32, "gemv"),
                               (64, 1024, 1028, 32, "mfma"), (3, 64, 10, 32, "simt"),
                               (24, 1024, 1028, 32, "skinny")]:
        log(f"bias {kern} M={M} K={K} N={N}")
        X, qw, s, z = _build_case(M, K, N, G, seed=7)
        b = (torch.randn(N) * 3).to(torch.float16).to(DEV)
        p = plan_for(M, N, K, G, kern)
        y = w4a16_matmul_planned(X, qw, s, z, G, p)
        assert_gemm_close(y, _ref(X, qw, s, z, G), f"no-bias {kern}")
        out = w4a16_matmul_planned(X, qw, s, z, G, p, bias=b)
        want = (y + b)                      # torch fp16 add on the device: one RNE rounding
        assert torch.equal(out, want), f"bias epilogue {kern}"


def test_out_parameter_and_empty():
    from w4a16 import w4a16_matmul

    X, qw, s, z = _build_case(16, 256, 128, 64)
    out = torch.full((16, 128), float("nan"), dtype=torch.float16, device=DEV)
    y = w4a16_matmul(X, qw, s, z, 64, out=out)
    assert y.data_ptr() == out.data_ptr()
    assert_gemm_close(out, _ref(X, qw, s, z, 64), "out=")
    y0 = w4a16_matmul(X[:0], qw, s, z, 64)
    assert y0.shape == (0, 128)
    # K = 0: Y = 0, and the fused linear gives exactly the bias
    from w4a16.hip_kernel import w4a16_linear
    Xk = torch.empty((3, 0), dtype=torch.float16, device=DEV)
    qk = torch.empty((0, 128), dtype=torch.int32, device=DEV)
    sk = torch.empty((0, 128), dtype=torch.float16, device=DEV)
    yk = w4a16_matmul(Xk, qk, sk, sk, 64, out=torch.full((3, 128), 7.0, dtype=torch.float16,
                                                           device=DEV))
    assert torch.equal(yk, torch.zeros_like(yk))
    b = torch.randn(128, dtype=torch.float16, device=DEV)
    yb = w4a16_linear(Xk, qk, sk, sk, b, 64)
    assert torch.equal(yb, b.expand(3, 128))


def test_kernel_asserts_contiguity():
    """Reference test_correctness.py:49-59."""
    from w4a16 import w4a16_matmul

    X, qw, s, z = _build_case(8, 128, 64, 64)
    X_bad = torch.randn(128, 8, dtype=torch.float16, device=DEV).t()
    assert not X_bad.is_contiguous()
    with pytest.raises(AssertionError):
        w4a16_matmul(X_bad, qw, s, z, 64)


def test_kernel_rejects_bad_group_size():
    """Reference test_correctness.py:62-70: G = 8 raises AssertionError."""
    from w4a16 import w4a16_matmul

    X, qw, s, z = _build_case(8, 64, 64, 8)
    with pytest.raises(AssertionError):
        w4a16_matmul(X, qw, s, z, 8)


def test_split_k_is_deterministic():
    """Forced split-K GEMV sums fp32 partials in split order in a second kernel:
    repeated runs agree bit for bit, whatever the workspace held before (the
    partials are rewritten by every call, nothing needs to start zeroed)."""
    from w4a16.hip_kernel import plan_for, w4a16_matmul_planned
    from w4a16 import _runtime

    M, K, N, G = 1, 4096, 1024, 128
    p = plan_for(M, N, K, G, "gemv", 4)
    assert p.split_k == 4 and p.workspace_bytes == 4 * M * N * 4
    X, qw, s, z = _build_case(M, K, N, G, seed=3)
    outs = []
    for i in range(5):
        ws = _runtime.workspace(X.device, p.workspace_bytes)
        ws.fill_(0xFF if i % 2 else 0x5A)          # stale garbage between calls
        outs.append(w4a16_matmul_planned(X, qw, s, z, G, p).clone())
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    assert_gemm_close(outs[0], _ref(X, qw, s, z, G), "split-K")


@pytest.mark.parametrize("M,K,N,G", [(1, 14336, 1024, 128), (2, 8192, 512, 64), (2, 8256, 260, 96)])
def test_gemv_auto_split_long_k(M, K, N, G):
    """Long K, few column blocks: the automatic decode plan splits K four ways
    (fp32 partials, split-order reduction, fused bias)."""
    from w4a16 import w4a16_matmul
    from w4a16.hip_kernel import plan_for, w4a16_linear

    p = plan_for(M, N, K, G)
    assert p.split_k == 4 and p.workspace_bytes == 4 * M * N * 4
    log(f"gemv auto split M={M} K={K} N={N} G={G}")
    X, qw, s, z = _build_case(M, K, N, G, seed=K + N)
    out = w4a16_matmul(X, qw, s, z, G)
    assert_gemm_close(out, _ref(X, qw, s, z, G), f"gemv auto split-K M={M} K={K} N={N}")
    b = (torch.randn(N) * 2).to(torch.float16).to(DEV)
    assert torch.equal(w4a16_linear(X, qw, s, z, b, G), out + b)


def test_streamed_prefill_far_apart_scales_zeros():
    """The streamed prefill kernels (cfg 11 / 12 / 13 / 14) read scales and zeros
    through one buffer resource based at the lower of the two; placed more
    than 2 GiB apart they take the register kernel of 128 x 256 tiles (cfg 7)
    instead, with the plan's k-split and workspace (its own split count never
    exceeds the plan's).  Unsplit and split plans of every row count, with a
    fused bias, against the oracle; the bias add is bit-exact."""
    from w4a16.hip_kernel import plan_for, w4a16_matmul_planned

    M, K, N, G = 256, 2048, 1028, 64
    X, qw, s, z = _build_case(M, K, N, G, seed=11)
    ref = _ref(X, qw, s, z, G)
    b = (torch.randn(N) * 2).to(torch.float16).to(DEV)
    # scales at the start and zeros at the end of one 2.5 GiB allocation
    big = torch.empty(5 << 29, dtype=torch.uint8, device=DEV)
    nb = s.numel() * 2
    s_far = big[:nb].view(torch.float16).view(s.shape).copy_(s)
    z_far = big[big.numel() - nb:].view(torch.float16).view(z.shape).copy_(z)
    dist = abs(z_far.data_ptr() - s_far.data_ptr())
    log(f"scales/zeros {dist / 2**30:.2f} GiB apart")
    assert dist >= (1 << 31)
    # the wrapper says once per process that such calls leave the streamed kernels
    import warnings

    from w4a16 import hip_kernel as hk

    hk._FAR_SZ_WARNED = False
    with warnings.catch_warnings(record=True) as seen:
        warnings.simplefilter("always")
        w4a16_matmul_planned(X, qw, s, z, G, plan_for(M, N, K, G))
        assert not seen, "adjacent scales / zeros must not warn"
        w4a16_matmul_planned(X, qw, s_far, z_far, G, plan_for(M, N, K, G))
        w4a16_matmul_planned(X, qw, s_far, z_far, G, plan_for(M, N, K, G))
    far = [w for w in seen if issubclass(w.category, RuntimeWarning) and "2 GiB" in str(w.message)]
    assert len(far) == 1, [str(w.message) for w in seen]
    for cfg, split in ((11, 1), (11, 3), (12, 2), (13, 4), (12, 8), (14, 1), (14, 2)):
        p = plan_for(M, N, K, G, "mfma", split)
        p.tile_cfg = cfg
        assert p.split_k == split
        log(f"far-apart cfg={cfg} split={p.split_k}")
        adj = w4a16_matmul_planned(X, qw, s, z, G, p)
        assert_gemm_close(adj, ref, f"cfg {cfg} split {split} adjacent")
        out = w4a16_matmul_planned(X, qw, s_far, z_far, G, p)
        assert_gemm_close(out, ref, f"cfg {cfg} split {split} scales/zeros far apart")
        outb = w4a16_matmul_planned(X, qw, s_far, z_far, G, p, bias=b)
        assert torch.equal(outb, out + b)
    del big


def test_graph_capture_replays():
    """Every kernel family captured once in a HIP graph and replayed several
    times, with eager work in between: each replay equals the eager result bit
    for bit (the library issues kernel launches only -- no memset -- and every
    path, split-K included, is deterministic)."""
    from w4a16 import w4a16_matmul
    from w4a16.hip_kernel import plan_for

    cases = [(1, 4096, 4096, 128), (1, 14336, 1024, 128), (4, 4096, 4096, 128),
             (1024, 4096, 4096, 128), (256, 8192, 2048, 64), (32, 4096, 28672, 128),
             (100, 2112, 520, 96)]
    for M, K, N, G in cases:
        p = plan_for(M, N, K, G)
        log(f"graph M={M} K={K} N={N} G={G} kernel={p.as_dict()['kernel_name']} "
            f"cfg={p.tile_cfg} split={p.split_k}")
        X, qw, s, z = _build_case(M, K, N, G, seed=M + K + N)
        eager = w4a16_matmul(X, qw, s, z, G)
        out = torch.empty_like(eager)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            w4a16_matmul(X, qw, s, z, G, out=out)     # warm-up: workspace, plan
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            w4a16_matmul(X, qw, s, z, G, out=out)
        for i in range(3):
            out.fill_(float("nan"))
            w4a16_matmul(X * 2, qw, s, z, G)           # eager work between replays
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {i} M={M} K={K} N={N}"
    assert plan_for(1, 1024, 14336, 128).split_k > 1
    assert plan_for(32, 28672, 4096, 128).split_k > 1


def test_graph_workspace_owned_by_capture():
    """Split-K calls captured into two graphs (torch's default capture stream
    for both) each own their workspace: after the eager workspace has grown
    (the old buffer freed and its memory handed out again), both graphs
    replayed at the same time on two streams, several times, still equal
    their eager results bit for bit."""
    from w4a16 import w4a16_matmul
    from w4a16.hip_kernel import plan_for

    shapes = [(1, 14336, 1024, 128), (32, 4096, 28672, 128)]
    graphs, outs, eagers, inputs = [], [], [], []
    for M, K, N, G in shapes:
        assert plan_for(M, N, K, G).split_k > 1
        log(f"capture split-K M={M} K={K} N={N} G={G}")
        X, qw, s, z = _build_case(M, K, N, G, seed=K + M)
        eager = w4a16_matmul(X, qw, s, z, G)
        out = torch.empty_like(eager)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            w4a16_matmul(X, qw, s, z, G, out=out)
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            w4a16_matmul(X, qw, s, z, G, out=out)
        graphs.append(g), outs.append(out), eagers.append(eager), inputs.append((X, qw, s, z, G))
    # grow the eager workspace well past both captures' needs, then churn the
    # allocator so the replaced buffer's memory is reused
    log("grow eager workspace")
    Xb, qwb, sb, zb = _build_case(256, 28672, 8192, 128, seed=5)
    w4a16_matmul(Xb, qwb, sb, zb, 128)
    junk = [torch.full((1 << 20,), 7.0, device=DEV) for _ in range(64)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(4):
        log(f"concurrent replay {rep}")
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        for g, st in zip(graphs, streams):
            with torch.cuda.stream(st):
                g.replay()
        w4a16_matmul(Xb, qwb, sb, zb, 128)          # eager split-K work meanwhile
        torch.cuda.synchronize()
        for o, e, (M, K, N, G) in zip(outs, eagers, shapes):
            assert torch.equal(o, e), f"replay {rep} M={M} K={K} N={N}"
    del junk


def test_baselines_on_gpu():
    """reference_w4a16 / dequant_then_matmul / fp16_matmul (reference.py:18-67)
    on the GPU, each against the oracle's own restatement of the same function
    (pinned by float64 brute force in test_oracle_pins), to the GEMM tolerance."""
    from w4a16 import dequant_then_matmul, dequantize_weight, fp16_matmul, reference_w4a16

    M, K, N, G = 32, 1024, 512, 128
    X, qw, s, z = _build_case(M, K, N, G, seed=4)
    Xn, qwn, sn, zn = np_(X), np_(qw), np_(s), np_(z)
    assert_gemm_close(reference_w4a16(X, qw, s, z, G), _ref(X, qw, s, z, G),
                      "reference_w4a16 (GPU)")
    y2 = dequant_then_matmul(X, qw, s, z, G)
    assert y2.dtype == torch.float16
    assert_gemm_close(y2, O.dequant_then_matmul(Xn, qwn, sn, zn, G), "dequant_then_matmul (GPU)")
    W = dequantize_weight(qw, s, z, G)
    y3 = fp16_matmul(X, W)
    assert y3.dtype == torch.float16
    assert_gemm_close(y3, O.fp16_matmul(Xn, np_(W)), "fp16_matmul (GPU)")
    # CPU inputs come back on the CPU
    y4 = fp16_matmul(X.cpu(), W.cpu())
    assert y4.device.type == "cpu" and torch.equal(y4, y3.cpu())


@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("cfg", [4, 5, 6, 7])
def test_gemv_staged_nonfinite_activations(M, cfg):
    """An inf in X on the staged GEMV blocks whose runs take an odd number of
    batches (K = 5120: five 4-row batches per row-lane on 64-column blocks):
    the batch after a run's end holds the next row-lane's rows, and its zero
    weights must meet the zero row of X, not that row-lane's inf.  Y must give
    the oracle's inf / NaN pattern: +-inf where the weight under the inf is
    non-zero, NaN where it dequantises to zero."""
    from w4a16.hip_kernel import plan_for, w4a16_matmul_planned

    K, N, G = 5120, 13824, 64
    X, qw, s, z = _build_case(M, K, N, G, seed=17, std=0.02)
    X[0, 777] = float("inf")
    if M == 2:
        X[1, 4100] = float("-inf")
    cols = sample_cols(N, 256)
    ref = oracle_cols(X, qw, s, z, G, cols)
    assert np.isinf(ref).any() and np.isnan(ref).any(), "the case must hold both inf and NaN"
    for cols_per_wg in (64, 128):
        if cfg in (4, 5) and cols_per_wg == 128:
            continue
        p = plan_for(M, N, K, G, "gemv", 1)
        p.tile_n, p.tile_cfg = cols_per_wg, cfg
        log(f"gemv inf M={M} K={K} N={N} G={G} cfg={cfg} cols={cols_per_wg}")
        out = w4a16_matmul_planned(X, qw, s, z, G, p)
        assert_gemm_close(out[:, cols], ref, f"gemv inf cfg={cfg} cols={cols_per_wg}")

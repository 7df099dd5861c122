"""GPU parity for zero-points outside what quantize_weight makes.

The reference's fused kernels dequantise ``(q - z) * s`` in fp16 for any fp16
zero-point (w4a16-kernel/src/w4a16/triton_kernel.py:117-119,
cuda/w4a16_gemm.cu:51-58), and ``w4a16_matmul`` accepts any zeros tensor.  Here
the fused kernels come in two forms (integer zeros with |z| <= 1024, and any
zero); ``w4a16_matmul`` checks each zeros tensor once on the GPU and picks the
form.  These tests feed every kernel family fractional, large, signed-zero and
non-finite zero-points and compare with the oracle (whose fp16 arithmetic is
pinned in test_oracle_pins.py), and check that the any-zero form gives the
integer form's bits where both apply.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import DEV, assert_gemm_close, log, np_, oracle_cols, sample_cols
from oracle import w4a16_oracle as O

pytestmark = pytest.mark.gpu

# fp16 zero-points the integer-zero kernels cannot take, and some they can
EXOTIC = [3.5, 0.1, 7.25, 15.0078125, 64.5, 100.0, 1025.0, -1025.0, 2000.5, -3.75, 1e-7]
INTEGRAL_EDGE = [-0.0, 0.0, 63.0, 64.0, 100.0, 1024.0, -1024.0, -63.0, 15.0]


def _case(M, K, N, G, seed):
    from w4a16 import quantize_weight

    g = torch.Generator().manual_seed(seed)
    X = torch.randn(M, K, generator=g).to(torch.float16)
    W = (torch.randn(K, N, generator=g) * 0.05).to(torch.float16)
    qw, s, z = quantize_weight(W.to(DEV), G)
    return X.to(DEV), qw, s, z


def _exotic_zeros(z: torch.Tensor, seed: int, values=EXOTIC, nonfinite: bool = False):
    """A fresh zeros tensor: the quantised zeros with about a third of the
    entries replaced by values from `values` (and, optionally, one NaN and
    one +inf in two fixed columns)."""
    rng = np.random.default_rng(seed)
    zn = np_(z).astype(np.float16).copy()
    mask = rng.random(zn.shape) < 0.35
    zn[mask] = rng.choice(np.array(values, dtype=np.float16), size=int(mask.sum()))
    if nonfinite:
        zn[0, 1] = np.float16(np.nan)
        zn[-1, 2] = np.float16(np.inf)
    return torch.from_numpy(zn).to(DEV)


def _ref(X, qw, s, z, G):
    return O.reference_w4a16(np_(X), np_(qw), np_(s), np_(z), G)


def test_zeros_check_flags_exactly_the_non_integer_zeros():
    """w4a16_zeros_check_f16 flags a tensor iff some zero is not an integer in
    [-1024, 1024]; the answer is kept per tensor version."""
    from w4a16.hip_kernel import zeros_need_any_form

    base = torch.arange(16, dtype=torch.float16, device=DEV).repeat(8, 4)
    assert not zeros_need_any_form(base)
    for v in INTEGRAL_EDGE:
        t = base.clone()
        t[3, 7] = v
        assert not zeros_need_any_form(t), v
    def fp16_in_domain(v):
        h = float(np.float16(v))
        return h == h and abs(h) <= 1024 and h.is_integer()

    cands = EXOTIC + [float("nan"), float("inf"), float("-inf"), 0.5, -1023.5, 60000.0, -1024.5]
    flagged = [v for v in cands if not fp16_in_domain(v)]
    assert 100.0 not in flagged and -1024.5 not in flagged and 3.5 in flagged   # -1024.5 -> -1024
    t = base.clone()
    t[5, 61] = -1024.5
    assert not zeros_need_any_form(t)
    for v in flagged:
        t = base.clone()
        t[5, 61] = v
        log(f"zeros check {v}")
        assert zeros_need_any_form(t), v
    # an in-place change bumps the version: checked again
    t = base.clone()
    assert not zeros_need_any_form(t)
    t[0, 0] = 2.5
    assert zeros_need_any_form(t)
    t[0, 0] = 2.0
    assert not zeros_need_any_form(t)
    # one element, the last of a long tensor
    t = torch.zeros(7 * 4099, dtype=torch.float16, device=DEV)
    t[-1] = 0.25
    assert zeros_need_any_form(t)


def _families(M, K, N, G):
    """(label, plan) for every kernel family and configuration that takes the shape."""
    from w4a16 import _lib
    from w4a16.hip_kernel import plan_for

    out = [("auto", None)]
    if M <= 8:
        for cfg in ((1, 2, 4, 5, 6, 7) if M <= 2 else (1,)):
            for cols in ((64, 128) if cfg >= 6 else (16, 64, 256)):
                for split in (1, 3):
                    p = plan_for(M, N, K, G, "gemv", split)
                    p.tile_n, p.tile_cfg = cols, cfg
                    out.append((f"gemv cfg={cfg} cols={cols} split={p.split_k}", p))
    if M <= 64:
        whole = (M + 15) // 16 * 16
        for rows in sorted({whole, 16, 8}):
            for cfg in (0, 2, 3):
                if (cfg == 2 and (rows > 32 or N % 2)) or (cfg == 3 and (rows > 16 or N % 4)):
                    continue
                p = plan_for(M, N, K, G, "skinny")
                p.tile_cfg, p.tile_m = cfg, rows
                out.append((f"skinny cfg={cfg} rows={rows}", p))
    for cfg in _lib.MFMA_CONFIGS:
        if (cfg == 7 and K % 64) or (cfg == 6 and K % 128) or (cfg >= 11 and K % 256):
            continue
        for split in ((1, 2) if cfg in _lib.MFMA_SPLIT_CONFIGS else (1,)):
            p = plan_for(M, N, K, G, "mfma", split)
            p.tile_cfg = cfg
            out.append((f"mfma cfg={cfg} split={p.split_k}", p))
    out.append(("simt", plan_for(M, N, K, G, "simt")))
    return out


@pytest.mark.parametrize("M,K,N,G", [
    (1, 1024, 516, 64), (2, 2048, 260, 128), (5, 512, 1028, 32), (16, 1024, 772, 64),
    (48, 512, 516, 128), (130, 1024, 520, 64),
])
def test_any_zero_points_every_family(M, K, N, G):
    """Fractional, large and signed-zero zero-points (and one NaN and one inf
    column group) through every kernel family against the oracle."""
    from w4a16 import w4a16_matmul
    from w4a16.hip_kernel import w4a16_matmul_planned

    X, qw, s, z0 = _case(M, K, N, G, seed=M * 31 + K)
    for nonfinite in (False, True):
        z = _exotic_zeros(z0, seed=M + N, nonfinite=nonfinite)
        ref = _ref(X, qw, s, z, G)
        assert (np.isnan(ref).any() if nonfinite else np.isfinite(ref).all())
        for label, p in _families(M, K, N, G):
            log(f"any-zero M={M} K={K} N={N} G={G} {label} nonfinite={nonfinite}")
            out = (w4a16_matmul(X, qw, s, z, G) if p is None
                   else w4a16_matmul_planned(X, qw, s, z, G, p))
            assert_gemm_close(out, ref, f"any-zero {label} nonfinite={nonfinite}")


@pytest.mark.parametrize("M,K,N,G", [(1, 4096, 4096, 128), (4, 4096, 6144, 128),
                                     (32, 4096, 4096, 128), (4096, 4096, 14336, 128)])
def test_any_zero_points_baseline_shapes(M, K, N, G):
    """The BASELINE shapes' default plans (C2 GEMV, C3 skinny, C4 streamed
    prefill) with fractional and signed-zero zero-points mixed in; oracle on
    sampled columns.  The zeros stay within a few steps of the codes: with
    zeros of 100 or 2000 the weights grow a hundredfold and a K = 4096 dot
    product cancels so far (sum |x w| / |y| ~ 1e5) that fp32 summation order
    alone moves y by more than the 1e-3 tolerance (one such element measured:
    exact 0.13545, this build 0.1359, the oracle's BLAS 0.1346); those zeros
    run in the short-K family tests above."""
    from w4a16 import w4a16_matmul

    X, qw, s, z0 = _case(M, K, N, G, seed=K + N + M)
    z = _exotic_zeros(z0, seed=7, values=[3.5, 12.75, -0.0, 7.125, 20.5, -2.25])
    log(f"any-zero baseline M={M} K={K} N={N}")
    out = w4a16_matmul(X, qw, s, z, G)
    cols = sample_cols(N, 128)
    assert_gemm_close(out[:, cols], oracle_cols(X, qw, s, z, G, cols), f"any-zero M={M}")


@pytest.mark.parametrize("M,K,N,G", [(1, 2048, 1028, 64), (3, 1024, 520, 32), (24, 2048, 516, 128),
                                     (200, 1024, 1028, 64)])
def test_any_zero_form_equals_integer_form(M, K, N, G):
    """With integer zeros (the edge values included) the any-zero kernels give
    the integer-zero kernels' bits, family by family."""
    from w4a16 import _lib
    from w4a16.hip_kernel import w4a16_matmul_planned

    X, qw, s, z0 = _case(M, K, N, G, seed=M + 3)
    z = _exotic_zeros(z0, seed=M, values=INTEGRAL_EDGE)
    for label, p in _families(M, K, N, G):
        if p is None:
            continue
        log(f"any-zero form vs integer form M={M} {label}")
        a = w4a16_matmul_planned(X, qw, s, z, G, p)
        pz = _lib.Plan.from_buffer_copy(p)
        pz.flags = _lib.PLAN_ANY_ZEROS
        b = w4a16_matmul_planned(X, qw, s, z, G, pz)
        assert torch.equal(a, b), label


def test_unknown_plan_flags_refused():
    from w4a16 import _lib
    from w4a16.hip_kernel import plan_for, w4a16_matmul_planned

    X, qw, s, z = _case(1, 256, 64, 32, seed=1)
    p = plan_for(1, 64, 256, 32)
    p.flags = 2
    with pytest.raises(RuntimeError, match="W4A16_ERR_BAD_PLAN"):
        w4a16_matmul_planned(X, qw, s, z, 32, p)
    assert _lib.PLAN_ANY_ZEROS == 1


def test_linear_any_zero_points():
    """W4A16Linear with zeros loaded from a state_dict that holds fractional
    zero-points: the module's forward matches the oracle's linear."""
    from w4a16 import W4A16Linear

    K, N, G = 1024, 516, 64
    lin = W4A16Linear(K, N, group_size=G, bias=True, device=DEV)
    W = (torch.randn(K, N) * 0.05).to(torch.float16)
    lin.quantize_from_dense(W.to(DEV))
    lin.bias.copy_((torch.randn(N) * 0.5).to(torch.float16).to(DEV))
    sd = {k: v.clone() for k, v in lin.state_dict().items()}
    sd["zeros"] = _exotic_zeros(sd["zeros"], seed=3)
    lin.load_state_dict(sd)
    x = torch.randn(3, 5, K).to(torch.float16).to(DEV)
    log("linear any-zero")
    y = lin(x)
    ref = O.linear_forward(np_(x.reshape(-1, K)), np_(lin.qweight), np_(lin.scales),
                           np_(lin.zeros), np_(lin.bias), G)
    assert_gemm_close(y.reshape(-1, N), ref, "W4A16Linear any-zero")

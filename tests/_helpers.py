"""Shared helpers for the GPU parity tests (imported by test modules)."""
from __future__ import annotations

import functools
import sys

import numpy as np
import torch

from oracle import w4a16_oracle as O

DEV = "cuda"


def log(msg: str) -> None:
    """Name the case before GPU work, flushed, so a failed run still says which."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def np_(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def assert_gemm_close(out: torch.Tensor, ref: np.ndarray, what: str) -> None:
    """Acceptance: every element within 1 fp16 ulp of the oracle, or within
    rtol = atol = 1e-3 (split-K reorders fp32 sums)."""
    o = np_(out)
    assert o.shape == ref.shape, (what, o.shape, ref.shape)
    ok = O.within_tolerance(o, ref)
    if not ok.all():
        bad = np.argwhere(~ok)
        i = tuple(bad[0])
        d = np.abs(o.astype(np.float64) - ref.astype(np.float64))
        raise AssertionError(
            f"{what}: {len(bad)} of {ok.size} outside tolerance; first {i}: "
            f"got {o[i]!r} want {ref[i]!r}; max |diff| {d.max():.3g}")


def quantized_on_gpu(W: torch.Tensor, G: int):
    """Quantise on the GPU with the product kernel; returns device tensors."""
    from w4a16 import quantize_weight

    return quantize_weight(W.to(DEV), G)


@functools.lru_cache(maxsize=2)
def _layer(config: str, K: int, N: int, G: int):
    from w4a16 import workloads as wl

    case = [c for c in wl.CONFIGS[config] if (c.K, c.N, c.G) == (K, N, G)][0]
    W = wl.make_w(case)
    qw, s, z = quantized_on_gpu(W, G)
    return W, qw, s, z


def case_tensors(case):
    """(X dev, W cpu, qw dev, s dev, z dev) for a workloads.Case; the quantised
    layer is cached across M."""
    from w4a16 import workloads as wl

    W, qw, s, z = _layer(case.config, case.K, case.N, case.G)
    return wl.make_x(case).to(DEV), W, qw, s, z


def oracle_cols(X: torch.Tensor, qw, s, z, G: int, cols: np.ndarray) -> np.ndarray:
    """Oracle Y restricted to columns `cols` (GEMM columns are independent)."""
    return O.reference_w4a16(np_(X), np_(qw)[:, cols], np_(s)[:, cols], np_(z)[:, cols], G)


STRATUM = 16   # narrowest column block any kernel gives a workgroup


def sample_cols(N: int, k: int = 96, seed: int = 0) -> np.ndarray:
    """Columns for an oracle check of a wide output (columns are independent).

    Stratified: one random column inside every STRATUM-column block, so every
    column block of every kernel (16/32/64/256 columns wide) and every tile of
    the XCD-grouped tile orders is checked at least once, at a random lane
    position within the block; plus `k` further random columns and the first
    and last four.
    """
    rng = np.random.default_rng(seed + N)
    edge = np.array([0, 1, 2, 3, N - 4, N - 3, N - 2, N - 1])
    starts = np.arange(0, N, STRATUM)
    widths = np.minimum(STRATUM, N - starts)
    strat = starts + (rng.random(len(starts)) * widths).astype(np.int64)
    mid = rng.choice(N, size=min(k, N), replace=False)
    return np.unique(np.concatenate([edge[edge >= 0], strat, mid]))

"""GPU: calls from several host threads at once, each thread on its own HIP
stream, give the same bits as the same calls made one after another.

What runs concurrently here: the C ABI's per-device caches (CU count, decode
table) on their first use in the process, the Python wrapper's per-stream
split-K workspaces, and the per-tensor zero-point check.  The kernels are
deterministic for a given plan (fixed reduction orders, split-order sums), so
the comparison is bit for bit; each sequential result is also checked against
the CPU oracle.
"""
from __future__ import annotations

import threading

import numpy as np
import pytest
import torch

from _helpers import DEV, assert_gemm_close, log, np_
from oracle import w4a16_oracle as O

pytestmark = pytest.mark.gpu

# M, K, N, G and what the planner makes of it (checked below): the decode
# GEMV, the skinny kernel, the streamed prefill kernel split along K (a
# workspace), and the decode GEMV split along K (a workspace, a second kernel)
CASES = [
    (1, 4096, 4096, 128, "gemv", 1),
    (16, 4096, 2048, 128, "skinny", 1),
    (256, 8192, 2048, 64, "mfma", None),
    (1, 14336, 1024, 128, "gemv", 4),
]
REPS = 6


def _inputs(i, M, K, N, G):
    from w4a16 import quantize_weight

    g = torch.Generator().manual_seed(100 + i)
    X = torch.randn(M, K, generator=g).to(torch.float16)
    W = (torch.randn(K, N, generator=g) * 0.02).to(torch.float16)
    qw, s, z = quantize_weight(W.to(DEV), G)
    b = (torch.randn(N, generator=g) * 0.5).to(torch.float16).to(DEV)
    return X.to(DEV), qw, s, z, b


def test_concurrent_threads_match_sequential():
    from w4a16 import w4a16_matmul
    from w4a16.hip_kernel import plan_for, w4a16_linear

    data = []
    for i, (M, K, N, G, kern, split) in enumerate(CASES):
        p = plan_for(M, N, K, G).as_dict()
        assert p["kernel_name"] == kern, (M, K, N, G, p)
        if split is not None:
            assert p["split_k"] == split, (M, K, N, G, p)
        else:
            assert p["split_k"] > 1 and p["workspace_bytes"] > 0, (M, K, N, G, p)
        X, qw, s, z, b = _inputs(i, M, K, N, G)
        if i == 1:
            # fractional zero-points: the any-zero kernel forms, and a zeros
            # tensor the thread sees unchecked (its own copy)
            z = z + torch.tensor(0.5, dtype=torch.float16, device=DEV)
        log(f"threads: sequential M={M} K={K} N={N} G={G} plan={kern} split={p['split_k']}")
        y = w4a16_matmul(X, qw, s, z.clone(), G)
        yb = w4a16_linear(X, qw, s, z.clone(), b, G)
        ref = O.reference_w4a16(np_(X), np_(qw), np_(s), np_(z), G)
        assert_gemm_close(y, ref, f"threads sequential case {i}")
        assert torch.equal(yb, y + b)
        data.append((X, qw, s, z.clone(), b, G, y, yb))
    torch.cuda.synchronize()

    errors: list[str] = []
    start = threading.Barrier(len(CASES), timeout=60)

    def run(i: int) -> None:
        X, qw, s, z, b, G, y, yb = data[i]
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                start.wait()
                outs = []
                for r in range(REPS):
                    outs.append(w4a16_matmul(X, qw, s, z, G))
                    outs.append(w4a16_linear(X, qw, s, z, b, G))
            stream.synchronize()
            for r, o in enumerate(outs):
                want = y if r % 2 == 0 else yb
                if not torch.equal(o, want):
                    d = (o.float() - want.float()).abs().max().item()
                    errors.append(f"case {i} call {r}: differs from the sequential result "
                                  f"(max |diff| {d:.3g})")
        except Exception as e:  # reported on the main thread
            errors.append(f"case {i}: {type(e).__name__}: {e}")

    log(f"threads: {len(CASES)} threads x {2 * REPS} calls, one stream each")
    threads = [threading.Thread(target=run, args=(i,)) for i in range(len(CASES))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "a thread did not finish"
    torch.cuda.synchronize()
    assert not errors, "\n".join(errors)


def test_threads_zero_point_check_once_per_tensor_version():
    """Several threads ask for the same unchecked zeros tensor's form at once:
    each gets the right answer (the GPU check may run more than once, its
    result is the same), and a later in-place change is checked again."""
    from w4a16.hip_kernel import zeros_need_any_form

    z = torch.randint(0, 16, (64, 4096), dtype=torch.int32).to(torch.float16).to(DEV)
    torch.cuda.synchronize()
    answers: list[bool] = []
    lock = threading.Lock()
    start = threading.Barrier(4, timeout=60)

    def ask() -> None:
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                start.wait()
                a = zeros_need_any_form(z)
        except Exception as e:  # reported on the main thread
            a = f"{type(e).__name__}: {e}"
        with lock:
            answers.append(a)

    log("threads: zeros check from 4 threads")
    threads = [threading.Thread(target=ask) for _ in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert answers == [False] * 4, answers
    z[3, 7] = 2.5                      # a new version: checked again
    assert zeros_need_any_form(z) is True
    assert np.isclose(float(np_(z)[3, 7]), 2.5)

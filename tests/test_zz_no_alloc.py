"""w4a16_gemm_f16_noalloc: the allocation-free GEMM entry point.

It has no reference counterpart (callers that cannot allocate: HIP graph
capture, serving loops).  Its split-K partials live in the library's static
device scratch; every call is compared, through the C ABI, with the
workspace-taking entry point w4a16_gemm_f16_strided run with the same plan
(bit for bit: the same kernels, the same fixed-order split sums), and with
the oracle to the GEMM tolerance, on two calls in a row, the second smaller.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from _helpers import DEV, assert_gemm_close, log, np_, oracle_cols, sample_cols
from oracle import w4a16_oracle as O

ERR_WORKSPACE = -4


def _lib():
    from w4a16 import _lib

    return _lib, _lib.load()


def _case(M, K, N, G, seed):
    from w4a16 import quantize_weight

    g = torch.Generator().manual_seed(seed)
    X = torch.randn(M, K, generator=g).to(torch.float16)
    W = (torch.randn(K, N, generator=g) * 0.05).to(torch.float16)
    qw, s, z = quantize_weight(W.to(DEV), G)
    return X.to(DEV), qw, s, z


def _noalloc(X, qw, s, z, G, plan=None, bias=None):
    L, lib = _lib()
    M, K = X.shape
    N = qw.shape[1]
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV)
    rc = lib.w4a16_gemm_f16_noalloc(
        None if plan is None else ctypes.byref(plan), X.data_ptr(), K, qw.data_ptr(),
        s.data_ptr(), z.data_ptr(), None if bias is None else bias.data_ptr(), y.data_ptr(), N,
        M, N, K, G, torch.cuda.current_stream().cuda_stream)
    return rc, y


def _strided(X, qw, s, z, G, plan, bias=None):
    """The existing entry point with the same plan and a workspace of its own."""
    L, lib = _lib()
    M, K = X.shape
    N = qw.shape[1]
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV)
    ws_bytes = max(int(plan.workspace_bytes), 256)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    rc = lib.w4a16_gemm_f16_strided(
        ctypes.byref(plan), X.data_ptr(), K, qw.data_ptr(), s.data_ptr(), z.data_ptr(),
        None if bias is None else bias.data_ptr(), y.data_ptr(), N, M, N, K, G,
        ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, L.status_text(rc)
    return y


def _plan_fitting(M, N, K, G):
    """The plan the allocation-free entry point takes by itself: the automatic
    plan with the most k-splits whose partials fit the scratch."""
    from w4a16 import _lib as L
    from w4a16.hip_kernel import plan_for

    p = plan_for(M, N, K, G)
    s = p.split_k
    while p.workspace_bytes > L.NOALLOC_SCRATCH_BYTES and s > 1:
        s -= 1
        p = plan_for(M, N, K, G, int(p.kernel), s)
    return p


def _check(X, qw, s, z, G, what, bias=None, sampled=False):
    M, K = X.shape
    N = qw.shape[1]
    p = _plan_fitting(M, N, K, G)
    log(f"noalloc {what} M={M} K={K} N={N} G={G} kernel={p.as_dict()['kernel_name']} "
        f"cfg={p.tile_cfg} split={p.split_k}")
    rc, y = _noalloc(X, qw, s, z, G, bias=bias)
    torch.cuda.synchronize()
    assert rc == 0, rc
    ref_entry = _strided(X, qw, s, z, G, p, bias=bias)
    torch.cuda.synchronize()
    assert torch.equal(y, ref_entry), f"{what}: differs from w4a16_gemm_f16_strided"
    if bias is None:
        if sampled:
            cols = sample_cols(N, 64)
            assert_gemm_close(y[:, cols], oracle_cols(X, qw, s, z, G, cols), what)
        else:
            assert_gemm_close(y, O.reference_w4a16(np_(X), np_(qw), np_(s), np_(z), G), what)
    return p


@pytest.mark.gpu
@pytest.mark.parametrize("big,small", [
    ((1, 14336, 1024, 128), (1, 8192, 512, 64)),       # GEMV, automatic 4-way split
    ((32, 4096, 28672, 128), (32, 4096, 8192, 128)),   # streamed 32-row tiles, split
    ((256, 8192, 2048, 64), (128, 4096, 1024, 64)),    # streamed 128-row tiles, split
    ((8, 4096, 4096, 128), (3, 1024, 256, 32)),        # no split (skinny MFMA)
])
def test_noalloc_matches_workspace_entry(big, small):
    """Two calls in a row, the second with a smaller input: both equal the
    workspace entry point bit for bit, and the oracle within tolerance."""
    Xb, qwb, sb, zb = _case(*big, seed=1)
    pb = _check(Xb, qwb, sb, zb, big[3], "first call")
    Xs, qws, ss, zs = _case(*small, seed=2)
    _check(Xs, qws, ss, zs, small[3], "second call (smaller)")
    # and the first shape again, after the smaller call left its partials
    _check(Xb, qwb, sb, zb, big[3], "third call (first shape again)")
    if big[0] in (1, 32, 256):
        assert pb.split_k > 1, "the case must exercise the scratch"


@pytest.mark.gpu
def test_noalloc_explicit_plans_and_bias():
    """Forced k-splits of every split-capable family through an explicit plan,
    with a fused bias: equal to the workspace entry point with that plan."""
    from w4a16.hip_kernel import plan_for

    M, K, N, G = 16, 8192, 2048, 128
    X, qw, s, z = _case(M, K, N, G, seed=3)
    bias = (torch.randn(N) * 0.5).to(torch.float16).to(DEV)
    for kern, split, cfg in (("gemv", 4, None), ("mfma", 4, 12), ("mfma", 3, 13), ("mfma", 2, 11)):
        Mx = 4 if kern == "gemv" else M
        p = plan_for(Mx, N, K, G, kern, split)
        if cfg is not None:
            p.tile_cfg = cfg
        log(f"noalloc explicit {kern} cfg={p.tile_cfg} split={p.split_k} M={Mx}")
        assert p.split_k > 1 and 0 < p.workspace_bytes <= (16 << 20)
        rc, y = _noalloc(X[:Mx], qw, s, z, G, plan=p, bias=bias)
        torch.cuda.synchronize()
        assert rc == 0, rc
        assert torch.equal(y, _strided(X[:Mx], qw, s, z, G, p, bias=bias))


@pytest.mark.gpu
def test_noalloc_large_layer_fits_scratch():
    """A prefill layer whose automatic plan's partials (4 x 256 x 8192 fp32 =
    32 MiB) exceed the scratch runs with fewer k-splits instead; equal to the
    workspace entry point with that plan."""
    from w4a16 import _lib as L
    from w4a16.hip_kernel import plan_for

    M, K, N, G = 256, 28672, 8192, 128
    assert plan_for(M, N, K, G).workspace_bytes > L.NOALLOC_SCRATCH_BYTES
    X, qw, s, z = _case(M, K, N, G, seed=4)
    p = _check(X, qw, s, z, G, "large layer", sampled=True)
    assert p.workspace_bytes <= L.NOALLOC_SCRATCH_BYTES


def test_noalloc_rejects_plan_beyond_scratch():
    """An explicit plan whose partials exceed the scratch is refused before
    anything touches a device (CPU test: no GPU needed)."""
    L, lib = _lib()
    M, K, N, G = 64, 8192, 28672, 128
    p = L.Plan()
    p.kernel, p.split_k, p.tile_cfg, p.tile_m, p.tile_n = 2, 4, 13, 64, 256
    assert 4 * M * N * 4 > L.NOALLOC_SCRATCH_BYTES
    rc = lib.w4a16_gemm_f16_noalloc(ctypes.byref(p), None, K, None, None, None, None, None, N,
                                    M, N, K, G, None)
    assert rc == ERR_WORKSPACE
    assert lib.w4a16_gemm_f16_noalloc(None, None, 64, None, None, None, None, None, N,
                                      M, N, 64, 48, None) == -3     # G does not divide K


# A fresh process whose first call into the library is a split-K noalloc call
# made while torch captures a HIP graph: the library's code object, and with
# it the static scratch, is loaded and the scratch's address resolved inside
# the capture.  The inputs are made with torch alone (no library kernel runs
# before the capture).
_CAPTURE_CHILD = r"""
import ctypes, sys
sys.path[:0] = [sys.argv[1], sys.argv[2]]
import torch
from w4a16 import _lib
lib = _lib.load()
dev = "cuda"
M, K, N, G = 1, 14336, 1024, 128          # automatic plan: GEMV, 4-way split
gen = torch.Generator(device=dev).manual_seed(0)
X = torch.randn(M, K, device=dev, generator=gen).half()
qw = torch.randint(-2**31, 2**31 - 1, (K // 8, N), dtype=torch.int32, device=dev, generator=gen)
s = (torch.rand(K // G, N, device=dev, generator=gen) * 0.01 + 0.001).half()
z = torch.randint(0, 16, (K // G, N), device=dev, generator=gen).half()
p = _lib.plan(M, N, K, G)
assert p.split_k > 1, p.as_dict()

def call(x, w, sc, zr, y, m, n, k):
    return lib.w4a16_gemm_f16_noalloc(None, x.data_ptr(), k, w.data_ptr(), sc.data_ptr(),
                                      zr.data_ptr(), None, y.data_ptr(), n, m, n, k, G,
                                      torch.cuda.current_stream().cuda_stream)

y_cap = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
side = torch.cuda.Stream()
with torch.cuda.graph(graph, stream=side):
    rc = call(X, qw, s, z, y_cap, M, N, K)
assert rc == 0, ("capture", rc)
# eager result, and a smaller split call that leaves other partials in the scratch
y_eager = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
before = torch.cuda.memory_allocated()
assert call(X, qw, s, z, y_eager, M, N, K) == 0
assert torch.cuda.memory_allocated() == before, "the call allocated through torch"
K2, N2 = 8192, 512
X2 = torch.randn(M, K2, device=dev, generator=gen).half()
qw2 = torch.randint(-2**31, 2**31 - 1, (K2 // 8, N2), dtype=torch.int32, device=dev, generator=gen)
s2 = (torch.rand(K2 // G, N2, device=dev, generator=gen) * 0.01).half()
z2 = torch.randint(0, 16, (K2 // G, N2), device=dev, generator=gen).half()
y2 = torch.empty(M, N2, dtype=torch.float16, device=dev)
torch.cuda.synchronize()
assert bool(torch.isfinite(y_eager).all())
for rep in range(3):
    y_cap.fill_(float("nan"))
    assert call(X2, qw2, s2, z2, y2, M, N2, K2) == 0
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(y_cap, y_eager), ("replay", rep)
print("CAPTURE-CHILD-OK", flush=True)
"""


@pytest.mark.gpu
def test_noalloc_first_call_inside_graph_capture():
    """In a fresh process, the library's first call is a split-K noalloc call
    under HIP-graph capture; three replays, each after an eager split call of
    another shape, equal the eager result bit for bit, and an eager call
    leaves torch's allocation counter unchanged."""
    import os
    import subprocess
    import sys

    root = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
    pkg = os.path.join(root, "w4a16-dequant-fused-matmul-kernel_amd")
    log("noalloc: first call inside graph capture (child process)")
    res = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, root, pkg], capture_output=True,
                         text=True, timeout=150)
    assert res.returncode == 0 and "CAPTURE-CHILD-OK" in res.stdout, (
        f"rc={res.returncode}\n{res.stdout[-2000:]}\n{res.stderr[-3000:]}")

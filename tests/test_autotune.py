"""Measured plan selection (w4a16.autotune): the candidate list on the CPU,
tuned calls against the oracle and the static planner on the GPU.

The reference autotunes its Triton kernel per (M, N, K, group_size)
(w4a16-kernel/src/w4a16/triton_kernel.py:41-62); here tuning is opt-in and
picks among the library's own plans, each of which the parity tests cover.
"""
from __future__ import annotations

import json

import pytest
import torch

from _helpers import DEV, assert_gemm_close, log, np_
from oracle import w4a16_oracle as O


@pytest.mark.parametrize("M,K,N,G", [(1, 4096, 4096, 128), (2, 28672, 8192, 64), (8, 4096, 28672, 128),
                                     (24, 4096, 4100, 32), (512, 14336, 4096, 128),
                                     (300, 4160, 1028, 64)])
def test_candidates_start_with_the_static_plan(M, K, N, G):
    """The static plan comes first, no plan appears twice, and every candidate
    names a family and configuration the library has."""
    from w4a16 import _lib, autotune

    c = autotune.candidates(M, N, K, G)
    static = _lib.plan(M, N, K, G)
    assert c[0][0] == "static"
    assert (c[0][1].kernel, c[0][1].split_k, c[0][1].tile_cfg) == (static.kernel, static.split_k,
                                                                  static.tile_cfg)
    keys = [(p.kernel, p.split_k, p.tile_cfg, p.tile_m, p.tile_n) for _, p in c]
    assert len(keys) == len(set(keys))
    for _, p in c:
        assert p.flags == 0
        if p.kernel == _lib.KERNEL_GEMV:
            assert M <= 8 and p.tile_n in (16, 32, 64, 128, 256)
            assert p.tile_cfg in _lib.GEMV_CONFIGS + _lib.GEMV_MFMA_CONFIGS
        elif p.kernel == _lib.KERNEL_SKINNY:
            assert M <= 64 and p.tile_cfg in _lib.SKINNY_CONFIGS
        elif p.kernel == _lib.KERNEL_MFMA:
            assert p.tile_cfg in _lib.MFMA_CONFIGS
            assert p.split_k == 1 or p.tile_cfg in _lib.MFMA_SPLIT_CONFIGS
    if M <= 2:
        assert any(p.kernel == _lib.KERNEL_GEMV and p.tile_cfg == 7 for _, p in c)
    if M > 64 and K % 256 == 0:
        assert {11, 14} <= {p.tile_cfg for _, p in c if p.kernel == _lib.KERNEL_MFMA}


def test_cache_file_roundtrip(tmp_path, monkeypatch):
    """Tuned plans load from the cache file by key and come back as plans."""
    from w4a16 import _lib, autotune

    path = tmp_path / "tuned.json"
    p = _lib.plan(16, 4096, 4096, 128, _lib.KERNEL_SKINNY)
    key = "dev|16x4096x4096|G128|ld4096,4096|intz"
    path.write_text(json.dumps({key: {"plan": autotune._plan_fields(p), "us": 7.0}}))
    monkeypatch.setenv("W4A16_AUTOTUNE_CACHE", str(path))
    monkeypatch.setitem(autotune._STATE, "loaded", False)
    autotune.clear()
    autotune._load_file()
    got = autotune._plan_from(autotune.tuned()[key]["plan"])
    assert (got.kernel, got.tile_cfg, got.tile_m, got.split_k) == (p.kernel, p.tile_cfg, p.tile_m,
                                                                   p.split_k)
    autotune.clear()
    monkeypatch.setitem(autotune._STATE, "loaded", False)


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N,G", [(1, 4096, 4096, 128), (2, 8192, 1024, 64), (16, 4096, 4096, 128),
                                     (48, 2048, 5120, 32), (300, 4096, 2048, 128)])
def test_autotuned_calls_match_oracle(M, K, N, G, tmp_path, monkeypatch):
    """With tuning on, the first call of a shape tunes it and every call matches
    the oracle; the tuned plan is cached (and written to the cache file) and
    reused, also under HIP-graph capture."""
    from w4a16 import autotune, quantize_weight, w4a16_matmul

    monkeypatch.setenv("W4A16_AUTOTUNE_CACHE", str(tmp_path / "tuned.json"))
    monkeypatch.setitem(autotune._STATE, "loaded", False)
    autotune.clear()
    autotune.enable(True)
    try:
        g = torch.Generator().manual_seed(M + K)
        X = torch.randn(M, K, generator=g).to(torch.float16).to(DEV)
        W = (torch.randn(K, N, generator=g) * 0.05).to(torch.float16)
        qw, s, z = quantize_weight(W.to(DEV), G)
        ref = O.reference_w4a16(np_(X), np_(qw), np_(s), np_(z), G)
        log(f"autotune M={M} K={K} N={N} G={G}")
        y1 = w4a16_matmul(X, qw, s, z, G)
        assert_gemm_close(y1, ref, "tuned first call")
        tuned = autotune.tuned()
        assert len(tuned) == 1
        entry = next(iter(tuned.values()))
        assert entry["us"] <= entry["static_us"] * 1.0001
        assert json.loads((tmp_path / "tuned.json").read_text()).keys() == tuned.keys()
        y2 = w4a16_matmul(X, qw, s, z, G)
        assert torch.equal(y1, y2)
        assert len(autotune.tuned()) == 1
        out = torch.empty_like(y1)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            w4a16_matmul(X, qw, s, z, G, out=out)
        for _ in range(2):
            out.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, y1)
    finally:
        autotune.enable(False)
        autotune.clear()
        monkeypatch.setitem(autotune._STATE, "loaded", False)

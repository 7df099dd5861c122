"""GPU parity: quantise / pack / unpack / dequantise kernels vs the CPU oracle.

Bit-exact comparisons (int32 words, fp16 bit patterns including -0.0
zero-points) against ``oracle/w4a16_oracle.py`` on the same inputs; mirrors the
reference's test_quant.py (w4a16-kernel/tests/test_quant.py) on the device.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from _helpers import DEV, log, np_
from oracle import w4a16_oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")


def _assert_quant_equal(W: torch.Tensor, G: int, what: str):
    from w4a16 import quantize_weight

    qw, s, z = quantize_weight(W.to(DEV), G)
    rq, rs, rz = O.quantize_weight(np_(W), G)
    assert qw.dtype == torch.int32 and s.dtype == torch.float16 and z.dtype == torch.float16
    assert np.array_equal(np_(qw), rq), f"{what}: qweight differs"
    assert np.array_equal(np_(s).view(np.uint16), rs.view(np.uint16)), f"{what}: scales differ"
    assert np.array_equal(np_(z).view(np.uint16), rz.view(np.uint16)), f"{what}: zeros differ"
    return qw, s, z


def test_quantize_known_answers():
    from w4a16 import pack_int4, quantize_weight, unpack_int4

    for c in json.load(open(GOLDEN)):
        log(c["name"])
        if c["kind"] == "pack":
            q = torch.tensor(c["codes"], dtype=torch.int32).reshape(c["K"], c["N"]).to(DEV)
            w = pack_int4(q)
            assert (np_(w).view(np.uint32).reshape(-1).tolist()) == c["words_u32"]
            assert torch.equal(unpack_int4(w), q)
        else:
            W = torch.tensor(c["W"], dtype=torch.float16).reshape(c["K"], c["N"]).to(DEV)
            qw, s, z = quantize_weight(W, c["G"])
            assert np_(unpack_int4(qw)).reshape(-1).tolist() == c["codes"]
            if "zeros_bits" in c:
                assert np_(z).view(np.uint16).reshape(-1).tolist() == c["zeros_bits"]
            if "scales_bits" in c:
                assert np_(s).view(np.uint16).reshape(-1).tolist() == c["scales_bits"]


@pytest.mark.parametrize("K,N,G", [
    (1024, 1024, 128),   # C1 shape
    (256, 64, 32),
    (128, 40, 64),
    (64, 33, 16),        # N % 4 != 0: one column per thread
    (8, 1, 4),           # G < 8: packed words straddle groups
    (24, 12, 12),        # G % 8 != 0
    (4096, 512, 128),
])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_quantize_bit_exact_random(K, N, G, dtype):
    log(f"quantize K={K} N={N} G={G} {dtype}")
    g = torch.Generator().manual_seed(K * 31 + N * 7 + G)
    W = (torch.randn(K, N, generator=g) * 0.05).to(dtype)
    _assert_quant_equal(W, G, f"K={K} N={N} G={G}")


def test_quantize_special_values():
    """Constant groups (scale 1), exact ties, zero minima (-0.0 zero-point), both
    zero signs, fp16 subnormals, huge ranges, and ties of W/scale at .5."""
    log("quantize special values")
    K, N, G = 64, 16, 32
    W = torch.zeros(K, N, dtype=torch.float16)
    W[:, 0] = 3.0
    W[:, 1] = -2.5
    W[:32, 2] = torch.tensor([0, 0.03125, 0.09375, 0.15625, 0.9375, 0.5, 0.25, 0.46875] * 4)
    W[:8, 3] = torch.tensor([0.0, -0.0, 1.0, 0.5, 0.25, 0.75, 0.125, 0.375])
    W[:8, 4] = torch.tensor([-0.0, 0.0, 1.0, 0.5, 0.25, 0.75, 0.125, 0.375])
    W[:, 5] = torch.tensor([6e-8, 1.2e-7, 3e-6, 6.1e-5] * 16, dtype=torch.float16)
    W[:, 6] = torch.linspace(-60000, 60000, K).to(torch.float16)
    W[:, 7] = -1e-3
    g = torch.Generator().manual_seed(5)
    W[:, 8:] = (torch.randn(K, 8, generator=g) * 1e-4).to(torch.float16)
    _assert_quant_equal(W, G, "special values")
    _assert_quant_equal(W, 8, "special values G=8")


@pytest.mark.parametrize("K,N,G", [
    (128, 68, 32),       # 4 columns per thread: block columns 0-63, tail 64-67
    (64, 33, 8),         # one column per thread: block 0-31, tail column 32
    (64, 70, 16),
    (48, 40, 12),        # G % 8 != 0 kernel
    (512, 1, 32),        # N = 1, G >= 32: torch's inner reduction
    (1024, 1, 64),
    (576, 1, 36),        # N = 1 through the G % 8 != 0 kernel
    (4096, 1, 4096),     # one group
    (256, 1, 16),        # N = 1, G < 32: first zero
])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_quantize_mixed_zero_minima(K, N, G, dtype):
    """Groups whose minimum is a zero and that hold both +0.0 and -0.0 at random
    rows: the zero-point's sign bit follows which zero torch's CPU amin returns
    (block / tail columns, N = 1 lanes), bit-exact against the oracle."""
    log(f"quantize mixed zero minima K={K} N={N} G={G} {dtype}")
    rng = np.random.default_rng(K * 13 + N * 7 + G)
    ng = K // G
    W = (np.abs(rng.standard_normal((ng, G, N))) * 0.1 + 0.01).astype(np.float32)
    for _ in range(3):
        rows = rng.integers(0, G, (ng, N))
        gi, ni = np.nonzero(rng.random((ng, N)) < 0.85)
        W[gi, rows[gi, ni], ni] = np.where(rng.integers(0, 2, gi.size) == 1, -0.0, 0.0)
    Wt = torch.from_numpy(W.reshape(K, N)).to(dtype)
    _, _, z = _assert_quant_equal(Wt, G, f"mixed zeros K={K} N={N} G={G}")
    if ng * N >= 16:
        zb = np_(z).view(np.uint16)
        assert (zb == 0x8000).any() and (zb == 0x0000).any()   # both zero signs occur


def test_quantize_fp32_tiny_and_denormal_ranges():
    log("quantize fp32 tiny ranges")
    K, N, G = 64, 8, 32
    g = torch.Generator().manual_seed(9)
    W = torch.randn(K, N, generator=g) * 1e-30
    W[:, 3] = torch.randn(K, generator=g) * 1e-39    # fp32 subnormals
    W[:, 4] = torch.randn(K, generator=g) * 1e30
    _assert_quant_equal(W, G, "fp32 tiny/huge")


def test_quantize_non_finite_raises():
    from w4a16 import quantize_weight

    for bad in (float("inf"), float("-inf"), float("nan")):
        log(f"quantize non-finite {bad}")
        W = torch.zeros(64, 8, dtype=torch.float16, device=DEV)
        W[5, 3] = bad
        with pytest.raises(AssertionError):
            quantize_weight(W, 32)


def test_quantize_cpu_input_returns_cpu():
    """CPU input: computed on the GPU, returned on the CPU, same bits."""
    from w4a16 import quantize_weight

    log("quantize cpu staging")
    W = (torch.randn(256, 64) * 0.1).to(torch.float16)
    qw, s, z = quantize_weight(W, 64)
    assert qw.device.type == "cpu" and s.device.type == "cpu"
    rq, rs, rz = O.quantize_weight(W.numpy(), 64)
    assert np.array_equal(qw.numpy(), rq) and np.array_equal(s.numpy().view(np.uint16), rs.view(np.uint16))


@pytest.mark.parametrize("cfg", ["C4", "C5a", "C5b"])
def test_quantize_full_size_layers(cfg):
    """Full-size weights of the large configs, quantised on the GPU; every group
    of three column slices compared bit-exact with the oracle (quantisation is
    independent per column), plus size-independent checks on all columns."""
    from w4a16 import quantize_weight, dequantize_weight
    from w4a16 import workloads as wl

    if cfg == "C4":
        case = wl.CONFIGS["C4"][0]
        Gs = [case.G]
    else:
        K, N = (8192, 28672) if cfg == "C5a" else (28672, 8192)
        case = [c for c in wl.CONFIGS["C5"] if c.K == K and c.N == N and c.M == 1][0]
        Gs = [32, 64, 128]
    W = wl.make_w(case)
    Wd = W.to(DEV)
    Kdim, N = W.shape
    for G in Gs:
        log(f"quantize full {cfg} K={Kdim} N={N} G={G}")
        qw, s, z = quantize_weight(Wd, G)
        # N and the slice width are multiples of 32, so each column is in a whole
        # 32-column block of both the slice and the full weight (zero-sign rule)
        for a, b in ((0, 256), (N // 2 - 128, N // 2 + 128), (N - 256, N)):
            rq, rs, rz = O.quantize_weight(W[:, a:b].numpy(), G)
            assert np.array_equal(np_(qw[:, a:b]), rq), (cfg, G, a)
            assert np.array_equal(np_(s[:, a:b]).view(np.uint16), rs.view(np.uint16)), (cfg, G, a)
            assert np.array_equal(np_(z[:, a:b]).view(np.uint16), rz.view(np.uint16)), (cfg, G, a)
        # all columns: zero-points are integers in [0, 15]; dequant error below one step
        zf = z.float()
        assert bool(((zf >= 0) & (zf <= 15) & (zf == zf.round())).all())
        dq = dequantize_weight(qw, s, z, G).float()
        step = s.float().repeat_interleave(G, dim=0)
        err = (dq - Wd.float()).abs()
        assert bool((err <= step * 1.01 + 1e-6).all())
        del qw, s, z, dq, step, err


# --------------------------------------------------------------------------- #
# pack / unpack / dequant                                                      #
# --------------------------------------------------------------------------- #
@pytest.mark.parametrize("K", [8, 64, 128, 4096])
@pytest.mark.parametrize("N", [1, 16, 4096])
def test_pack_unpack_roundtrip(K, N):
    """Reference test_quant.py:21-31 on the device, words compared with the oracle."""
    from w4a16 import pack_int4, unpack_int4

    log(f"pack/unpack K={K} N={N}")
    x = torch.randint(0, 16, (K, N), dtype=torch.int32, device=DEV)
    packed = pack_int4(x)
    assert packed.shape == (K // 8, N) and packed.dtype == torch.int32
    assert np.array_equal(np_(packed), O.pack_int4(np_(x)))
    restored = unpack_int4(packed, K)
    assert restored.shape == (K, N)
    assert torch.equal(restored, x)


def test_pack_extremes_and_position():
    from w4a16 import pack_int4, unpack_int4

    for val in (0, 15):
        x = torch.full((16, 8), val, dtype=torch.int32, device=DEV)
        assert torch.equal(unpack_int4(pack_int4(x)), x)
    x = torch.zeros((8, 1), dtype=torch.int32, device=DEV)
    x[3, 0] = 0xA
    assert int(pack_int4(x)[0, 0]) == (0xA << 12)


@pytest.mark.parametrize("bad", [16, -1, 1 << 20])
def test_pack_range_assertion(bad):
    from w4a16 import pack_int4

    x = torch.zeros((16, 4), dtype=torch.int32, device=DEV)
    x[9, 2] = bad
    with pytest.raises(AssertionError):
        pack_int4(x)


@pytest.mark.parametrize("K,N,G", [(128, 256, 64), (4096, 512, 128), (64, 33, 32), (24, 12, 12)])
def test_dequant_bit_exact(K, N, G):
    from w4a16 import dequantize_weight

    log(f"dequant K={K} N={N} G={G}")
    g = torch.Generator().manual_seed(K + N + G)
    q = torch.randint(0, 16, (K, N), generator=g, dtype=torch.int32)
    qw = torch.from_numpy(O.pack_int4(q.numpy()))
    s = (torch.rand(K // G, N, generator=g) * 0.1).to(torch.float16)
    z = torch.randint(0, 16, (K // G, N), generator=g).to(torch.float16)
    z[0, 0] = -0.0
    z[-1, -1] = 3.5      # non-integer zero-point: fp16 subtraction semantics
    out = dequantize_weight(qw.to(DEV), s.to(DEV), z.to(DEV), G)
    ref = O.dequantize_weight(qw.numpy(), s.numpy(), z.numpy(), G)
    assert np.array_equal(np_(out).view(np.uint16), ref.view(np.uint16))


def test_quant_dequant_roundtrip_error():
    """Reference test_quant.py:71-90 on the device: mean relative error < 0.15."""
    from w4a16 import dequantize_weight, quantize_weight

    for G in (64, 128):
        torch.manual_seed(1)
        W = torch.randn(4096, 1024, dtype=torch.float16, device=DEV)
        qw, s, z = quantize_weight(W, G)
        dq = dequantize_weight(qw, s, z, G)
        rel = ((dq.float() - W.float()).abs().mean() / W.float().abs().mean()).item()
        assert rel < 0.15

"""Pins for the CPU oracle (``oracle/w4a16_oracle.py``), all on the CPU.

Every check here is independent of the oracle's own code: known answers from
the reference's spec and tests, hand-derived corner cases, exact rational
arithmetic, numpy's own fp16 arithmetic, and float64 brute force.  Each one is
chosen so that a plausible mistake (a dropped term, a transposed operand, an
fp16 instead of an fp32 scale, round-half-away instead of half-even, losing the
-0.0 zero-point, a nibble-order swap) fails it.
"""
from __future__ import annotations

import json
import os
from fractions import Fraction

import numpy as np
import pytest

from oracle import w4a16_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _u32(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.int32).view(np.uint32)


# --------------------------------------------------------------------------- #
# packing                                                                      #
# --------------------------------------------------------------------------- #
def test_pack_spec_word():
    """Spec W4A16_SPEC.md:148-165: codes [8,0,15,4,1,7,2,12] -> 0xC2714F08."""
    q = np.array([8, 0, 15, 4, 1, 7, 2, 12], dtype=np.int32).reshape(8, 1)
    w = O.pack_int4(q)
    assert w.dtype == np.int32 and w.shape == (1, 1)
    assert int(_u32(w)[0, 0]) == 0xC2714F08
    assert int(w[0, 0]) == -1032761592
    # spec's unpack checks: nibble 0 -> 8, nibble 2 -> 15, nibble 7 -> 12
    u = O.unpack_int4(w)
    assert u[:, 0].tolist() == [8, 0, 15, 4, 1, 7, 2, 12]


def test_pack_nibble_position():
    """Reference test_quant.py:41-47: x[3,0]=0xA -> word 0xA << 12."""
    q = np.zeros((8, 1), dtype=np.int32)
    q[3, 0] = 0xA
    assert int(O.pack_int4(q)[0, 0]) == 0xA << 12


@pytest.mark.parametrize("val,word", [(0, 0), (15, -1)])
def test_pack_extremes(val, word):
    """Reference test_quant.py:34-38: all-0 and all-15 (sign bit set) words."""
    q = np.full((16, 8), val, dtype=np.int32)
    w = O.pack_int4(q)
    assert (w == word).all()
    assert (O.unpack_int4(w) == q).all()


@pytest.mark.parametrize("K", [8, 64, 128, 4096])
@pytest.mark.parametrize("N", [1, 16, 4096])
def test_pack_unpack_roundtrip(K, N):
    """Reference test_quant.py:21-31 grid."""
    rng = np.random.default_rng(K * 7 + N)
    q = rng.integers(0, 16, size=(K, N), dtype=np.int32)
    w = O.pack_int4(q)
    assert w.shape == (K // 8, N) and w.dtype == np.int32
    assert (O.unpack_int4(w, K) == q).all()


def test_pack_matches_bitwise_closed_form():
    """word = sum_j q[8i+j] * 16**j, computed with Python integers."""
    rng = np.random.default_rng(3)
    q = rng.integers(0, 16, size=(32, 5), dtype=np.int32)
    w = _u32(O.pack_int4(q))
    for i in range(4):
        for n in range(5):
            ref = sum(int(q[8 * i + j, n]) * 16 ** j for j in range(8))
            assert int(w[i, n]) == ref


def test_pack_asserts():
    with pytest.raises(AssertionError):
        O.pack_int4(np.zeros((7, 4), dtype=np.int32))          # test_quant.py:50-52
    with pytest.raises(AssertionError):
        O.pack_int4(np.full((8, 1), 16, dtype=np.int32))       # quant.py:62-63
    with pytest.raises(AssertionError):
        O.pack_int4(np.full((8, 1), -1, dtype=np.int32))


# --------------------------------------------------------------------------- #
# quantize                                                                     #
# --------------------------------------------------------------------------- #
def test_quantize_spec_example():
    """Spec W4A16_SPEC.md:84-105: W=[0.1,-0.3,0.5,-0.1], G=4 -> zero 6, q=[8,0,15,4],
    dequant [0.1067, -0.3200, 0.4800, -0.1067].  K must be a multiple of 8, so the
    example is the first of two groups of 4."""
    W = np.array([0.1, -0.3, 0.5, -0.1, 1.0, 2.0, 3.0, 4.0], dtype=np.float16).reshape(8, 1)
    qw, s, z = O.quantize_weight(W, group_size=4)
    q = O.unpack_int4(qw)[:, 0]
    assert q[:4].tolist() == [8, 0, 15, 4]
    assert float(z[0, 0]) == 6.0
    # scale = (0.5 - (-0.3)) / 15 from the fp16 inputs of the worked example
    # (W4A16_SPEC.md:84-100): fp32(fp16(0.5) - fp16(-0.3)) / 15 rounds to fp16 0x2ad4
    assert int(s.view(np.uint16)[0, 0]) == 0x2AD4
    dq = O.dequantize_weight(qw, s, z, 4)[:4, 0].astype(np.float64)
    np.testing.assert_allclose(dq, [0.1067, -0.3200, 0.4800, -0.1067], atol=5e-4)
    # second group: [1,2,3,4]: scale = 3/15 = 0.2, zero = clamp(round(-5)) = 0,
    # q = clamp(round(W/0.2)) = [5, 10, 15, 15]
    assert q[4:].tolist() == [5, 10, 15, 15]
    assert float(z[1, 0]) == 0.0


def test_quantize_ties_half_even_and_negative_zero_point():
    """Hand-derived: gmin=0, gmax=0.9375 -> scale=0.0625 exactly.  W/scale hits
    exact .5 ties: 0.5->0, 1.5->2, 2.5->2, 7.5->8 under round-half-even (half-away
    would give 1,2,3,8).  round(-0/0.0625) = -0.0 and clamp keeps it: the
    zero-point is stored as fp16 0x8000."""
    W = np.array([0, 0.03125, 0.09375, 0.15625, 0.9375, 0.5, 0.25, 0.46875],
                 dtype=np.float16).reshape(8, 1)
    qw, s, z = O.quantize_weight(W, group_size=8)
    assert O.unpack_int4(qw)[:, 0].tolist() == [0, 0, 2, 2, 15, 8, 4, 8]
    assert int(_u32(qw)[0, 0]) == 0x848F2200
    assert float(s[0, 0]) == 0.0625
    assert int(z.view(np.uint16)[0, 0]) == 0x8000


def test_quantize_uses_fp32_scale_not_fp16():
    """gmax-gmin = 1 -> scale32 = fl(1/15) = 0.0666666701...; 0.5/scale32 = 7.4999996
    -> 7.  With the fp16-rounded scale 0.06665039 it would be 7.5018 -> 8."""
    W = np.array([0, 1.0, 0.5, 0.25, 0.75, 0.125, 0.375, 0.625], dtype=np.float16).reshape(8, 1)
    qw, s, z = O.quantize_weight(W, group_size=8)
    q = O.unpack_int4(qw)[:, 0].tolist()
    assert q[2] == 7
    assert float(s[0, 0]) == float(np.float16(np.float32(1) / np.float32(15)))


def test_quantize_constant_groups():
    """quant.py:129-132 guard: range 0 -> scale 1.  Constant 3.0: zero = clamp(-3)=0,
    q = 3, dequant exact (reference test_quant.py:93-100).  Constant 0.0: zero =
    round(-0/1) = -0.0 (0x8000), q = 0, dequant +0."""
    K, N, G = 128, 8, 64
    W = np.zeros((K, N), dtype=np.float16)
    W[:, 0] = 3.0
    qw, s, z = O.quantize_weight(W, G)
    assert (s == 1.0).all()
    assert (O.unpack_int4(qw)[:, 0] == 3).all()
    assert int(z.view(np.uint16)[0, 0]) == 0x0000
    assert (z.view(np.uint16)[:, 1:] == 0x8000).all()
    dq = O.dequantize_weight(qw, s, z, G)
    assert np.array_equal(dq.astype(np.float32), W.astype(np.float32))


def test_quantize_matches_exact_rational_arithmetic():
    """Every scale, zero and code of a random matrix equals the value obtained by
    exact rational arithmetic with one IEEE fp32 rounding per operation (true
    division, half-even rint).  Catches a reciprocal-multiply scale, a
    non-IEEE division, or an fp16 scale in the code computation."""
    rng = np.random.default_rng(11)
    K, N, G = 64, 24, 16
    W = (rng.standard_normal((K, N)) * 0.05).astype(np.float16)
    qw, s, z = O.quantize_weight(W, G)
    q = O.unpack_int4(qw)

    def f32(x: Fraction) -> np.float32:
        return np.float32(float(x))   # 53->24 bit double rounding is innocuous here

    for g in range(K // G):
        for n in range(N):
            col = [Fraction(float(v)) for v in W[g * G:(g + 1) * G, n]]
            gmax, gmin = max(col), min(col)
            sc = f32(Fraction(float(f32(gmax - gmin))) / 15)
            sc = sc if sc > 0 else np.float32(1)
            zr = np.rint(f32(-gmin / Fraction(float(sc))))
            zr = min(max(zr, 0.0), 15.0)
            assert np.float16(sc).view(np.uint16) == s.view(np.uint16)[g, n]
            assert float(z[g, n]) == zr
            for r in range(G):
                v = Fraction(float(W[g * G + r, n]))
                code = np.rint(f32(v / Fraction(float(sc)))) + np.float32(zr)
                code = int(min(max(code, 0.0), 15.0))
                assert q[g * G + r, n] == code, (g, n, r)


def test_quantize_reciprocal_scale_would_differ():
    """Sanity of the previous pin: for these inputs fl(d/15) and fl(d*fl(1/15))
    disagree somewhere, so the pin really separates the two readings."""
    rng = np.random.default_rng(11)
    d = (rng.standard_normal(100000) * 0.2).astype(np.float16).astype(np.float32)
    a = d / np.float32(15)
    b = d * (np.float32(1) / np.float32(15))
    assert (a.view(np.uint32) != b.view(np.uint32)).any()


def test_group_min_zero_sign_block_and_tail_columns():
    """A group whose minimum is a zero, holding both +0.0 and -0.0 (hand-derived):
    a column in a whole block of 32 takes the last zero in k order, a tail column
    (n >= 32 * (N // 32)) the first; zero-point = clamp(round(-gmin/scale)) then
    carries the opposite sign.  Scale and codes do not depend on it."""
    a = np.array([0.0, -0.0, 1.0, 0.5, 0.25, 0.75, 0.125, 0.375], dtype=np.float16)
    b = np.array([-0.0, 0.0, 1.0, 0.5, 0.25, 0.75, 0.125, 0.375], dtype=np.float16)
    W = np.tile(np.ones(8, np.float16)[:, None], (1, 33))
    W[:, 0], W[:, 1], W[:, 31], W[:, 32] = a, b, a, b
    qa, sa, za = O.quantize_weight(W, 8)
    zbits = za.view(np.uint16)[0]
    assert int(zbits[0]) == 0x0000    # block column, last zero -0.0 -> zero +0
    assert int(zbits[1]) == 0x8000    # block column, last zero +0.0 -> zero -0
    assert int(zbits[31]) == 0x0000
    assert int(zbits[32]) == 0x0000   # tail column, first zero -0.0 -> zero +0
    Wt = W[:, [32]]                   # N = 1: its only column is a tail column
    _, _, z1 = O.quantize_weight(Wt, 8)
    assert int(z1.view(np.uint16)[0, 0]) == 0x0000
    _, _, z1a = O.quantize_weight(W[:, [0]], 8)
    assert int(z1a.view(np.uint16)[0, 0]) == 0x8000   # first zero +0.0 -> zero -0
    # N = 1, G = 32: lane p % 8 of accumulator (p // 8) % 4; the lower lane wins,
    # then the higher accumulator
    c = np.ones((32, 1), np.float16)
    c[0], c[1] = 0.0, -0.0            # lanes 0 and 1: lane 0 (+0.0) -> zero -0
    assert int(O.quantize_weight(c, 32)[2].view(np.uint16)[0, 0]) == 0x8000
    c[1], c[8] = 1.0, -0.0            # lane 0 of accumulators 0 and 1: -0.0 -> zero +0
    assert int(O.quantize_weight(c, 32)[2].view(np.uint16)[0, 0]) == 0x0000
    # codes and scales are the same for both zero signs
    assert (qa[:, 0] == qa[:, 1]).all() and sa[0, 0] == sa[0, 1]


def _planted_zero_groups(rng, ng, G, N):
    """Positive groups with 1-3 zeros of random sign at random rows."""
    W = (np.abs(rng.standard_normal((ng, G, N))) + 0.5).astype(np.float32)
    for count in range(3):
        rows = rng.integers(0, G, (ng, N))
        sign = rng.integers(0, 2, (ng, N)).astype(bool)
        keep = rng.random((ng, N)) < 0.8
        gi, ni = np.nonzero(keep)
        W[gi, rows[gi, ni], ni] = np.where(sign[gi, ni], -0.0, 0.0)
    return W


@pytest.mark.parametrize("threads", [1, 8])
def test_group_min_matches_torch_amin(threads):
    """The oracle's group minimum against torch's CPU ``amin(dim=1)`` itself (the
    routine quant.py:127 calls), bit for bit including the sign of zero minima,
    on the [ng, G, N] view quant.py:125 reduces: every N from 1 to 70 (tail-only,
    block-only and mixed layouts), single-column weights with G from 32 to 4096
    (torch's contiguous inner reduction) and 4096 x 4100 weights."""
    torch = pytest.importorskip("torch")
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        rng = np.random.default_rng(21 + threads)
        shapes = [(2, G, N) for N in range(1, 71) for G in (2, 8, 32)] + [(32, 128, 4100)]
        shapes += [(64, G, 1) for G in (33, 40, 64, 96, 100, 128, 256, 4096)]
        for ng, G, N in shapes:
            W = _planted_zero_groups(rng, ng, G, N)
            # quant.py:124-127: fp32 copy of the [K, N] weight, reshaped, amin over dim 1
            t = torch.from_numpy(W.reshape(ng * G, N).copy()).reshape(ng, G, N).amin(dim=1)
            o = O._group_min(W)
            mism = np.nonzero(t.numpy().view(np.uint32) != o.view(np.uint32))
            assert mism[0].size == 0, f"ng={ng} G={G} N={N}: first mismatch at {mism[0][0], mism[1][0]}"
    finally:
        torch.set_num_threads(prev)


def test_quant_primitives_match_torch():
    """The oracle's fp32 steps against the torch CPU routines quant.py:129-138
    calls: ``/ 15`` (IEEE division), ``round`` (half to even, -0.0 kept) and
    ``clamp`` (-0.0 kept) -- bit for bit, on random values, halves and zeros."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    x = np.concatenate([
        (rng.standard_normal(200000) * 3).astype(np.float32),
        np.arange(-40, 41, dtype=np.float32) / 2,                       # exact halves
        np.array([0.0, -0.0, -0.4, 0.4, 15.5, -1e-30, 16.0, 14.5], np.float32),
    ])
    t = torch.from_numpy(x)
    div = (t / 15).numpy()
    assert (div.view(np.uint32) == (x / np.float32(15)).view(np.uint32)).all()
    rnd = torch.round(t).numpy()
    assert (rnd.view(np.uint32) == np.rint(x).view(np.uint32)).all()
    r = np.rint(x).astype(np.float32)
    clp = torch.clamp(torch.from_numpy(r), 0, 15).numpy()
    assert (clp.view(np.uint32) == O._clamp_keep_neg_zero(r, 0, 15).view(np.uint32)).all()
    assert np.signbit(O._clamp_keep_neg_zero(np.float32([-0.0]), 0, 15)[0])


@pytest.mark.parametrize("group_size", [64, 128])
@pytest.mark.parametrize("K,N", [(128, 256), (4096, 512)])
def test_quant_shapes_dtypes(K, N, group_size):
    """Reference test_quant.py:58-68."""
    W = np.random.default_rng(0).standard_normal((K, N)).astype(np.float16)
    qw, s, z = O.quantize_weight(W, group_size)
    assert qw.shape == (K // 8, N) and qw.dtype == np.int32
    assert s.shape == (K // group_size, N) and s.dtype == np.float16
    assert z.shape == (K // group_size, N) and z.dtype == np.float16
    assert (z >= 0).all() and (z <= 15).all()
    assert (z == np.round(z.astype(np.float32))).all()


@pytest.mark.parametrize("group_size,expect", [(64, 0.098), (128, 0.109)])
def test_quant_dequant_roundtrip_error(group_size, expect):
    """Reference test_quant.py:71-90: mean relative error < 0.15; the reference's
    docstring reports ~9.8% (G=64) and ~10.9% (G=128) for N(0,1) weights."""
    W = np.random.default_rng(1).standard_normal((4096, 1024)).astype(np.float16)
    qw, s, z = O.quantize_weight(W, group_size)
    dq = O.dequantize_weight(qw, s, z, group_size)
    rel = np.abs(dq.astype(np.float64) - W.astype(np.float64)).mean() / np.abs(W.astype(np.float64)).mean()
    assert rel < 0.15
    assert abs(rel - expect) < 0.006


def test_quant_divisibility_errors():
    """Reference test_quant.py:103-109."""
    with pytest.raises(ValueError):
        O.quantize_weight(np.zeros((100, 16), np.float16), group_size=64)
    with pytest.raises(ValueError):
        O.quantize_weight(np.zeros((96, 16), np.float16), group_size=64)


def test_quantize_non_finite_asserts():
    W = np.zeros((8, 2), np.float16)
    W[3, 1] = np.inf
    with pytest.raises(AssertionError):
        O.quantize_weight(W, 8)


# --------------------------------------------------------------------------- #
# dequantize                                                                   #
# --------------------------------------------------------------------------- #
def test_dequant_equals_numpy_fp16_arithmetic():
    """Brute force over every code, integer zero-point and -0.0, and many fp16
    scales (normal and subnormal): the oracle equals numpy's own fp16
    arithmetic (q.fp16 - z) * s, i.e. RNE_fp16((q-z)*s)."""
    rng = np.random.default_rng(5)
    scales = np.concatenate([
        rng.uniform(1e-4, 0.5, 400).astype(np.float16),
        np.array([6e-8, 1e-6, 3e-5, 6.1e-5, 1.0, 0.0625], dtype=np.float16),
    ])
    zs = np.array(list(range(16)) + [-0.0], dtype=np.float16)
    # K = 16 rows, one group: column c uses (scale, zero) pair c
    pairs = [(s, zv) for s in scales for zv in zs]
    N = len(pairs)
    q = np.tile(np.arange(16, dtype=np.int32)[:, None], (1, N))
    sc = np.array([p[0] for p in pairs], np.float16)[None, :]
    zr = np.array([p[1] for p in pairs], np.float16)[None, :]
    qw = O.pack_int4(q)
    got = O.dequantize_weight(qw, sc, zr, 16)
    ref = (q.astype(np.float16) - zr) * sc           # numpy fp16 arithmetic
    assert ref.dtype == np.float16
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


def test_fp16_subtract_is_one_rounding_for_every_zero():
    """The any-zero kernels compute fp16(q) - z with one hardware RNE subtract.
    For every finite fp16 zero-point and every code, numpy's fp16 subtraction
    (the oracle's arithmetic) equals the exact difference (float64 holds it
    exactly) rounded once to fp16; and the oracle's dequant with such zeros is
    that rounding followed by one rounding of the product (exact in float64:
    11-bit x 11-bit significands)."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    z = bits.view(np.float16)
    z = z[np.isfinite(z)]
    q = np.arange(16, dtype=np.float16)
    got = q[:, None] - z[None, :]
    exact = q.astype(np.float64)[:, None] - z.astype(np.float64)[None, :]
    with np.errstate(over="ignore"):
        once = exact.astype(np.float16)
    assert np.array_equal(got.view(np.uint16), once.view(np.uint16))
    # the oracle's dequant: zeros spread over 16 columns per code row block
    rng = np.random.default_rng(11)
    zs = rng.choice(z, size=4096).astype(np.float16)
    ss = rng.uniform(1e-3, 0.2, size=4096).astype(np.float16)
    qcodes = np.tile(np.arange(16, dtype=np.int32)[:, None], (1, 4096))
    dq = O.dequantize_weight(O.pack_int4(qcodes), ss[None, :], zs[None, :], 16)
    with np.errstate(over="ignore", invalid="ignore"):
        a = (qcodes.astype(np.float64) - zs.astype(np.float64)[None, :]).astype(np.float16)
        ref = (a.astype(np.float64) * ss.astype(np.float64)[None, :]).astype(np.float16)
    assert np.array_equal(dq.view(np.uint16), ref.view(np.uint16))


def test_dequant_constant_group_is_exact():
    """Reference test_quant.py:93-100."""
    W = np.zeros((128, 8), np.float16)
    W[:, 0] = 3.0
    qw, s, z = O.quantize_weight(W, 64)
    assert np.allclose(O.dequantize_weight(qw, s, z, 64).astype(np.float32), W, atol=1e-3)


# --------------------------------------------------------------------------- #
# GEMM oracle                                                                  #
# --------------------------------------------------------------------------- #
@pytest.mark.parametrize("M,K,N,G", [(3, 16, 5, 8), (1, 64, 7, 32), (5, 256, 33, 128)])
def test_reference_gemm_float64_bruteforce(M, K, N, G):
    """Y equals the float64 product of X and the dequantised weight (computed here
    with explicit loops, row-by-column) rounded to fp16, within one fp16 ulp.
    Non-square shapes catch a transposed operand."""
    rng = np.random.default_rng(M * 100 + K + N)
    X = rng.standard_normal((M, K)).astype(np.float16)
    W = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
    qw, s, z = O.quantize_weight(W, G)
    Y = O.reference_w4a16(X, qw, s, z, G)
    assert Y.shape == (M, N) and Y.dtype == np.float16
    q = O.unpack_int4(qw)
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                g = k // G
                wdq = float(np.float16((np.float16(q[k, n]) - z[g, n]) * s[g, n]))
                acc += float(X[m, k]) * wdq
            ref = np.float16(acc)
            assert O.within_tolerance(Y[m, n], ref), (m, n, float(Y[m, n]), float(ref))


def _f64_product(X: np.ndarray, W: np.ndarray) -> np.ndarray:
    """fp16(X @ W) with the sums formed in Python floats (float64), row by
    column, with no BLAS involved."""
    M, K = X.shape
    N = W.shape[1]
    out = np.empty((M, N), np.float16)
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                acc += float(X[m, k]) * float(W[k, n])
            out[m, n] = np.float16(acc)
    return out


@pytest.mark.parametrize("M,K,N,G", [(3, 32, 5, 8), (2, 96, 11, 32), (4, 256, 7, 128)])
def test_dequant_then_matmul_float64_bruteforce(M, K, N, G):
    """reference.py:43-53: fp16 weights materialised, then a matmul with an fp16
    result.  Pinned against float64 brute force over the weight dequantised by
    hand from the unpacked codes (not by the oracle's dequantize_weight), on
    non-square shapes, so a transposed operand or a wrong group index fails."""
    rng = np.random.default_rng(7 * M + K + N)
    X = rng.standard_normal((M, K)).astype(np.float16)
    W = (rng.standard_normal((K, N)) * 0.05).astype(np.float16)
    qw, s, z = O.quantize_weight(W, G)
    Y = O.dequant_then_matmul(X, qw, s, z, G)
    assert Y.shape == (M, N) and Y.dtype == np.float16
    q = O.unpack_int4(qw)
    wdq = np.empty((K, N), np.float16)
    for k in range(K):
        for n in range(N):
            wdq[k, n] = np.float16((np.float16(q[k, n]) - z[k // G, n]) * s[k // G, n])
    exp = _f64_product(X, wdq)
    assert O.within_tolerance(Y, exp).all()
    # the two baselines of reference.py agree with its oracle at fp16 output
    assert O.within_tolerance(Y, O.reference_w4a16(X, qw, s, z, G)).all()
    with pytest.raises(AssertionError):
        O.dequant_then_matmul(X.astype(np.float32), qw, s, z, G)


@pytest.mark.parametrize("M,K,N", [(1, 40, 3), (5, 64, 9), (3, 17, 6)])
def test_fp16_matmul_float64_bruteforce(M, K, N):
    """reference.py:56-67: plain fp16 [M, K] @ [K, N].  Pinned by float64 brute
    force (within one fp16 ulp) and by its preconditions: fp16 operands and a
    matching K (a transposed W of a non-square shape is refused)."""
    rng = np.random.default_rng(M * 31 + K * 7 + N)
    X = rng.standard_normal((M, K)).astype(np.float16)
    W = (rng.standard_normal((K, N)) * 0.1).astype(np.float16)
    Y = O.fp16_matmul(X, W)
    assert Y.shape == (M, N) and Y.dtype == np.float16
    assert O.within_tolerance(Y, _f64_product(X, W)).all()
    with pytest.raises(AssertionError):
        O.fp16_matmul(X, np.ascontiguousarray(W.T))
    with pytest.raises(AssertionError):
        O.fp16_matmul(X.astype(np.float32), W)


def test_fp16_baselines_match_torch_cpu():
    """The third-party boundary: the reference runs both baselines through
    ``torch.matmul`` on fp16 tensors (reference.py:53, :67).  torch's own CPU
    result must lie within one fp16 ulp of the oracle's."""
    import torch

    rng = np.random.default_rng(11)
    M, K, N, G = 6, 512, 40, 64
    X = rng.standard_normal((M, K)).astype(np.float16)
    W = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
    qw, s, z = O.quantize_weight(W, G)
    wdq = O.dequantize_weight(qw, s, z, G)
    t_dq = torch.matmul(torch.from_numpy(X), torch.from_numpy(wdq)).numpy()
    t_fp = torch.matmul(torch.from_numpy(X), torch.from_numpy(W)).numpy()
    assert O.within_tolerance(O.dequant_then_matmul(X, qw, s, z, G), t_dq).all()
    assert O.within_tolerance(O.fp16_matmul(X, W), t_fp).all()


def test_linear_forward_bias_double_rounding():
    """linear.py:90-91: y = fp16(Y) + bias in fp16 (two roundings).  Checked
    against float64 brute force with the two roundings applied explicitly."""
    rng = np.random.default_rng(2)
    M, K, N, G = 4, 64, 9, 32
    x = rng.standard_normal((2, M // 2, K)).astype(np.float16)
    W = (rng.standard_normal((K, N)) * 0.05).astype(np.float16)
    b = (rng.standard_normal(N) * 0.5).astype(np.float16)
    qw, s, z = O.quantize_weight(W, G)
    y = O.linear_forward(x, qw, s, z, b, G)
    assert y.shape == (2, M // 2, N)
    wdq = O.dequantize_weight(qw, s, z, G).astype(np.float64)
    x2 = x.reshape(-1, K).astype(np.float64)
    exp = (np.float16(x2 @ wdq).astype(np.float64) + b.astype(np.float64)).astype(np.float16)
    assert O.within_tolerance(y.reshape(-1, N), exp).all()


def test_tolerance_rule():
    ref = np.array([1.0, 100.0, 0.0, 1e-4], np.float16)
    one_ulp = np.array([1.0009765625, 100.0625, 0.0005, 1e-4 + 6e-8], np.float16)
    assert O.within_tolerance(one_ulp, ref).all()
    bad = np.array([1.01, 100.5, 0.01, 0.01], np.float16)
    assert not O.within_tolerance(bad, ref).any()


# --------------------------------------------------------------------------- #
# golden fixtures                                                              #
# --------------------------------------------------------------------------- #
def test_golden_fixture_vectors():
    """tests/golden/known_answers.json: the spec's and the reference tests' known
    answers, transcribed by tests/golden/make_known_answers.py."""
    with open(os.path.join(GOLDEN, "known_answers.json")) as f:
        cases = json.load(f)
    assert cases
    for c in cases:
        if c["kind"] == "pack":
            q = np.array(c["codes"], dtype=np.int32).reshape(c["K"], c["N"])
            got = _u32(O.pack_int4(q)).reshape(-1).tolist()
            assert got == c["words_u32"], c["name"]
        elif c["kind"] == "quantize":
            W = np.array(c["W"], dtype=np.float16).reshape(c["K"], c["N"])
            qw, s, z = O.quantize_weight(W, c["G"])
            assert O.unpack_int4(qw).reshape(-1).tolist() == c["codes"], c["name"]
            if "zeros_bits" in c:
                assert z.view(np.uint16).reshape(-1).tolist() == c["zeros_bits"], c["name"]
            if "scales_bits" in c:
                assert s.view(np.uint16).reshape(-1).tolist() == c["scales_bits"], c["name"]
        else:
            raise AssertionError(c["kind"])

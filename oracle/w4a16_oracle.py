"""CPU oracle for the W4A16 fused dequant-GEMM path.

TEST INFRASTRUCTURE ONLY.  This module is a numpy restatement of the reference's
pure-PyTorch quantizer and fp32-accumulate oracle.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import
it, and only as the checker (or the timed CPU baseline).  The product package never
imports it and has no CPU fallback.

Reference files followed (paths under the reference checkout
``w4a16-kernel/src/w4a16/``):

* ``pack_int4``          quant.py:45-70
* ``unpack_int4``        quant.py:73-95
* ``quantize_weight``    quant.py:101-144
* ``dequantize_weight``  quant.py:147-178
* ``reference_w4a16``    reference.py:18-40   (the correctness oracle)
* ``dequant_then_matmul`` reference.py:43-53
* ``fp16_matmul``        reference.py:56-67
* ``linear_forward``     linear.py:82-92       (kernel result + bias, fp16 add)

Arithmetic contract (what the reference computes when torch runs it on the CPU):

* quantize math is IEEE fp32: ``(gmax - gmin) / 15`` is a true division (torch's
  CPU ``div`` by a Python scalar divides; it does not multiply by ``1/15``),
  ``round`` is round-half-to-even, ``clamp`` keeps a ``-0.0`` produced by
  ``round`` (so a zero-point can be stored as fp16 ``0x8000``), and ``q`` uses the
  fp32 scale, not the fp16-rounded one.
* group min: when the minimum of a group is a zero and the group holds both
  ``+0.0`` and ``-0.0``, which zero ``amin(dim=1)`` returns depends on the layout
  of torch's CPU reduction.  N >= 2 (strided rows): the columns in whole blocks
  of 32 (``n < 32 * (N // 32)``, the vectorised outer reduction, whose
  ``minimum`` keeps the newer operand on a tie) take the zero that comes LAST in
  k order, the ``N % 32`` tail columns (its scalar loop, which replaces the
  running minimum only on ``<``) the FIRST.  N == 1 (contiguous groups): G < 32
  takes the first zero; G >= 32 follows the vectorised inner reduction (4
  accumulators x 8 lanes over the first ``32 * (G // 32)`` values, then the
  scalar tail; ``_inner_zero_min``).  torch does not document any of this; the
  tests pin it against ``torch.amin`` itself on the CPU (every N up to 70, N = 1
  for G up to 4096, 4096 x 4100 weights, 1 and 8 threads; identical under its
  DEFAULT, AVX2 and AVX512 code paths).  Only the sign bit of that group's
  zero-point depends on it (scale, codes and the dequantised weights do not).
  **Parity unpinned**: a single group of a single column (``N == 1`` and
  ``G == K``) with ``K > 32768``, where torch splits the one reduction across its
  threads and the answer depends on the thread count; the oracle gives the
  single-thread answer.
* non-finite weights make the reference's ``pack_int4`` range assertion fire
  (NaN codes cast to int32 fall outside [0, 15]); the oracle raises
  ``AssertionError`` up front for any non-finite weight.
* dequant is fp16 arithmetic ``(q - z) * s``.  ``q - z`` is exact for integer
  zero-points, so the result is ``RNE_fp16((q - z) * s)``; the float32 product of
  an integer in [-15, 15] and an fp16 scale is exact, so computing it in float32
  and rounding once to fp16 gives the same bits (pinned by brute force in the
  tests against numpy's own fp16 arithmetic).
* ``reference_w4a16`` is ``fp16(fp32(X) @ fp32(W_dq))``.  The fp32 summation order
  of a BLAS sgemm is unspecified, so GEMM results are compared with a tolerance.

Parity pins (each checked by a test under ``tests/``): the spec's packing word
``0xC2714F08`` and quantisation example, the reference tests' nibble-position and
extreme-value cases, hand-derived tie / ``-0.0`` / fp32-scale cases, the fp32
primitives and the group minimum against torch's own CPU routines (``/ 15``,
``round``, ``clamp``, ``amin``), closed forms for dequant, and float64 brute
force for the GEMM on small shapes.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "pack_int4",
    "unpack_int4",
    "quantize_weight",
    "dequantize_weight",
    "reference_w4a16",
    "dequant_then_matmul",
    "fp16_matmul",
    "linear_forward",
    "fp16_ulp",
    "within_tolerance",
]

_NIBBLES = 8
_QMAX = 15


# --------------------------------------------------------------------------- #
# packing (quant.py:45-95)                                                     #
# --------------------------------------------------------------------------- #
def pack_int4(q: np.ndarray) -> np.ndarray:
    """[K, N] integer codes in [0, 15] -> int32 [K//8, N]; row 8i+j -> nibble j.

    Follows quant.py:45-70 (asserts 2-D, K % 8 == 0, range [0, 15]).
    """
    q = np.asarray(q)
    assert q.ndim == 2, f"pack_int4 expects 2D [K, N], got {q.shape}"
    K, N = q.shape
    assert K % _NIBBLES == 0, f"K={K} must be divisible by 8 to pack int4"
    qi = q.astype(np.int64)
    if qi.size:
        lo, hi = int(qi.min()), int(qi.max())
        assert 0 <= lo and hi <= _QMAX, f"uint4 values must be in [0,15], got [{lo},{hi}]"
    qi = qi.reshape(K // _NIBBLES, _NIBBLES, N).astype(np.uint32)
    packed = np.zeros((K // _NIBBLES, N), dtype=np.uint32)
    for j in range(_NIBBLES):
        packed |= (qi[:, j, :] & np.uint32(0xF)) << np.uint32(4 * j)
    return packed.view(np.int32)


def unpack_int4(qweight: np.ndarray, K: int | None = None) -> np.ndarray:
    """int32 [K//8, N] -> int32 [K, N] codes in [0, 15] (quant.py:73-95)."""
    qweight = np.asarray(qweight)
    assert qweight.ndim == 2, f"unpack_int4 expects 2D [K//8, N], got {qweight.shape}"
    assert qweight.dtype == np.int32, f"qweight must be int32, got {qweight.dtype}"
    Kp, N = qweight.shape
    if K is None:
        K = Kp * _NIBBLES
    assert K == Kp * _NIBBLES, f"K={K} incompatible with qweight rows {Kp}"
    u = qweight.view(np.uint32)
    out = np.empty((Kp, _NIBBLES, N), dtype=np.int32)
    for j in range(_NIBBLES):
        out[:, j, :] = ((u >> np.uint32(4 * j)) & np.uint32(0xF)).astype(np.int32)
    return out.reshape(K, N)


# --------------------------------------------------------------------------- #
# quantize / dequantize (quant.py:101-178)                                     #
# --------------------------------------------------------------------------- #
def _clamp_keep_neg_zero(x: np.ndarray, lo: float, hi: float) -> np.ndarray:
    """torch.clamp semantics on finite input: compare-select, -0.0 survives."""
    x = np.where(x < np.float32(lo), np.float32(lo), x)
    return np.where(x > np.float32(hi), np.float32(hi), x).astype(np.float32)


def _inner_zero_min(col: np.ndarray) -> np.float32:
    """N == 1, G >= 32: the zero torch's vectorised inner reduction returns for a
    contiguous group whose minimum is a zero.  Positions p < 32 * (G // 32) sit in
    lane p % 8 of accumulator (p // 8) % 4 (a tie keeps the later value); the
    accumulators fold 0..3 in turn (a tie keeps the later one) and the lanes
    toward lane 0 (a tie keeps the lower lane); the G % 32 tail is then scanned
    (a tie keeps the running minimum).  So: lowest lane, then highest
    accumulator, then latest position; a tail zero only without a zero before
    the tail, and then the first."""
    G = col.size
    zs = np.nonzero(col == 0)[0]
    head = zs[zs < 32 * (G // 32)]
    if head.size == 0:
        return col[zs[0]]
    slot = head % 32
    best = min(zip((slot % 8).tolist(), (-(slot // 8)).tolist(), (-head).tolist(), head.tolist()))
    return col[best[3]]


def _group_min(Wg: np.ndarray) -> np.ndarray:
    """torch's CPU ``amin(dim=1)`` of [ng, G, N] float32 (quant.py:127), including
    which zero a group holding both zero signs returns (see module docstring)."""
    gmin = Wg.min(axis=1)
    G, N = Wg.shape[1], Wg.shape[2]
    n_block = 32 * (N // 32)
    zg, zn = np.nonzero(gmin == 0)
    for g, n in zip(zg.tolist(), zn.tolist()):
        col = Wg[g, :, n]
        if N == 1 and G >= 32:
            gmin[g, n] = _inner_zero_min(col)
            continue
        zeros_at = np.nonzero(col == 0)[0]
        gmin[g, n] = col[zeros_at[-1] if n < n_block else zeros_at[0]]
    return gmin


def quantize_weight(W: np.ndarray, group_size: int = 128):
    """Group-wise asymmetric uint4 quantisation along K (quant.py:101-144).

    Args:
        W: [K, N] float16 or float32.
    Returns:
        (qweight int32 [K//8, N], scales float16 [K//G, N], zeros float16 [K//G, N])
    """
    W = np.asarray(W)
    assert W.ndim == 2, f"quantize_weight expects 2D [K, N], got {W.shape}"
    K, N = W.shape
    if K % _NIBBLES != 0:
        raise ValueError(f"K={K} must be divisible by 8 (got remainder {K % 8})")
    if K % group_size != 0:
        raise ValueError(f"K={K} must be divisible by group_size={group_size}")
    G = group_size
    ng = K // G
    Wf = W.astype(np.float32)
    assert np.isfinite(Wf).all(), "uint4 values must be in [0,15] (non-finite weight)"
    Wg = Wf.reshape(ng, G, N)
    gmax = Wg.max(axis=1)                                               # :126
    gmin = _group_min(Wg)                                               # :127
    scale = ((gmax - gmin) / np.float32(_QMAX)).astype(np.float32)      # :129
    scale = np.where(scale > 0, scale, np.float32(1.0)).astype(np.float32)  # :132
    zero = _clamp_keep_neg_zero(np.rint(-gmin / scale), 0, _QMAX)           # :134
    q = _clamp_keep_neg_zero(np.rint(Wg / scale[:, None, :]) + zero[:, None, :], 0, _QMAX)
    q = q.reshape(K, N).astype(np.int32)                                    # :139
    qweight = pack_int4(q)
    return qweight, scale.astype(np.float16), zero.astype(np.float16)


def dequantize_weight(qweight, scales, zeros, group_size: int) -> np.ndarray:
    """W_dq = (q - z) * s in fp16 -> float16 [K, N] (quant.py:147-178)."""
    qweight = np.asarray(qweight)
    assert qweight.dtype == np.int32, f"qweight must be int32, got {qweight.dtype}"
    Kp, N = qweight.shape
    K = Kp * _NIBBLES
    G = group_size
    assert K % G == 0, f"K={K} must be divisible by group_size={G}"
    ng = K // G
    scales = np.asarray(scales)
    zeros = np.asarray(zeros)
    assert scales.shape == (ng, N), f"scales shape {scales.shape} != {(ng, N)}"
    assert zeros.shape == (ng, N), f"zeros shape {zeros.shape} != {(ng, N)}"
    q = unpack_int4(qweight, K).astype(np.float32).reshape(ng, G, N)
    s = scales.astype(np.float16).astype(np.float32)[:, None, :]
    z = zeros.astype(np.float16).astype(np.float32)[:, None, :]
    # (q - z): fp16-exact for integer zero-points; round it to fp16 anyway so a
    # non-integer zero-point follows fp16 subtraction like the reference.
    d = (q - z).astype(np.float16).astype(np.float32)
    w = (d * s).astype(np.float16)   # float32 product is exact; one RNE to fp16
    return np.ascontiguousarray(w.reshape(K, N))


# --------------------------------------------------------------------------- #
# GEMM oracle and baselines (reference.py:18-67, linear.py:82-92)              #
# --------------------------------------------------------------------------- #
def reference_w4a16(X, qweight, scales, zeros, group_size: int) -> np.ndarray:
    """Y = fp16(fp32(X) @ fp32(dequant(W)))  (reference.py:18-40)."""
    X = np.asarray(X)
    assert X.dtype == np.float16, f"X must be fp16, got {X.dtype}"
    assert X.ndim == 2, f"X must be 2D [M, K], got {X.shape}"
    M, K = X.shape
    W_dq = dequantize_weight(qweight, scales, zeros, group_size)
    assert W_dq.shape[0] == K, f"K mismatch: X K={K} vs weight K={W_dq.shape[0]}"
    Y = X.astype(np.float32) @ W_dq.astype(np.float32)
    return Y.astype(np.float16)


def dequant_then_matmul(X, qweight, scales, zeros, group_size: int) -> np.ndarray:
    """Baseline (reference.py:43-53): fp16 weights then an fp16-output matmul.

    numpy has no fp16 GEMM with an fp32 accumulator, so the product is formed in
    fp32 and rounded once, which is what an fp32-accumulating fp16 GEMM returns.
    """
    X = np.asarray(X)
    assert X.dtype == np.float16
    W_dq = dequantize_weight(qweight, scales, zeros, group_size)
    return (X.astype(np.float32) @ W_dq.astype(np.float32)).astype(np.float16)


def fp16_matmul(X, W) -> np.ndarray:
    """Baseline (reference.py:56-67): unquantised fp16 [M,K] @ [K,N]."""
    X = np.asarray(X)
    W = np.asarray(W)
    assert X.dtype == np.float16 and W.dtype == np.float16
    assert X.shape[1] == W.shape[0], f"K mismatch: X {X.shape} vs W {W.shape}"
    return (X.astype(np.float32) @ W.astype(np.float32)).astype(np.float16)


def linear_forward(x, qweight, scales, zeros, bias, group_size: int) -> np.ndarray:
    """W4A16Linear.forward (linear.py:82-92): flatten, GEMM, fp16 ``+ bias``."""
    x = np.asarray(x)
    K = qweight.shape[0] * _NIBBLES
    assert x.dtype == np.float16 and x.shape[-1] == K
    y = reference_w4a16(x.reshape(-1, K), qweight, scales, zeros, group_size)
    if bias is not None:
        b = np.asarray(bias).astype(np.float16)
        y = (y.astype(np.float32) + b.astype(np.float32)).astype(np.float16)
    return y.reshape(*x.shape[:-1], y.shape[-1])


# --------------------------------------------------------------------------- #
# tolerance                                                                    #
# --------------------------------------------------------------------------- #
def fp16_ulp(y: np.ndarray) -> np.ndarray:
    """Spacing of fp16 at |y| (float64), i.e. one unit in the last place."""
    a = np.abs(np.asarray(y, dtype=np.float16))
    nxt = np.nextafter(a, np.float16(np.inf), dtype=np.float16)
    return (nxt.astype(np.float64) - a.astype(np.float64))


def within_tolerance(out, ref, ulps: float = 1.0, rtol: float = 1e-3, atol: float = 1e-3):
    """Elementwise: |out-ref| <= ulps*ulp(ref) or |out-ref| <= atol + rtol*|ref|.

    This is the acceptance rule for fp16 GEMM output: one fp16 ulp of the oracle,
    or rtol = atol = 1e-3 where split-K reorders the fp32 sums.  Returns a bool
    array; non-finite values must match exactly.
    """
    o = np.asarray(out).astype(np.float64)
    r = np.asarray(ref).astype(np.float64)
    d = np.abs(o - r)
    ok = (d <= ulps * fp16_ulp(ref)) | (d <= atol + rtol * np.abs(r))
    same_nonfinite = (~np.isfinite(o)) & (~np.isfinite(r)) & ((o == r) | (np.isnan(o) & np.isnan(r)))
    return np.where(np.isfinite(o) & np.isfinite(r), ok, same_nonfinite)

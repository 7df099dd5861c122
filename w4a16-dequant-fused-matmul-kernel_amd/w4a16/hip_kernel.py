"""Fused W4A16 GEMM entry point on MI355X: ``Y = X @ dequant(qweight)``.

Drop-in for the reference's primary backend ``w4a16_matmul``
(w4a16-kernel/src/w4a16/triton_kernel.py:131-200): same signature, same
preconditions raised as ``AssertionError`` (:153-187), optional ``out``.  The
kernel is chosen inside ``libw4a16.so`` by shape:

* M <= 2 (M <= 4 on weights wider than 16384 columns): decode GEMV -- VALU
  v_dot2_f32_f16, no MFMA, column blocks wide enough to give every CU a
  workgroup, split-K only when N is too narrow;
* other M <= 64 on small weights: skinny GEMM on v_mfma_f32_16x16x32_f16, 16
  columns per workgroup over the whole of K;
* 4 <= M <= 64 on larger weights, and M > 64: the streamed prefill GEMM on
  MFMA (32-, 64- or 128-row tiles, split along K where the tiles are few);
* shapes the vector kernels do not take (N % 4 != 0 beyond the skinny range,
  G % 32 != 0, misaligned views, operands >= 2 GiB): the sequential-k SIMT
  kernel.

Row-strided views (inner stride 1, row stride >= the row length) are accepted
for ``x`` and ``out``: the reference's kernel takes strides (:71-75) though its
wrapper asserts contiguity (:170-173); any other layout raises the same
``AssertionError`` as the reference.

Group size: the reference's Triton path needs every autotune BLOCK_K to divide
G (:177-182), i.e. G % 64 == 0.  These kernels need G % 32 == 0, so G = 32 works
here as well; G = 8 still raises AssertionError like the reference.

Zero-points: the reference dequantises ``(q - z) * s`` in fp16 for any fp16
zero (:117-119).  The fused kernels have two forms: one for integer zeros
with |z| <= 1024 (what quantize_weight makes, 0..15) and one for any zero (one
more fp16 subtract per pair of weights).  Each zeros tensor is checked once on
the GPU (``w4a16_zeros_check_f16``); the result is kept on the tensor with
its version counter, so an in-place change is checked again.
"""
from __future__ import annotations

import ctypes
import warnings

import torch
from torch import Tensor

from . import _lib
from . import _runtime as rt
from . import autotune

__all__ = ["w4a16_matmul", "w4a16_linear", "plan_for", "GROUP_MULTIPLE", "zeros_need_any_form"]

GROUP_MULTIPLE = 32


def _check_operands(x: Tensor, qweight: Tensor, scales: Tensor, zeros: Tensor, group_size: int):
    assert x.is_cuda, "x must be on a HIP device"
    assert qweight.is_cuda and scales.is_cuda and zeros.is_cuda, "all inputs must be on a HIP device"
    assert x.dtype == torch.float16, f"x must be fp16, got {x.dtype}"
    assert qweight.dtype == torch.int32, f"qweight must be int32, got {qweight.dtype}"
    assert scales.dtype == torch.float16, f"scales must be fp16, got {scales.dtype}"
    assert zeros.dtype == torch.float16, f"zeros must be fp16, got {zeros.dtype}"
    assert x.dim() == 2 and qweight.dim() == 2, "x and qweight must be 2D"
    M, K = x.shape
    Kp, N = qweight.shape
    assert Kp * 8 == K, f"qweight rows (K//8)={Kp} incompatible with x K={K}"
    assert K % 8 == 0, f"K={K} must be divisible by 8"
    assert group_size > 0 and K % group_size == 0, (
        f"K={K} must be divisible by group_size={group_size}")
    num_groups = K // group_size
    assert scales.shape == (num_groups, N), f"scales shape {tuple(scales.shape)} != {(num_groups, N)}"
    assert zeros.shape == (num_groups, N), f"zeros shape {tuple(zeros.shape)} != {(num_groups, N)}"
    assert _rows_ok(x), "x must be contiguous"
    assert qweight.is_contiguous(), "qweight must be contiguous"
    assert scales.is_contiguous(), "scales must be contiguous"
    assert zeros.is_contiguous(), "zeros must be contiguous"
    assert group_size % GROUP_MULTIPLE == 0, (
        f"group_size={group_size} must be a multiple of {GROUP_MULTIPLE} for the fused kernels")
    dev = x.device
    assert qweight.device == dev and scales.device == dev and zeros.device == dev, (
        "all inputs must be on the same device")
    return M, K, N


def _rows_ok(t: Tensor) -> bool:
    """Contiguous, or row-major with unit inner stride and rows >= a row apart."""
    return t.is_contiguous() or (t.dim() == 2 and t.stride(1) == 1
                                 and t.stride(0) >= t.shape[1])


def _row_stride(t: Tensor) -> int:
    # a single row's stride is arbitrary (torch calls such a view contiguous)
    return t.stride(0) if t.shape[0] > 1 else t.shape[1]


_ZKEY = "_w4a16_zeros_checked"


def zeros_need_any_form(zeros: Tensor) -> bool:
    """Whether `zeros` holds a value the integer-zero kernels cannot take (not an
    integer in [-1024, 1024]).  Checked on the GPU once per tensor version and
    kept on the tensor; under HIP-graph capture, where the answer cannot be read
    back, an unchecked tensor is taken to need the any-zero form (exact for
    every zero)."""
    key = (zeros._version, zeros.data_ptr(), zeros.numel(), zeros.device)
    hit = getattr(zeros, _ZKEY, None)
    if hit is not None and hit[0] == key:
        return hit[1]
    if zeros.numel() == 0:
        return False
    if torch.cuda.is_current_stream_capturing():
        return True
    with rt.on_device(zeros.device):
        flag = torch.zeros(1, dtype=torch.int32, device=zeros.device)
        _lib.check(rt.lib().w4a16_zeros_check_f16(zeros.data_ptr(), zeros.numel(),
                                                   flag.data_ptr(), rt.stream_ptr(zeros.device)),
                   "w4a16 zeros check")
        need = bool(flag.item())
    setattr(zeros, _ZKEY, (key, need))
    return need


def mark_integer_zeros(zeros: Tensor) -> None:
    """Record that `zeros` (as it is now) holds integers in [0, 15], as made by
    quantize_weight, so its first GEMM needs no check."""
    setattr(zeros, _ZKEY, ((zeros._version, zeros.data_ptr(), zeros.numel(), zeros.device),
                           False))


_FAR_SZ_WARNED = False


def _warn_far_scales_zeros(scales: Tensor, zeros: Tensor, M: int) -> None:
    """Warn once per process when scales and zeros lie 2 GiB or more apart:
    the streamed MFMA kernels (prefill, and small batches on large weights)
    reach both through one buffer resource, so such calls run the
    register-tiled kernel instead -- same results, slower."""
    global _FAR_SZ_WARNED
    if _FAR_SZ_WARNED or M < 4:
        return
    if abs(scales.data_ptr() - zeros.data_ptr()) + scales.numel() * 2 >= (1 << 31):
        _FAR_SZ_WARNED = True
        warnings.warn(
            "w4a16: scales and zeros lie 2 GiB or more apart in device memory; the streamed "
            "MFMA kernels read both through one buffer resource, so GEMMs with M >= 4 on "
            "their plans run the register-tiled kernel instead (same results, slower: "
            "measured +19-28 % at M = 16-32 on a Llama-70B gate+up layer). Allocate them "
            "together, e.g. as the two halves of one [2, K // G, N] fp16 tensor.",
            RuntimeWarning, stacklevel=4)


def _launch(x, qweight, scales, zeros, bias, y, M, N, K, G, plan: "_lib.Plan | None"):
    dev = x.device
    _warn_far_scales_zeros(scales, zeros, M)
    with rt.on_device(dev):
        any_zeros = zeros_need_any_form(zeros)
        if plan is None and autotune.enabled():
            plan = autotune.plan_for_call(x, qweight, scales, zeros, G, M, N, K, _row_stride(x),
                                          _row_stride(y), any_zeros)
        if any_zeros:
            # the any-zero kernels, through a plan carrying the flag
            if plan is None:
                plan = _lib.plan(M, N, K, G)
            else:
                plan = _lib.Plan.from_buffer_copy(plan)
            plan.flags |= _lib.PLAN_ANY_ZEROS
        if plan is None:
            ws_bytes = rt.lib().w4a16_gemm_workspace_bytes(M, N, K, G)
        else:
            ws_bytes = int(plan.workspace_bytes)
        ws = rt.workspace(dev, ws_bytes)
        stream = rt.stream_ptr(dev)
        ldx, ldy = _row_stride(x), _row_stride(y)
        if ldx != K or ldy != N:
            code = rt.lib().w4a16_gemm_f16_strided(
                None if plan is None else ctypes.byref(plan), x.data_ptr(), ldx,
                qweight.data_ptr(), scales.data_ptr(), zeros.data_ptr(), rt.ptr(bias),
                y.data_ptr(), ldy, M, N, K, G, rt.ptr(ws), 0 if ws is None else ws.numel(),
                stream)
        elif plan is None:
            code = rt.lib().w4a16_linear_f16(
                x.data_ptr(), qweight.data_ptr(), scales.data_ptr(), zeros.data_ptr(),
                rt.ptr(bias), y.data_ptr(), M, N, K, G, rt.ptr(ws),
                0 if ws is None else ws.numel(), stream)
        else:
            code = rt.lib().w4a16_gemm_f16_planned(
                ctypes.byref(plan), x.data_ptr(), qweight.data_ptr(), scales.data_ptr(),
                zeros.data_ptr(), rt.ptr(bias), y.data_ptr(), M, N, K, G, rt.ptr(ws),
                0 if ws is None else ws.numel(), stream)
    _lib.check(code, "w4a16 GEMM")
    return y


def _output(x: Tensor, M: int, N: int, out: Tensor | None) -> Tensor:
    if out is None:
        return torch.empty((M, N), device=x.device, dtype=torch.float16)
    assert out.shape == (M, N) and out.dtype == torch.float16 and _rows_ok(out)
    assert out.device == x.device, "out must be on the same device as x"
    return out


def w4a16_matmul(
    x: Tensor,
    qweight: Tensor,
    scales: Tensor,
    zeros: Tensor,
    group_size: int,
    out: Tensor | None = None,
) -> Tensor:
    """Fused W4A16 GEMM: ``Y = X @ dequant(qweight)`` (triton_kernel.py:131-200).

    Args:
        x: activations [M, K] fp16, contiguous or row-strided, on a HIP device.
        qweight: int32 [K//8, N], contiguous.
        scales, zeros: fp16 [K//G, N], contiguous.
        group_size: G, with G | K, 8 | K and G % 32 == 0.
        out: optional preallocated fp16 [M, N] output (contiguous or row-strided).
    Returns:
        fp16 [M, N], fp32-accumulated.
    """
    M, K, N = _check_operands(x, qweight, scales, zeros, group_size)
    y = _output(x, M, N, out)
    return _launch(x, qweight, scales, zeros, None, y, M, N, K, group_size, None)


def w4a16_linear(x: Tensor, qweight: Tensor, scales: Tensor, zeros: Tensor,
                 bias: Tensor | None, group_size: int, out: Tensor | None = None) -> Tensor:
    """``fp16(X @ dequant(W)) + bias`` with the bias add fused into the epilogue.

    Same arithmetic as W4A16Linear's kernel call followed by ``y + bias``
    (linear.py:89-91): the GEMM result is rounded to fp16, then the fp16 bias is
    added with one more fp16 rounding.
    """
    M, K, N = _check_operands(x, qweight, scales, zeros, group_size)
    if bias is not None:
        assert bias.shape == (N,) and bias.dtype == torch.float16 and bias.is_contiguous()
        assert bias.device == x.device
    y = _output(x, M, N, out)
    return _launch(x, qweight, scales, zeros, bias, y, M, N, K, group_size, None)


def plan_for(M: int, N: int, K: int, group_size: int, kernel: str | int = 0,
             split_k: int = 0) -> "_lib.Plan":
    """The launch plan for a shape; `kernel` may force "gemv", "mfma", "simt" or
    "skinny" (the plan's ``tile_cfg`` then selects the MFMA tile configuration
    or the GEMV wave count)."""
    if isinstance(kernel, str):
        kernel = {"auto": 0, "gemv": 1, "mfma": 2, "simt": 3, "skinny": 4}[kernel]
    return _lib.plan(M, N, K, group_size, kernel, split_k)


def w4a16_matmul_planned(x: Tensor, qweight: Tensor, scales: Tensor, zeros: Tensor,
                         group_size: int, plan: "_lib.Plan", bias: Tensor | None = None,
                         out: Tensor | None = None) -> Tensor:
    """Run the fused GEMM with an explicit plan (tests and benchmarks)."""
    M, K, N = _check_operands(x, qweight, scales, zeros, group_size)
    y = _output(x, M, N, out)
    return _launch(x, qweight, scales, zeros, bias, y, M, N, K, group_size, plan)

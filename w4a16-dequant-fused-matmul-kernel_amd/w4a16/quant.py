"""Group-wise asymmetric 4-bit weight quantisation + int4 packing on the GPU.

Same API, layout and results as the reference's ``w4a16/quant.py``
(w4a16-kernel/src/w4a16/quant.py:36-178); every function runs a HIP kernel from
``libw4a16.so``:

* ``quantize_weight(W, group_size=128) -> (qweight, scales, zeros)``  quant.py:101-144
* ``dequantize_weight(qweight, scales, zeros, group_size) -> W_dq``    quant.py:147-178
* ``pack_int4(q) -> qweight``                                          quant.py:45-70
* ``unpack_int4(qweight, K=None) -> q``                                quant.py:73-95

Layout: ``qweight`` int32 [K//8, N], row 8i+j in bits [4j, 4j+4) of word (i, n),
unsigned codes; ``scales``/``zeros`` fp16 [K//G, N].

Results are bit-exact with the reference evaluated by torch on the CPU (IEEE fp32
division for the scale, round-half-even, ``-0.0`` zero-points kept).  Inputs on
the CPU are computed on the current HIP device and the results are returned on
the input's device; without a HIP device these functions raise RuntimeError.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _lib
from . import _runtime as rt
from .hip_kernel import mark_integer_zeros

__all__ = ["quantize_weight", "dequantize_weight", "pack_int4", "unpack_int4"]

_NIBBLES_PER_INT32 = 8
_MAX_UINT4 = 15


def _flag(device: torch.device) -> Tensor:
    return torch.zeros(1, dtype=torch.int32, device=device)


def pack_int4(q: Tensor) -> Tensor:
    """Pack ``[K, N]`` uint4 codes (0..15) into int32 ``[K//8, N]`` (quant.py:45-70).

    Raises AssertionError for a non-2-D input, K % 8 != 0, or codes outside
    [0, 15], like the reference.
    """
    assert q.dim() == 2, f"pack_int4 expects 2D [K, N], got {tuple(q.shape)}"
    K, N = q.shape
    assert K % _NIBBLES_PER_INT32 == 0, f"K={K} must be divisible by 8 to pack int4"
    home, dev, (qd,) = rt.stage_to_device(q)
    with rt.on_device(dev):
        qi = qd.to(torch.int32).contiguous()
        out = torch.empty((K // _NIBBLES_PER_INT32, N), dtype=torch.int32, device=dev)
        if qi.numel() == 0:
            return out.to(home)
        flag = _flag(dev)
        _lib.check(rt.lib().w4a16_pack_int4(qi.data_ptr(), out.data_ptr(), K, N,
                                             flag.data_ptr(), rt.stream_ptr(dev)),
                   "w4a16_pack_int4")
        if int(flag.item()) != 0:      # host sync, as the reference's range check
            lo, hi = int(qi.min()), int(qi.max())
            raise AssertionError(f"uint4 values must be in [0,15], got [{lo},{hi}]")
    return out.to(home)


def unpack_int4(qweight: Tensor, K: int | None = None) -> Tensor:
    """Inverse of :func:`pack_int4`: int32 [K//8, N] -> int32 [K, N] (quant.py:73-95)."""
    assert qweight.dim() == 2, f"unpack_int4 expects 2D [K//8, N], got {tuple(qweight.shape)}"
    assert qweight.dtype == torch.int32, f"qweight must be int32, got {qweight.dtype}"
    Kp, N = qweight.shape
    if K is None:
        K = Kp * _NIBBLES_PER_INT32
    assert K == Kp * _NIBBLES_PER_INT32, f"K={K} incompatible with qweight rows {Kp}"
    home, dev, (qw,) = rt.stage_to_device(qweight)
    with rt.on_device(dev):
        qw = qw.contiguous()
        out = torch.empty((K, N), dtype=torch.int32, device=dev)
        if out.numel():
            _lib.check(rt.lib().w4a16_unpack_int4(qw.data_ptr(), out.data_ptr(), K, N,
                                                   rt.stream_ptr(dev)), "w4a16_unpack_int4")
    return out.to(home)


def quantize_weight(W: Tensor, group_size: int = 128) -> tuple[Tensor, Tensor, Tensor]:
    """Group-wise asymmetric 4-bit quantisation of ``W`` [K, N] along K (quant.py:101-144).

    Args:
        W: weight [K, N], fp16 or fp32 (quantised in fp32 either way; fp32
           weights are not rounded to fp16 first, as in the reference).
        group_size: G; requires G | K and 8 | K (ValueError otherwise).
    Returns:
        (qweight int32 [K//8, N], scales fp16 [K//G, N], zeros fp16 [K//G, N])
    """
    assert W.dim() == 2, f"quantize_weight expects 2D [K, N], got {tuple(W.shape)}"
    K, N = W.shape
    if K % _NIBBLES_PER_INT32 != 0:
        raise ValueError(f"K={K} must be divisible by 8 (got remainder {K % 8})")
    if K % group_size != 0:
        raise ValueError(f"K={K} must be divisible by group_size={group_size}")
    G = group_size
    home, dev, (Wd,) = rt.stage_to_device(W.detach())
    with rt.on_device(dev):
        if Wd.dtype not in (torch.float16, torch.float32):
            Wd = Wd.to(torch.float32)
        Wd = Wd.contiguous()
        fn = (rt.lib().w4a16_quantize_pack_f32 if Wd.dtype == torch.float32
              else rt.lib().w4a16_quantize_pack_f16)
        qweight = torch.empty((K // _NIBBLES_PER_INT32, N), dtype=torch.int32, device=dev)
        scales = torch.empty((K // G, N), dtype=torch.float16, device=dev)
        zeros = torch.empty((K // G, N), dtype=torch.float16, device=dev)
        if Wd.numel():
            flag = _flag(dev)
            _lib.check(fn(Wd.data_ptr(), qweight.data_ptr(), scales.data_ptr(), zeros.data_ptr(),
                          K, N, G, flag.data_ptr(), rt.stream_ptr(dev)), "w4a16_quantize_pack")
            if int(flag.item()) != 0:
                raise AssertionError(
                    "uint4 values must be in [0,15]: W holds a non-finite value")
    zeros = zeros.to(home)
    mark_integer_zeros(zeros)   # zero-points 0..15: the integer-zero kernels take them
    return qweight.to(home), scales.to(home), zeros


def dequantize_weight(qweight: Tensor, scales: Tensor, zeros: Tensor, group_size: int) -> Tensor:
    """W_dq = (q - zero) * scale in fp16 -> fp16 [K, N] (quant.py:147-178)."""
    assert qweight.dtype == torch.int32, f"qweight must be int32, got {qweight.dtype}"
    Kp, N = qweight.shape
    K = Kp * _NIBBLES_PER_INT32
    G = group_size
    assert K % G == 0, f"K={K} must be divisible by group_size={G}"
    num_groups = K // G
    assert scales.shape == (num_groups, N), f"scales shape {tuple(scales.shape)} != {(num_groups, N)}"
    assert zeros.shape == (num_groups, N), f"zeros shape {tuple(zeros.shape)} != {(num_groups, N)}"
    home, dev, (qw, s, z) = rt.stage_to_device(qweight, scales, zeros)
    with rt.on_device(dev):
        qw = qw.contiguous()
        s = s.to(torch.float16).contiguous()
        z = z.to(torch.float16).contiguous()
        out = torch.empty((K, N), dtype=torch.float16, device=dev)
        if out.numel():
            _lib.check(rt.lib().w4a16_dequantize_f16(qw.data_ptr(), s.data_ptr(), z.data_ptr(),
                                                      out.data_ptr(), K, N, G,
                                                      rt.stream_ptr(dev)), "w4a16_dequantize_f16")
    return out.to(home)

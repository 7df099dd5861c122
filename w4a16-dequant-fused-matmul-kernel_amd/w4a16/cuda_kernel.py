"""Native sequential-k SIMT backend (API of the reference's ``w4a16.cuda_kernel``).

The reference JIT-builds a CUDA SIMT kernel with ``torch.utils.cpp_extension``
(w4a16-kernel/src/w4a16/cuda_kernel.py:22-87, cuda/w4a16_gemm.cu:20-115).  Here
the same role -- a plain, any-group-size kernel with per-element fp16 dequant and
sequential fp32 accumulation over k -- is the SIMT kernel inside the prebuilt
``libw4a16.so``; nothing is compiled at run time.

* ``is_available()``      -> bool (a HIP device is visible and the library loads)
* ``load_cuda_module()``  -> the loaded library handle (memoised), or raises
* ``w4a16_matmul_cuda(x, qweight, scales, zeros, group_size) -> Tensor``
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _lib
from . import _runtime as rt

__all__ = ["w4a16_matmul_cuda", "load_cuda_module", "is_available"]


def is_available() -> bool:
    if not torch.cuda.is_available():
        return False
    try:
        _lib.load()
    except ImportError:
        return False
    return True


def load_cuda_module(verbose: bool = True):
    """Return the loaded native library (cuda_kernel.py:35-62 builds; this loads)."""
    if not torch.cuda.is_available():
        raise RuntimeError("a HIP GPU is required for the W4A16 native kernels")
    lib = _lib.load()
    if verbose:
        print(f"w4a16: loaded {_lib.LIB_PATH}")
    return lib


def w4a16_matmul_cuda(x: Tensor, qweight: Tensor, scales: Tensor, zeros: Tensor,
                      group_size: int) -> Tensor:
    """SIMT W4A16 GEMM; same contract as the fused entry point (cuda_kernel.py:65-87).

    Like the reference's native launcher it makes its inputs contiguous instead of
    asserting, and accepts any group size that divides K.
    """
    assert x.is_cuda, "x must be on a HIP device"
    assert x.dtype == torch.float16, f"x must be fp16, got {x.dtype}"
    assert qweight.dtype == torch.int32, f"qweight must be int32, got {qweight.dtype}"
    assert scales.dtype == torch.float16 and zeros.dtype == torch.float16
    assert x.dim() == 2 and qweight.dim() == 2
    M, K = x.shape
    Kp, N = qweight.shape
    assert Kp * 8 == K, f"qweight rows (K//8)={Kp} incompatible with x K={K}"
    assert group_size > 0 and K % group_size == 0, (
        f"K={K} not divisible by group_size={group_size}")
    ng = K // group_size
    assert scales.shape == (ng, N) and zeros.shape == (ng, N)
    dev = x.device
    x, qweight, scales, zeros = (t.contiguous() for t in (x, qweight, scales, zeros))
    y = torch.empty((M, N), device=dev, dtype=torch.float16)
    p = _lib.plan(M, N, K, group_size, _lib.KERNEL_SIMT, 0)
    import ctypes

    with rt.on_device(dev):
        code = rt.lib().w4a16_gemm_f16_planned(
            ctypes.byref(p), x.data_ptr(), qweight.data_ptr(), scales.data_ptr(),
            zeros.data_ptr(), None, y.data_ptr(), M, N, K, group_size, None, 0,
            rt.stream_ptr(dev))
    _lib.check(code, "w4a16 SIMT GEMM")
    return y

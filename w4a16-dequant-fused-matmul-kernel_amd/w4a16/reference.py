"""GPU baselines with the reference's ``w4a16/reference.py`` API.

The reference's module is its PyTorch oracle and its benchmark baselines
(w4a16-kernel/src/w4a16/reference.py:18-67).  Here the same three functions run
on the HIP device: the dequantisation is this package's HIP kernel, the matmul is
PyTorch-ROCm's BLAS (hipBLASLt / rocBLAS).  They are what the fused kernel is
compared against in benchmarks ("vs fp16", "vs dequant+matmul").  The
correctness oracle of the test-suite is the CPU restatement under ``oracle/``,
not this module.

CPU inputs are staged to the current HIP device and results returned on the
input's device.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _runtime as rt
from .quant import dequantize_weight

__all__ = ["reference_w4a16", "dequant_then_matmul", "fp16_matmul"]


def reference_w4a16(X: Tensor, qweight: Tensor, scales: Tensor, zeros: Tensor,
                    group_size: int) -> Tensor:
    """dequant -> fp32-accumulated matmul -> fp16 (reference.py:18-40)."""
    assert X.dtype == torch.float16, f"X must be fp16, got {X.dtype}"
    assert X.dim() == 2, f"X must be 2D [M, K], got {tuple(X.shape)}"
    M, K = X.shape
    home, dev, (Xd, qw, s, z) = rt.stage_to_device(X, qweight, scales, zeros)
    W_dq = dequantize_weight(qw, s, z, group_size)
    assert W_dq.shape[0] == K, f"K mismatch: X K={K} vs weight K={W_dq.shape[0]}"
    Y = torch.matmul(Xd.to(torch.float32), W_dq.to(torch.float32))
    return Y.to(torch.float16).to(home)


def dequant_then_matmul(X: Tensor, qweight: Tensor, scales: Tensor, zeros: Tensor,
                        group_size: int) -> Tensor:
    """Materialise fp16 weights, then an fp16 BLAS matmul (reference.py:43-53)."""
    assert X.dtype == torch.float16
    home, dev, (Xd, qw, s, z) = rt.stage_to_device(X, qweight, scales, zeros)
    W_dq = dequantize_weight(qw, s, z, group_size)
    return torch.matmul(Xd, W_dq).to(home)


def fp16_matmul(X: Tensor, W: Tensor) -> Tensor:
    """Unquantised fp16 matmul, W in logical [K, N] layout (reference.py:56-67)."""
    assert X.dtype == torch.float16 and W.dtype == torch.float16
    assert X.shape[1] == W.shape[0], f"K mismatch: X {tuple(X.shape)} vs W {tuple(W.shape)}"
    home, dev, (Xd, Wd) = rt.stage_to_device(X, W)
    return torch.matmul(Xd, Wd).to(home)

"""W4A16 dequant-fused matmul for AMD Instinct MI355X (gfx950).

Drop-in for the reference package ``w4a16`` (w4a16-kernel/src/w4a16/__init__.py:18-39):
the same public names, tensor formats and results, computed by hand-written HIP
kernels in ``libw4a16.so`` (decode GEMV, MFMA prefill GEMM, SIMT GEMM,
quantise/pack/unpack/dequantise) reached through a C ABI.

Public API:
    quantize_weight / dequantize_weight / pack_int4 / unpack_int4   (quant.py)
    reference_w4a16 / dequant_then_matmul / fp16_matmul             (reference.py, GPU baselines)
    w4a16_matmul                                                    (hip_kernel.py; alias triton_kernel.py)
    W4A16Linear                                                     (linear.py)

``HAS_TRITON`` is kept for import compatibility and is always False: no Triton is
used.  ``HAS_HIP`` tells whether the native library loaded.
"""
from __future__ import annotations

from .quant import quantize_weight, dequantize_weight, pack_int4, unpack_int4
from .reference import reference_w4a16, dequant_then_matmul, fp16_matmul
from .hip_kernel import w4a16_matmul
from .linear import W4A16Linear

__all__ = [
    "quantize_weight",
    "dequantize_weight",
    "pack_int4",
    "unpack_int4",
    "reference_w4a16",
    "dequant_then_matmul",
    "fp16_matmul",
    "w4a16_matmul",
    "W4A16Linear",
]

HAS_TRITON = False

try:
    from . import _lib as _l

    _l.load()
    HAS_HIP = True
except ImportError:  # the library is not built; every kernel call raises
    HAS_HIP = False

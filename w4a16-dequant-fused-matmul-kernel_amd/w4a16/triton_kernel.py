"""Import-path alias: ``from w4a16.triton_kernel import w4a16_matmul`` keeps working.

The reference's primary backend lives in ``w4a16/triton_kernel.py``
(w4a16-kernel/src/w4a16/triton_kernel.py:131).  This build has no Triton; the
name resolves to the HIP entry point in :mod:`w4a16.hip_kernel`.
"""
from __future__ import annotations

from .hip_kernel import w4a16_matmul

__all__ = ["w4a16_matmul"]

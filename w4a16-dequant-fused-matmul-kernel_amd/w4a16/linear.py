"""``W4A16Linear``: an ``nn.Linear`` stand-in whose weight lives as packed uint4.

Interface of the reference module (w4a16-kernel/src/w4a16/linear.py:19-98):
the constructor's arguments, the four buffers (names, dtypes and shapes, so a
``state_dict`` saved by either loads into the other), ``from_linear``,
``quantize_from_dense``, ``forward`` and the exception types
(``ValueError`` for sizes the packing cannot hold, ``AssertionError`` for bad
inputs).

Layout: ``nn.Linear.weight`` is [out_features, in_features] = [N, K]; this
module's logical weight is [K, N] (``y = x @ W``), so ``from_linear``
quantises the transpose.  ``forward`` keeps the reference's arithmetic -- the
GEMM result rounded to fp16, then an fp16 ``+ bias`` -- with the bias add done
in the GEMM kernel's epilogue rather than by a second kernel.
"""
from __future__ import annotations

import torch
from torch import Tensor, nn

from .hip_kernel import mark_integer_zeros, w4a16_linear
from .quant import quantize_weight

__all__ = ["W4A16Linear"]


def _check_sizes(in_features: int, group_size: int) -> None:
    # eight 4-bit codes per int32 word along K, whole quantisation groups
    if in_features % 8:
        raise ValueError(f"W4A16Linear: in_features ({in_features}) is not a multiple of 8, "
                         "the codes packed per int32 word")
    if in_features % group_size:
        raise ValueError(f"W4A16Linear: in_features ({in_features}) is not a whole number of "
                         f"groups of {group_size}")


class W4A16Linear(nn.Module):
    """Inference linear layer: fp16 activations, weight as packed uint4 codes.

    With K = ``in_features``, N = ``out_features`` and G = ``group_size`` the
    module holds buffers only (no parameters):

    * ``qweight`` int32 [K/8, N]: word (i, n) packs the codes of rows 8i..8i+7
      of column n, row 8i + j in bits [4j, 4j + 4);
    * ``scales``, ``zeros`` fp16 [K/G, N]: one scale and zero-point per group
      of G rows and column;
    * ``bias`` fp16 [N], or ``None`` for ``bias=False``.

    All start zeroed; ``from_linear`` or ``quantize_from_dense`` fills them.
    """

    def __init__(
        self,
        in_features: int,
        out_features: int,
        group_size: int = 128,
        bias: bool = True,
        device: torch.device | str | None = None,
    ) -> None:
        super().__init__()
        _check_sizes(in_features, group_size)
        self.in_features = in_features
        self.out_features = out_features
        self.group_size = group_size

        def blank(rows: int, dtype: torch.dtype) -> Tensor:
            return torch.zeros((rows, out_features), dtype=dtype, device=device)

        n_groups = in_features // group_size
        self.register_buffer("qweight", blank(in_features // 8, torch.int32))
        self.register_buffer("scales", blank(n_groups, torch.float16))
        self.register_buffer("zeros", blank(n_groups, torch.float16))
        if bias:
            self.register_buffer("bias", torch.zeros(out_features, dtype=torch.float16,
                                                     device=device))
        else:
            self.bias = None

    @classmethod
    def from_linear(cls, linear: nn.Linear, group_size: int = 128) -> "W4A16Linear":
        """A quantised copy of ``linear`` (reference linear.py:55-70), on the
        same device; its bias, if any, converted to fp16."""
        out_features, in_features = linear.weight.shape
        has_bias = linear.bias is not None
        layer = cls(in_features, out_features, group_size=group_size, bias=has_bias,
                    device=linear.weight.device)
        # [out, in] -> the [K, N] layout quantize_weight expects
        layer.quantize_from_dense(linear.weight.detach().t().contiguous())
        if has_bias:
            layer.bias.copy_(linear.bias.detach().to(torch.float16))
        return layer

    def quantize_from_dense(self, W: Tensor) -> None:
        """Fill the buffers from a dense [K, N] weight (reference linear.py:72-80),
        with ``quantize_weight``'s group-wise uint4 quantisation."""
        want = (self.in_features, self.out_features)
        if tuple(W.shape) != want:
            raise AssertionError(f"quantize_from_dense: W must be [in_features, out_features] = "
                                 f"{list(want)}, got {list(W.shape)}")
        packed = quantize_weight(W, self.group_size)
        for buf, val in zip((self.qweight, self.scales, self.zeros), packed):
            buf.copy_(val.to(buf.device))
        # codes from quantize_weight have integer zero-points: no zeros check
        mark_integer_zeros(self.zeros)

    def forward(self, x: Tensor) -> Tensor:
        """``fp16(x @ dequant(W)) + bias`` over the last dimension of ``x``
        (reference linear.py:82-92); leading dimensions are kept."""
        if x.dtype != torch.float16:
            raise AssertionError(f"W4A16Linear expects fp16 activations, got {x.dtype}")
        if x.shape[-1] != self.in_features:
            raise AssertionError(f"W4A16Linear: last dimension of x is {x.shape[-1]}, "
                                 f"in_features is {self.in_features}")
        lead = x.shape[:-1]
        rows = x.reshape(-1, self.in_features)
        # the kernels take rows at any stride >= K with unit inner stride
        if rows.stride(-1) != 1 or rows.stride(0) < self.in_features:
            rows = rows.contiguous()
        y = w4a16_linear(rows, self.qweight, self.scales, self.zeros, self.bias, self.group_size)
        return y.view(*lead, self.out_features)

    def extra_repr(self) -> str:
        bias = self.bias is not None
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"group_size={self.group_size}, bias={bias}")

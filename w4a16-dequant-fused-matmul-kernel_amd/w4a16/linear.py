"""``W4A16Linear`` -- drop-in ``nn.Linear`` replacement on the MI355X kernels.

Same constructor, buffers (names, dtypes, shapes -- so ``state_dict`` files
interchange with the reference's), ``from_linear``, ``quantize_from_dense`` and
``forward`` as the reference (w4a16-kernel/src/w4a16/linear.py:19-98).

``nn.Linear`` stores weight as [out, in] = [N, K]; the logical weight here is
[K, N], so ``from_linear`` transposes before quantising (linear.py:66).
``forward`` flattens leading dims, runs the fused GEMM and adds the bias with the
reference's arithmetic (fp16 GEMM result, then an fp16 ``+ bias``), the add fused
into the kernel epilogue instead of a second kernel.
"""
from __future__ import annotations

import torch
from torch import Tensor, nn

from .hip_kernel import mark_integer_zeros, w4a16_linear
from .quant import quantize_weight

__all__ = ["W4A16Linear"]


class W4A16Linear(nn.Module):
    """Linear layer holding its weight as packed uint4 codes, computing in fp16.

    K = ``in_features``, N = ``out_features``, G = ``group_size``.  The module
    owns four buffers and no parameters (it is for inference): the packed codes
    ``qweight`` (int32, K/8 rows of N words, eight 4-bit codes per word along
    K), the per-group ``scales`` and ``zeros`` (fp16, K/G rows of N), and an
    fp16 ``bias`` of N entries, or ``None`` when built with ``bias=False``.
    Buffers start zeroed; ``from_linear`` or ``quantize_from_dense`` fills them.
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
        if in_features % 8 != 0:
            raise ValueError(f"in_features={in_features} must be divisible by 8")
        if in_features % group_size != 0:
            raise ValueError(f"in_features={in_features} must be divisible by group_size={group_size}")
        self.in_features = in_features
        self.out_features = out_features
        self.group_size = group_size

        K, N = in_features, out_features
        self.register_buffer("qweight", torch.zeros((K // 8, N), dtype=torch.int32, device=device))
        self.register_buffer("scales", torch.zeros((K // group_size, N), dtype=torch.float16, device=device))
        self.register_buffer("zeros", torch.zeros((K // group_size, N), dtype=torch.float16, device=device))
        if bias:
            self.register_buffer("bias", torch.zeros(N, dtype=torch.float16, device=device))
        else:
            self.bias = None

    @classmethod
    def from_linear(cls, linear: nn.Linear, group_size: int = 128) -> "W4A16Linear":
        """Quantise an existing ``nn.Linear`` (linear.py:55-70)."""
        N, K = linear.weight.shape
        mod = cls(
            in_features=K,
            out_features=N,
            group_size=group_size,
            bias=linear.bias is not None,
            device=linear.weight.device,
        )
        W = linear.weight.detach().t().contiguous()  # [N, K] -> [K, N]
        mod.quantize_from_dense(W)
        if linear.bias is not None:
            mod.bias.copy_(linear.bias.detach().to(torch.float16))
        return mod

    def quantize_from_dense(self, W: Tensor) -> None:
        """Quantise a dense ``W`` of shape [K, N] into the buffers (linear.py:72-80)."""
        assert W.shape == (self.in_features, self.out_features), (
            f"expected weight [K,N]={(self.in_features, self.out_features)}, got {tuple(W.shape)}"
        )
        qweight, scales, zeros = quantize_weight(W, self.group_size)
        self.qweight.copy_(qweight.to(self.qweight.device))
        self.scales.copy_(scales.to(self.scales.device))
        self.zeros.copy_(zeros.to(self.zeros.device))
        mark_integer_zeros(self.zeros)

    def forward(self, x: Tensor) -> Tensor:
        """y = (x @ dequant(W)) + bias over the last dim (linear.py:82-92)."""
        assert x.dtype == torch.float16, f"x must be fp16, got {x.dtype}"
        assert x.shape[-1] == self.in_features, (
            f"x last dim {x.shape[-1]} != in_features {self.in_features}"
        )
        orig_shape = x.shape
        x2d = x.reshape(-1, self.in_features).contiguous()
        y = w4a16_linear(x2d, self.qweight, self.scales, self.zeros, self.bias, self.group_size)
        return y.reshape(*orig_shape[:-1], self.out_features)

    def extra_repr(self) -> str:
        return (
            f"in_features={self.in_features}, out_features={self.out_features}, "
            f"group_size={self.group_size}, bias={self.bias is not None}"
        )

"""The five benchmark/parity configurations and their seeded synthetic inputs.

Configurations (one weight layer each; X ~ N(0, 1) fp16):

  C1  CPU plumbing      M=16, K=N=1024, G=128; W ~ N(0, 0.02)                 seed 0
  C2  decode GEMV       M=1, K=N=4096, G=128; W ~ N(0, 0.02)                  seed 1
  C3  decode sweep      M in {1,4,8,16,32} x (K,N) in {(4096,6144),(4096,4096),
                        (4096,28672),(14336,4096)}, G=128; W ~ N(0, 0.02)     seed 2
  C4  prefill           M in {512,2048,4096}, K=4096, N=14336, G=128;
                        W ~ N(0, 0.02), then in every group a seeded 1% of the
                        columns scaled x8 ("outlier columns")                  seed 3
  C5  large layer       (K,N) in {(8192,28672),(28672,8192)}, M in {1,16,256},
                        G in {32,64,128}; W ~ N(0, 0.015) with a seeded 1% of
                        entries redrawn from N(0, 0.2)                        seed 4

Inputs are drawn on the CPU from ``torch.Generator`` in fp32, then cast to fp16,
so every process on the same image draws the same bits.  W has its own generator
seeded from (config seed, K, N, G) -- one weight layer serves every M -- and X
has one seeded from (config seed, M, K).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

__all__ = ["Case", "CONFIGS", "cases", "make_x", "make_w", "make_inputs"]


@dataclass(frozen=True)
class Case:
    config: str
    M: int
    K: int
    N: int
    G: int
    seed: int
    weight_kind: str = "normal"   # "normal" | "outlier_cols" | "heavy_tail"
    w_std: float = 0.02

    @property
    def name(self) -> str:
        return f"{self.config}_M{self.M}_K{self.K}_N{self.N}_G{self.G}"

    def bytes(self) -> int:
        """Algorithmic bytes: X + packed W + scales + zeros + Y (bench_gemm.py:61-67)."""
        ng = self.K // self.G
        return 2 * self.M * self.K + 4 * (self.K // 8) * self.N + 2 * 2 * ng * self.N + 2 * self.M * self.N

    def flops(self) -> int:
        """2*M*N*K (bench_gemm.py:86)."""
        return 2 * self.M * self.N * self.K


def _c3():
    out = []
    for (K, N) in [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)]:
        for M in (1, 4, 8, 16, 32):
            out.append(Case("C3", M, K, N, 128, 2))
    return out


def _c5():
    out = []
    for (K, N) in [(8192, 28672), (28672, 8192)]:
        for G in (32, 64, 128):
            for M in (1, 16, 256):
                out.append(Case("C5", M, K, N, G, 4, "heavy_tail", 0.015))
    return out


CONFIGS: dict[str, list[Case]] = {
    "C1": [Case("C1", 16, 1024, 1024, 128, 0)],
    "C2": [Case("C2", 1, 4096, 4096, 128, 1)],
    "C3": _c3(),
    "C4": [Case("C4", M, 4096, 14336, 128, 3, "outlier_cols") for M in (512, 2048, 4096)],
    "C5": _c5(),
}


def cases(*names: str) -> list[Case]:
    names = names or tuple(CONFIGS)
    return [c for n in names for c in CONFIGS[n]]


def _mix(*vals: int) -> int:
    h = 0x3243F6A8
    for v in vals:
        h = (h * 1_000_003 + int(v) + 0x9E3779B9) % (2**61 - 1)
    return h % (2**31 - 1)


def make_x(c: Case, m_rows: int | None = None) -> torch.Tensor:
    """Activations X fp16 [M, K] (CPU) for case `c`; `m_rows` overrides M."""
    M = c.M if m_rows is None else m_rows
    g = torch.Generator().manual_seed(_mix(c.seed, 1, M, c.K))
    return torch.randn(M, c.K, generator=g, dtype=torch.float32).to(torch.float16)


def make_w(c: Case) -> torch.Tensor:
    """Weight W fp16 [K, N] (CPU) for case `c`; independent of M."""
    g = torch.Generator().manual_seed(_mix(c.seed, 2, c.K, c.N, c.G))
    W = torch.randn(c.K, c.N, generator=g, dtype=torch.float32) * c.w_std
    if c.weight_kind == "outlier_cols":
        ng = c.K // c.G
        pick = torch.rand(ng, c.N, generator=g) < 0.01
        mult = torch.where(pick, torch.tensor(8.0), torch.tensor(1.0))
        W = (W.view(ng, c.G, c.N) * mult[:, None, :]).view(c.K, c.N)
    elif c.weight_kind == "heavy_tail":
        tail = torch.rand(c.K, c.N, generator=g) < 0.01
        W = torch.where(tail, torch.randn(c.K, c.N, generator=g) * 0.2, W)
    return W.to(torch.float16)


def make_inputs(c: Case):
    """(X fp16 [M, K], W fp16 [K, N]) on the CPU for case `c`."""
    return make_x(c), make_w(c)

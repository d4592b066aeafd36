"""SwiGLU shared expert: ``w2(silu(w1 x) * w3 x)``
(torchtitan/models/common/feed_forward.py:34-54)."""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .configurable import Module
from .linear import Linear

__all__ = ["FeedForward", "compute_ffn_hidden_dim"]


def compute_ffn_hidden_dim(dim: int, *, multiple_of: int = 1, ffn_dim_multiplier: float | None = None) -> int:
    """Llama-style SwiGLU width: 2/3 of 4*dim, optional multiplier, rounded up to multiple_of."""
    hidden = int(2 * 4 * dim / 3)
    if ffn_dim_multiplier is not None:
        hidden = int(ffn_dim_multiplier * hidden)
    return multiple_of * ((hidden + multiple_of - 1) // multiple_of)


class FeedForward(Module):
    @dataclass(kw_only=True, slots=True)
    class Config(Module.Config):
        w1: Linear.Config
        w2: Linear.Config
        w3: Linear.Config

    def __init__(self, config: Config):
        super().__init__()
        self.w1 = config.w1.build()
        self.w2 = config.w2.build()
        self.w3 = config.w3.build()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # Three dense GEMMs: plain library GEMMs (hipBLASLt through torch), with the
        # reference's bf16 roundings of w1 x, w3 x, silu, the product and w2.
        return self.w2(F.silu(self.w1(x)) * self.w3(x))

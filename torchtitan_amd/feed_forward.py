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
        if _use_grouped_kernel(self, x):
            # One expert holding every token: the same bf16 roundings as the three
            # Linear calls (outputs of w1, w3, silu, the product and w2).
            from . import ops

            lead = x.shape[:-1]
            x2 = x.reshape(-1, x.shape[-1])
            counts = torch.full((1,), x2.shape[0], dtype=torch.int64, device=x.device)
            y, _, _, _ = ops.grouped_swiglu(
                x2, self.w1.weight.unsqueeze(0), self.w2.weight.unsqueeze(0),
                self.w3.weight.unsqueeze(0), counts,
            )
            return y.reshape(*lead, y.shape[-1])
        return self.w2(F.silu(self.w1(x)) * self.w3(x))


def _use_grouped_kernel(ff: FeedForward, x: torch.Tensor) -> bool:
    """The MI355X grouped kernel serves the bias-free bf16 case on the GPU."""
    w1, w2, w3 = ff.w1.weight, ff.w2.weight, ff.w3.weight
    return (
        x.is_cuda
        and x.dtype == torch.bfloat16
        and all(w.dtype == torch.bfloat16 for w in (w1, w2, w3))
        and ff.w1.bias is None and ff.w2.bias is None and ff.w3.bias is None
        and x.shape[-1] % 256 == 0
        and w1.shape[0] % 256 == 0
        and not torch.is_autocast_enabled("cuda")
    )

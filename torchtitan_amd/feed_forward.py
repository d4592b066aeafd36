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


class _SwiGLUFFN(torch.autograd.Function):
    """w2(silu(w1 x) * w3 x) for bias-free projections, with one GEMM for the
    weight gradients of w1 and w3.

    Forward: the same F.linear, silu and mul calls as the three nn.Linear
    modules (feed_forward.py:53-54), so the output is theirs bit for bit.
    Backward: dh = dy w2, dW2 = dy^T h, dx = (dg w1) + (du w3) and the SwiGLU
    derivative (dg = silu_backward(dh * u, g), du = dh * silu(g)) are autograd's
    own calls and roundings. dg and du are written side by side into one
    [tokens, 2 Hs] buffer, so dW1 and dW3 come out of a single dgu^T x GEMM
    (fp32 accumulation, one rounding per element, as each of autograd's two):
    a 2 Hs-row output fills the chip where two Hs-row outputs leave most
    compute units idle (1024 x 2304 is 144 library tiles on 256 CUs)."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor) -> torch.Tensor:
        a1 = F.linear(x, w1)
        a3 = F.linear(x, w3)
        s = F.silu(a1)
        h = s * a3
        ctx.save_for_backward(x, w1, w2, w3, a1, a3, s, h)
        return F.linear(h, w2)

    @staticmethod
    def backward(ctx, dy: torch.Tensor):
        x, w1, w2, w3, a1, a3, s, h = ctx.saved_tensors
        d, hs = x.shape[-1], w1.shape[0]
        x2, dy2 = x.reshape(-1, d), dy.reshape(-1, d)
        dh = dy2.mm(w2)
        dw2 = dy2.t().mm(h.reshape(-1, hs)) if ctx.needs_input_grad[2] else None
        dgu = torch.empty(x2.shape[0], 2 * hs, dtype=dh.dtype, device=dh.device)
        dg, du = dgu[:, :hs], dgu[:, hs:]
        torch.mul(dh, s.reshape(-1, hs), out=du)
        dsilu = dh * a3.reshape(-1, hs)
        if dg.device.type == "cpu":
            # the CPU's vectorised kernel (contiguous output) and its strided one
            # evaluate exp differently; the GPU's elementwise kernels do not
            dg.copy_(torch.ops.aten.silu_backward(dsilu, a1.reshape(-1, hs)))
        else:
            torch.ops.aten.silu_backward.grad_input(dsilu, a1.reshape(-1, hs), grad_input=dg)
        dx = (dg.mm(w1) + du.mm(w3)).view(x.shape) if ctx.needs_input_grad[0] else None
        dw1 = dw3 = None
        if ctx.needs_input_grad[1] or ctx.needs_input_grad[3]:
            dw13 = dgu.t().mm(x2)
            dw1, dw3 = dw13[:hs], dw13[hs:]
        return dx, dw1, dw2, dw3


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

    def _fused_backward_applies(self, x: torch.Tensor) -> bool:
        lins = (self.w1, self.w2, self.w3)
        if any(lin.bias is not None for lin in lins) or torch.is_autocast_enabled():
            return False
        if not torch.is_grad_enabled() or not (x.requires_grad or any(lin.weight.requires_grad for lin in lins)):
            return False
        ws = [lin.weight for lin in lins]
        return all(type(w) is torch.nn.Parameter and w.dtype == x.dtype and w.device == x.device for w in ws)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # Three dense GEMMs: plain library GEMMs (hipBLASLt through torch), with the
        # reference's bf16 roundings of w1 x, w3 x, silu, the product and w2.
        if self._fused_backward_applies(x):
            return _SwiGLUFFN.apply(x, self.w1.weight, self.w2.weight, self.w3.weight)
        return self.w2(F.silu(self.w1(x)) * self.w3(x))

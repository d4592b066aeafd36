"""SwiGLU shared expert: ``w2(silu(w1 x) * w3 x)``
(torchtitan/models/common/feed_forward.py:34-54)."""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import ops
from .configurable import Module, called_plainly
from .linear import Linear

__all__ = ["FeedForward", "compute_ffn_hidden_dim"]


def compute_ffn_hidden_dim(dim: int, *, multiple_of: int = 1, ffn_dim_multiplier: float | None = None) -> int:
    """Llama-style SwiGLU width: 2/3 of 4*dim, optional multiplier, rounded up to multiple_of."""
    hidden = int(2 * 4 * dim / 3)
    if ffn_dim_multiplier is not None:
        hidden = int(ffn_dim_multiplier * hidden)
    return multiple_of * ((hidden + multiple_of - 1) // multiple_of)


@torch.library.custom_op("moe_mi355x::swiglu_ffn_backward", mutates_args=())
def swiglu_ffn_backward(
    dy: torch.Tensor, x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor,
    a1: torch.Tensor, a3: torch.Tensor, h: torch.Tensor,
    need_dx: bool, need_dw13: bool, need_dw2: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dx, [dW1; dW3], dW2) of w2(silu(w1 x) * w3 x) from the forward's a1 = w1 x,
    a3 = w3 x and h = silu(a1) * a3; unrequested results are empty.

    dh = dy w2, dW2 = dy^T h, du = dh * silu(a1) and dg = silu_backward(dh * a3, a1)
    are autograd's own calls and roundings, dx = (dg w1) + (du w3) its sum. dg and du
    are written side by side into one [tokens, 2 Hs] buffer (on the GPU by one
    launch, ops.swiglu_backward, which recomputes silu(a1) instead of reading it),
    so [dW1; dW3] is a single dgu^T x GEMM (fp32 accumulation, one rounding per
    element). A custom op, so that a compiled graph calls it whole: the CPU path's
    side-by-side writes are out= views that graph capture does not trace."""
    d, hs = x.shape[-1], w1.shape[0]
    x2, dy2 = x.reshape(-1, d), dy.reshape(-1, d)
    empty = x.new_empty(0)
    dh = dy2.mm(w2)
    dw2 = dy2.t().mm(h.reshape(-1, hs)) if need_dw2 else empty
    a1_2, a3_2 = a1.reshape(-1, hs), a3.reshape(-1, hs)
    if dh.device.type == "cpu":
        dgu = torch.empty(x2.shape[0], 2 * hs, dtype=dh.dtype, device=dh.device)
        torch.mul(dh, F.silu(a1_2), out=dgu[:, hs:])
        # the CPU's vectorised kernel (contiguous output) and its strided one
        # evaluate exp differently
        dgu[:, :hs].copy_(torch.ops.aten.silu_backward(dh * a3_2, a1_2))
    else:
        dgu = ops.swiglu_backward(dh, a1_2, a3_2)
    dg, du = dgu[:, :hs], dgu[:, hs:]
    dx = (dg.mm(w1) + du.mm(w3)).view(x.shape) if need_dx else empty.clone()
    dw13 = dgu.t().mm(x2) if need_dw13 else empty.clone()
    return dx, dw13, dw2


@swiglu_ffn_backward.register_fake
def _(dy, x, w1, w2, w3, a1, a3, h, need_dx, need_dw13, need_dw2):
    hs, d = w1.shape
    return (x.new_empty(x.shape if need_dx else (0,)), x.new_empty((2 * hs, d) if need_dw13 else (0,)),
            x.new_empty((d, hs) if need_dw2 else (0,)))


class _SwiGLUFFN(torch.autograd.Function):
    """w2(silu(w1 x) * w3 x) for bias-free projections, with one GEMM for the
    weight gradients of w1 and w3.

    Forward: the same F.linear calls as the three nn.Linear modules
    (feed_forward.py:53-54), and silu(a1) * a3 with torch's two roundings (on the
    GPU one launch, ops.swiglu_forward), so the output is theirs bit for bit.
    Backward: dh = dy w2, dW2 = dy^T h, dx = (dg w1) + (du w3) and the SwiGLU
    derivative (dg = silu_backward(dh * u, g), du = dh * silu(g)) are autograd's
    own calls and roundings (swiglu_ffn_backward). dg and du are written side by
    side into one [tokens, 2 Hs] buffer, so dW1 and dW3 come out of a single
    dgu^T x GEMM (fp32 accumulation, one rounding per element, as each of
    autograd's two): a 2 Hs-row output fills the chip where two Hs-row outputs
    leave most compute units idle (1024 x 2304 is 144 library tiles on 256 CUs)."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor) -> torch.Tensor:
        a1 = F.linear(x, w1)
        a3 = F.linear(x, w3)
        h = F.silu(a1) * a3 if a1.device.type == "cpu" else ops.swiglu_forward(a1, a3)
        ctx.save_for_backward(x, w1, w2, w3, a1, a3, h)
        return F.linear(h, w2)

    @staticmethod
    def backward(ctx, dy: torch.Tensor):
        x, w1, w2, w3, a1, a3, h = ctx.saved_tensors
        need = ctx.needs_input_grad
        dx, dw13, dw2 = swiglu_ffn_backward(dy, x, w1, w2, w3, a1, a3, h, need[0], need[1] or need[3], need[2])
        hs = w1.shape[0]
        return (dx if need[0] else None, dw13[:hs] if need[1] else None, dw2 if need[2] else None,
                dw13[hs:] if need[3] else None)


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
        # the fused function reads the three weights instead of calling the Linear
        # modules: only for plain Linear modules without hooks, outside autocast of
        # x's device type (where F.linear would return another dtype than the weights')
        lins = (self.w1, self.w2, self.w3)
        if any(type(lin) is not Linear or lin.bias is not None for lin in lins):
            return False
        if torch.is_autocast_enabled(x.device.type) or not called_plainly(*lins):
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

"""gpt-oss experts on the MI355X grouped GEMMs.

Same classes, Config fields, parameter names and shapes as
torchtitan/models/gpt_oss/moe.py: ``GptOssGroupedExperts`` holds
``mlp1_weight [E, 2H, D]`` (glu row 2j, linear row 2j + 1), ``mlp1_bias
[E, 2H]``, ``mlp2_weight [E, D, H]``, ``mlp2_bias [E, D]``; ``GptOssMoE`` is the
MoE layer with those experts. Both expert paths (grouped-mm and for-loop,
moe.py:55-122) run ``ops.grouped_swiglu_oss``: bf16 GEMMs with fp32
accumulation, the biases added in bf16, and the clamped SwiGLU

    swiglu(h1) = clamp(g, max=L) * sigmoid(1.702 clamp(g, max=L)) * (clamp(u, -L, L) + 1)

(moe.py:43-52) with g = h1[:, 0::2], u = h1[:, 1::2].
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import nn

from . import ops
from .configurable import Module
from .moe import MoE, GroupedExperts, _local

__all__ = ["GptOssGroupedExperts", "GptOssMoE", "swiglu"]


def swiglu(x: torch.Tensor, alpha: float = 1.702, limit: float = 7.0) -> torch.Tensor:
    """The reference's activation on an interleaved [.., 2H] tensor in torch ops
    (moe.py:43-52); the layer itself runs it inside the gate_up kernel."""
    x_glu, x_linear = x[..., ::2], x[..., 1::2]
    x_glu = x_glu.clamp(min=None, max=limit)
    x_linear = x_linear.clamp(min=-limit, max=limit)
    return x_glu * torch.sigmoid(alpha * x_glu) * (x_linear + 1)


def _check_tp(tp_degree: int) -> None:
    if tp_degree != 1:
        raise NotImplementedError("tensor-parallel expert biases (tp_degree > 1) need a device mesh; "
                                  "this layer runs on one GPU")


def _run_experts_grouped_mm(
    mlp1_weight: torch.Tensor, mlp1_bias: torch.Tensor, mlp2_weight: torch.Tensor, mlp2_bias: torch.Tensor,
    swiglu_limit: float, x: torch.Tensor, num_tokens_per_expert: torch.Tensor, tp_degree: int = 1,
) -> torch.Tensor:
    """moe.py:92-122: routed rows past sum(counts) get no expert (their output
    rows are zero, as the reference's zero bias row leaves them)."""
    _check_tp(tp_degree)
    y, _, _, _ = ops.grouped_swiglu_oss(
        x.bfloat16(), mlp1_weight.bfloat16(), mlp1_bias, mlp2_weight.bfloat16(), mlp2_bias,
        num_tokens_per_expert, float(swiglu_limit),
    )
    return y


def _run_experts_for_loop(
    mlp1_weight: torch.Tensor, mlp1_bias: torch.Tensor, mlp2_weight: torch.Tensor, mlp2_bias: torch.Tensor,
    swiglu_limit: float, x: torch.Tensor, num_tokens_per_expert: torch.Tensor, tp_degree: int = 1,
) -> torch.Tensor:
    """moe.py:55-89: per-expert matmuls on rows [0, sum(counts)) in x's dtype,
    returning those rows. bf16 runs the bf16 grouped kernels, whose rounding
    points are those of the reference's bf16 matmuls and bias adds. The gpt-oss
    epilogues have no fp32 kernels, so other dtypes raise instead of running in
    a narrower one."""
    _check_tp(tp_degree)
    if x.dtype != torch.bfloat16 or mlp1_weight.dtype != torch.bfloat16 or mlp2_weight.dtype != torch.bfloat16:
        raise TypeError("the gpt-oss expert for-loop path runs in bfloat16 on MI355X; got "
                        f"x {x.dtype}, mlp1_weight {mlp1_weight.dtype}, mlp2_weight {mlp2_weight.dtype}")
    total = int(num_tokens_per_expert.sum().item())
    return _run_experts_grouped_mm(mlp1_weight, mlp1_bias, mlp2_weight, mlp2_bias, swiglu_limit,
                                   x[:total], num_tokens_per_expert)


class GptOssGroupedExperts(Module):
    @dataclass(kw_only=True, slots=True)
    class Config(GroupedExperts.Config):
        swiglu_limit: float = 7.0

    def __init__(self, config: Config):
        super().__init__()
        dim, hidden_dim, num_experts = config.dim, config.hidden_dim, config.num_experts
        self.num_experts = num_experts
        self.use_grouped_mm = config.use_grouped_mm
        self.swiglu_limit = config.swiglu_limit
        self.mlp1_weight = nn.Parameter(torch.empty((num_experts, hidden_dim * 2, dim)))
        self.mlp1_bias = nn.Parameter(torch.empty((num_experts, hidden_dim * 2)))
        self.mlp2_weight = nn.Parameter(torch.empty((num_experts, dim, hidden_dim)))
        self.mlp2_bias = nn.Parameter(torch.empty((num_experts, dim)))

    def forward(self, x: torch.Tensor, num_tokens_per_expert: torch.Tensor) -> torch.Tensor:
        w1, b1, w2, b2 = (_local(t) for t in (self.mlp1_weight, self.mlp1_bias, self.mlp2_weight, self.mlp2_bias))
        run = _run_experts_grouped_mm if self.use_grouped_mm else _run_experts_for_loop
        return run(w1, b1, w2, b2, self.swiglu_limit, x, num_tokens_per_expert)


class GptOssMoE(MoE):
    """MoE layer whose experts are GptOssGroupedExperts (moe.py:199-224)."""

    @dataclass(kw_only=True, slots=True)
    class Config(MoE.Config):
        swiglu_limit: float = 7.0

    def __init__(self, config: Config):
        super().__init__(config)
        ec = config.experts
        self.experts = GptOssGroupedExperts.Config(
            dim=ec.dim, hidden_dim=ec.hidden_dim, num_experts=ec.num_experts,
            swiglu_limit=config.swiglu_limit, use_grouped_mm=ec.use_grouped_mm, param_init=ec.param_init,
        ).build()

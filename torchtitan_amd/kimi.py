"""Kimi-Linear's MoE host on the MI355X layer.

Mirrors ``KimiMoE`` (torchtitan/experiments/attention_residual/kimi_linear/model.py:597-707):
the Kimi config knobs are mapped onto ``MoE.Config`` and the layer is held as
``self._moe``, so parameter names under a decoder layer stay
``layers.{i}.ffn._moe.*`` exactly as in the reference. ``init_kimi_moe_weights``
follows the MoE part of the model's init (model.py:938-952).
"""

from __future__ import annotations

import torch
from torch import nn

from .feed_forward import FeedForward
from .linear import Linear
from .moe import GroupedExperts, MoE, TokenChoiceTopKRouter

__all__ = ["KimiMoE", "kimi_moe_config", "init_kimi_moe_weights"]


def kimi_moe_config(config) -> MoE.Config:
    """Maps a Kimi-Linear config (attributes hidden_size, num_experts,
    num_expert_group, topk_group, num_experts_per_token,
    moe_router_activation_func, moe_renormalize, routed_scaling_factor,
    moe_intermediate_size, num_shared_experts) onto MoE.Config
    (model.py:640-704): group limiting only when num_expert_group > 1; the
    shared expert's width is moe_intermediate_size * num_shared_experts;
    score_before_experts=True; load_balance_coeff=1e-3."""
    if config.num_experts is None or config.num_experts <= 0:
        raise AssertionError("KimiMoE needs num_experts > 0")
    grouped = config.num_expert_group > 1
    router = TokenChoiceTopKRouter.Config(
        num_experts=config.num_experts,
        gate=Linear.Config(in_features=config.hidden_size, out_features=config.num_experts, bias=False),
        num_expert_groups=config.num_expert_group if grouped else None,
        num_limited_groups=config.topk_group if grouped else None,
        top_k=config.num_experts_per_token,
        score_func=config.moe_router_activation_func,
        route_norm=config.moe_renormalize,
        route_scale=config.routed_scaling_factor,
    )
    experts = GroupedExperts.Config(
        dim=config.hidden_size, hidden_dim=config.moe_intermediate_size, num_experts=config.num_experts,
        use_grouped_mm=True,
    )
    shared = None
    if config.num_shared_experts > 0:
        hs = config.moe_intermediate_size * config.num_shared_experts
        shared = FeedForward.Config(
            w1=Linear.Config(in_features=config.hidden_size, out_features=hs, bias=False),
            w2=Linear.Config(in_features=hs, out_features=config.hidden_size, bias=False),
            w3=Linear.Config(in_features=config.hidden_size, out_features=hs, bias=False),
        )
    return MoE.Config(
        num_experts=config.num_experts, experts=experts, router=router, score_before_experts=True,
        load_balance_coeff=1e-3, shared_experts=shared,
    )


class KimiMoE(nn.Module):
    def __init__(self, config) -> None:
        super().__init__()
        self._moe = kimi_moe_config(config).build()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._moe(x)


def init_kimi_moe_weights(module: nn.Module, std: float) -> None:
    """normal(0, std) on every GroupedExperts w1/w2/w3 and zeros on the MoE
    load-balance buffers (model.py:941-952)."""
    with torch.no_grad():
        for m in module.modules():
            if isinstance(m, GroupedExperts):
                for name in ("w1", "w2", "w3"):
                    nn.init.normal_(getattr(m, name), mean=0.0, std=std)
            elif isinstance(m, MoE):
                for buf in ("expert_bias", "tokens_per_expert"):
                    b = getattr(m, buf, None)
                    if b is not None:
                        b.zero_()

"""``Linear``: nn.Linear with the Config protocol (torchtitan/models/common/linear.py:14-35).

Used for the router gate (fp32 logits: moe.gate_logits_f32 calls it under the
reference's fp32 autocast; an opt-in variant runs bf16 weights on bf16 GEMMs with
fp32 accumulation) and the shared expert's projections.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch.nn as nn

from .configurable import Module


class Linear(nn.Linear, Module):
    @dataclass(kw_only=True, slots=True)
    class Config(Module.Config):
        in_features: int
        out_features: int
        bias: bool = False

    def __init__(self, config: Config):
        super().__init__(config.in_features, config.out_features, bias=config.bias)

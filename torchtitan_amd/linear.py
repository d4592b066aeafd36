"""``Linear``: nn.Linear with the Config protocol (torchtitan/models/common/linear.py:14-35).

Used for the router gate (an fp32 GEMM under autocast, kept on torch so the
logits are the reference's bits) and the shared expert's projections.
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
